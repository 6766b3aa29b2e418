"""Writes the fixed-vector fixtures of tests/golden from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Each fixture is data (inputs are regenerated from seeds, expected outputs
are stored): BOA2 containers of the config-1 model (random-init seed 0,
synth.write_random_weights) over fixed slices of synth.gen_c1(), in cold,
warm-start and bf16 modes, plus a quantised-CDF / coder-stream vector.
manifest.json records how each was made and its SHA-256.  The fixtures
freeze today's oracle output: tests compare the oracle (CPU) and the HIP
library (GPU) with them, so an unintended change of either shows up.
"""
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "boa-constrictor_amd"), os.path.join(ROOT, "oracle")]

import refcpu  # noqa: E402
import synth  # noqa: E402

CONTAINERS = [
    # name, n bytes of gen_c1, chunk, extra compress options, bf16
    ("c1_cold_3x700", 2100, 700, {}, False),
    ("c1_cold_ragged", 5 * 256 + 37, 256, {"tile": 100}, False),
    ("c1_warm_7x300_b3", 7 * 300 + 13, 300, {"warm_start": True, "gpu_batch": 3}, False),
    ("c1_temp07_4x400", 1600, 400, {"temperature": 0.7}, False),
    ("c1_bf16_3x700", 2100, 700, {}, True),
]


def cdf_vector():
    rng = np.random.default_rng(11)
    logits = (rng.standard_normal((4, 256)) * np.array([[0.5], [3.0], [12.0], [40.0]])).astype(np.float32)
    q = np.stack([refcpu.cdf_quantize(refcpu.cdf_build(l)) for l in logits])
    syms = rng.integers(0, 256, size=64, dtype=np.uint8)
    cdfs = q[np.arange(64) % 4]
    words = refcpu.encode_cdf_stream(cdfs, syms)
    return dict(logits=logits.tolist(), qcdf=q.tolist(), symbols=syms.tolist(),
                cdf_row_of_symbol="i % 4", words=[int(w) for w in words])


def main():
    tmp = tempfile.mkdtemp()
    w = os.path.join(tmp, "c1.bin")
    synth.write_random_weights(w, 64, 2, 16, seed=0)
    data = synth.gen_c1()
    manifest = {"weights": "synth.write_random_weights(d_model=64, n_layers=2, d_state=16, seed=0)",
                "input": "synth.gen_c1()[:n]", "containers": {}}
    for name, n, chunk, opts, bf16 in CONTAINERS:
        m = refcpu.Model(w, 64, 2, bf16=bf16)
        blob = m.compress(data[:n], chunk_size=chunk, **opts)
        assert m.decompress(blob, temperature=opts.get("temperature", 1.0)) == data[:n]
        with open(os.path.join(HERE, name + ".boa"), "wb") as f:
            f.write(blob)
        manifest["containers"][name] = dict(n=n, chunk=chunk, options=opts, bf16=bf16,
                                            bytes=len(blob),
                                            sha256=hashlib.sha256(blob).hexdigest())
    with open(os.path.join(HERE, "cdf_coder_vector.json"), "w") as f:
        json.dump(cdf_vector(), f)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print("wrote", len(CONTAINERS), "containers and the CDF/coder vector to", HERE)


if __name__ == "__main__":
    main()
