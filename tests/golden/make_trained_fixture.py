"""Writes the trained-model fixture of tests/golden from the reference's own
checkpoint and the CPU oracle.

Run from the repository root (needs the reference mounted at
/root/reference):  python tests/golden/make_trained_fixture.py

The checkpoint experiments/cms_experiment/
cms_experiment_final_model_fp32_mambav1_64_2_20ep.pt (a mambav1 model of
the BASELINE config-1 shape, d_model 64, 2 layers, trained on CMS jet
features) is loaded with torch.load(weights_only=True) and written as an
fp16 "BOA\\x01" weight file by this repository's converter.  The fixture is
that weight file plus the oracle's BOA2 containers of three inputs, so that
GPU tests can run a trained model -- peaked distributions, long inverted
coder runs, real compression -- where the reference is not mounted.
trained_manifest.json records the inputs and SHA-256s.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "boa-constrictor_amd"), os.path.join(ROOT, "oracle")]

import convert_weights  # noqa: E402
import refcpu  # noqa: E402
import synth  # noqa: E402

CKPT = ("/root/reference/experiments/cms_experiment/"
        "cms_experiment_final_model_fp32_mambav1_64_2_20ep.pt")
WEIGHTS = "trained_mambav1_64_2_fp16.bin"


def inputs():
    """name -> (bytes, chunk): the config-1 input, zeros, and float32
    records with few distinct values (a low-entropy structured stream)."""
    rng = np.random.default_rng(21)
    rec = rng.choice(np.array([0.0, 1.0, 2.5, -1.0], np.float32), size=(4096, 4)).astype("<f4")
    return {
        "trained_c1_16x2048": (synth.gen_c1()[:16 * 2048], 2048),
        "trained_zeros_4x4096": (bytes(4 * 4096), 4096),
        "trained_records_4x4096": (rec.tobytes()[:4 * 4096], 4096),
    }


def main():
    wpath = os.path.join(HERE, WEIGHTS)
    info = convert_weights.convert(CKPT, wpath, fp16=True)
    assert (info["d_model"], info["n_layers"]) == (64, 2), info
    with open(wpath, "rb") as f:
        wbytes = f.read()
    m = refcpu.Model(wpath, 64, 2)
    manifest = {"checkpoint": os.path.basename(CKPT), "loader": "torch.load(weights_only=True)",
                "weights": dict(file=WEIGHTS, bytes=len(wbytes),
                                sha256=hashlib.sha256(wbytes).hexdigest()),
                "containers": {}}
    for name, (data, chunk) in inputs().items():
        blob = m.compress(data, chunk_size=chunk)
        assert m.decompress(blob) == data
        with open(os.path.join(HERE, name + ".boa"), "wb") as f:
            f.write(blob)
        manifest["containers"][name] = dict(n=len(data), chunk=chunk, bytes=len(blob),
                                            ratio=round(len(data) / len(blob), 4),
                                            sha256=hashlib.sha256(blob).hexdigest())
    with open(os.path.join(HERE, "trained_manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
