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
# the reference's d_model-80 checkpoint (one layer; dt_rank 5): a shape
# whose d_model is not a power of two
CKPT80 = ("/root/reference/experiments/cms_experiment/"
          "cms_experiment_final_model_fp32_mambav1_80_1_20.pt")
WEIGHTS80 = "trained_mambav1_80_1_fp16.bin"


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
    # d_model 80: its weights and one container of the config-1 input
    w80 = os.path.join(HERE, WEIGHTS80)
    info80 = convert_weights.convert(CKPT80, w80, fp16=True)
    assert (info80["d_model"], info80["n_layers"]) == (80, 1), info80
    with open(w80, "rb") as f:
        wb80 = f.read()
    m80 = refcpu.Model(w80, 80, 1)
    data80, chunk80 = synth.gen_c1()[:8 * 1024], 1024
    blob80 = m80.compress(data80, chunk_size=chunk80)
    assert m80.decompress(blob80) == data80
    with open(os.path.join(HERE, "trained80_c1_8x1024.boa"), "wb") as f:
        f.write(blob80)
    manifest["d_model_80"] = {
        "checkpoint": os.path.basename(CKPT80),
        "weights": dict(file=WEIGHTS80, bytes=len(wb80), sha256=hashlib.sha256(wb80).hexdigest()),
        "container": dict(file="trained80_c1_8x1024.boa", n=len(data80), chunk=chunk80,
                          bytes=len(blob80), sha256=hashlib.sha256(blob80).hexdigest())}
    with open(os.path.join(HERE, "trained_manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
