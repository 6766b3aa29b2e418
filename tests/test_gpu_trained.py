"""GPU parity on a trained model: the reference's own mambav1 checkpoint
(experiments/cms_experiment/..._mambav1_64_2_20ep.pt, BASELINE config-1
shape), converted to an fp16 weight file by tests/golden/
make_trained_fixture.py.  A trained model gives the peaked distributions
that random-init weights do not (long inverted coder runs, near-one-hot
CDFs, real compression).  The GPU containers must equal the fixture's
oracle containers byte for byte (and the live oracle's), and round-trip.
Also: the CLI with --gpu-batch 0 (memory-based batch sizing)."""
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

import boa_hip

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden")
MANIFEST = json.load(open(os.path.join(GOLD, "trained_manifest.json")))
WEIGHTS = os.path.join(GOLD, MANIFEST["weights"]["file"])


def _inputs():
    import synth
    rng = np.random.default_rng(21)
    rec = rng.choice(np.array([0.0, 1.0, 2.5, -1.0], np.float32), size=(4096, 4)).astype("<f4")
    return {"trained_c1_16x2048": synth.gen_c1()[:16 * 2048],
            "trained_zeros_4x4096": bytes(4 * 4096),
            "trained_records_4x4096": rec.tobytes()[:4 * 4096]}


def test_fixture_integrity():
    raw = open(WEIGHTS, "rb").read()
    assert raw[:4] == b"BOA\x01" and len(raw) == MANIFEST["weights"]["bytes"]
    assert hashlib.sha256(raw).hexdigest() == MANIFEST["weights"]["sha256"]


@pytest.mark.parametrize("name", sorted(MANIFEST["containers"]))
def test_trained_model_containers(oracle, name):
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    spec = MANIFEST["containers"][name]
    data = _inputs()[name]
    assert len(data) == spec["n"]
    gold = open(os.path.join(GOLD, name + ".boa"), "rb").read()
    c = boa_hip.Codec(64, 2, 16, 16)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(WEIGHTS)
    blob = c.compress(data, chunk_size=spec["chunk"])
    assert blob == gold, f"{name}: GPU container differs from the fixture"
    assert blob == oracle.Model(WEIGHTS, 64, 2).compress(data, chunk_size=spec["chunk"])
    assert c.decompress(blob) == data
    if name == "trained_zeros_4x4096":
        assert len(data) / len(blob) > 1.5, "the trained model compresses a zero run"
    c.close()


def test_trained_d_model_80(oracle):
    """The reference's d_model-80 checkpoint (..._mambav1_80_1_20.pt, one
    layer, dt_rank 5): a d_model that is not a power of two."""
    import synth
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    spec = MANIFEST["d_model_80"]
    w80 = os.path.join(GOLD, spec["weights"]["file"])
    raw = open(w80, "rb").read()
    assert hashlib.sha256(raw).hexdigest() == spec["weights"]["sha256"]
    cs = spec["container"]
    data = synth.gen_c1()[:cs["n"]]
    gold = open(os.path.join(GOLD, cs["file"]), "rb").read()
    c = boa_hip.Codec(80, 1, 16, 8)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w80)
    blob = c.compress(data, chunk_size=cs["chunk"])
    assert blob == gold
    assert blob == oracle.Model(w80, 80, 1).compress(data, chunk_size=cs["chunk"])
    assert c.decompress(blob) == data
    c.close()


def test_cli_auto_batch(oracle, w_c1, tmp_path):
    """--gpu-batch 0 sizes the batch from free memory (auto_size_params,
    boa.cpp:109-156) and still writes the oracle's container."""
    import synth
    exe = os.path.join(os.path.dirname(__file__), "..", "boa-constrictor_amd", "boa")
    data = synth.gen_c1()[:9 * 1000 + 5]
    src, out, back = tmp_path / "in.bin", tmp_path / "o.boa", tmp_path / "back.bin"
    src.write_bytes(data)
    r = subprocess.run([exe, "compress", str(w_c1), str(src), str(out), "64", "2", "--gpu-batch",
                        "0", "--chunk-size", "1000", "--show-timings"], check=True, timeout=120,
                       capture_output=True, text=True)
    assert "Auto-sizing: Selected Batch=" in r.stdout and "Timing (s): H2D=" in r.stdout
    assert out.read_bytes() == oracle.Model(w_c1, 64, 2).compress(data, chunk_size=1000)
    r = subprocess.run([exe, "decompress", str(w_c1), str(out), str(back), "64", "2",
                        "--gpu-batch", "0", "--kernel-timings"], check=True, timeout=120,
                       capture_output=True, text=True)
    assert "Auto-sizing: Selected Batch=" in r.stdout
    assert "(profiled run" in r.stdout and "Kernel time (s): Forward=" in r.stdout
    assert back.read_bytes() == data
