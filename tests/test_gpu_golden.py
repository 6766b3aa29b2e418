"""The HIP library reproduces the frozen fixtures of tests/golden.

fp32 containers (cold, ragged with tiles, warm-start, temperature) must be
written byte for byte by the GPU and decoded by it; the CDF / coder vector
must come out of boa_cdf_from_logits and boa_rc_encode_cdf unchanged.  The
bf16 fixture is checked on the CPU only (bf16 MFMA sums differ from the
oracle's within tolerance, not bit for bit).
"""
import json
import os

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))
FP32 = sorted(k for k, v in MANIFEST["containers"].items() if not v["bf16"])


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


@pytest.mark.parametrize("name", FP32)
def test_gpu_writes_and_reads_fixture(torch_dev, w_c1, name):
    import boa_hip
    torch = torch_dev
    spec = MANIFEST["containers"][name]
    opts = spec["options"]
    with open(os.path.join(GOLDEN, name + ".boa"), "rb") as f:
        blob = f.read()
    data = synth.gen_c1()[:spec["n"]]
    c = boa_hip.Codec(64, 2, 16, 8, opts.get("tile", 0), opts.get("temperature", 1.0))
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w_c1)
    if opts.get("warm_start"):
        c.set_warm_start(opts["gpu_batch"])
    assert c.compress(data, chunk_size=spec["chunk"]) == blob
    assert c.decompress(blob) == data


def test_gpu_cdf_and_coder_vector(torch_dev, w_c1):
    import boa_hip
    torch = torch_dev
    v = json.load(open(os.path.join(GOLDEN, "cdf_coder_vector.json")))
    c = boa_hip.Codec(64, 2, 16, 8)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w_c1)
    logits = torch.tensor(np.array(v["logits"], np.float32)).cuda()
    q = torch.zeros((4, 257), dtype=torch.int32, device="cuda")
    c.cdf_from_logits(logits, None, 4, q)
    torch.cuda.synchronize()
    want_q = np.array(v["qcdf"], np.uint32)
    assert np.array_equal(q.cpu().numpy().view(np.uint32), want_q)
    syms = np.array(v["symbols"], np.uint8)
    n = len(syms)
    cdf = torch.tensor(want_q[np.arange(n) % 4].view(np.int32)).cuda().reshape(1, n, 257)
    pitch = 4 * n + 64
    words = torch.zeros(pitch, dtype=torch.int32, device="cuda")
    sizes = torch.zeros(1, dtype=torch.int32, device="cuda")
    c.rc_encode_cdf(cdf, torch.tensor(syms).cuda(), n, 1, words, pitch, sizes)
    torch.cuda.synchronize()
    nw = int(sizes.item())
    assert words[:nw].cpu().numpy().view(np.uint32).tolist() == v["words"]
