"""GPU parity of the bf16 precision (BASELINE configs 3 and 5: bf16 weights
and activations, fp32 scan state).

bf16 MFMA sums its 32 products with an internal precision and order that a
CPU fma chain does not reproduce bit for bit, so the GPU is compared with
the oracle's bf16 restatement within the bf16 tolerance (2e-2 of the logit
scale), while everything the decoder depends on is exact: compress-mode and
step-mode logits on the GPU are bit-identical, and compress -> decompress
round-trips byte for byte.  The compression ratio must agree with the
oracle's bf16 ratio within 0.5 %.
"""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

TOL = 2e-2


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


def _codec(d, L, ds=16, lanes=64, tile=0, w=None):
    import boa_hip
    import torch
    c = boa_hip.Codec(d, L, ds, lanes, tile, precision="bf16")
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    if w is not None:
        c.load_weights(w)
    return c


@pytest.mark.parametrize("d,L,ds", [(64, 2, 16), (256, 2, 16), (512, 1, 32)])
def test_bf16_logits_within_tolerance_and_step_equals_chunk(torch_dev, oracle, make_weights, d, L, ds):
    torch = torch_dev
    w = make_weights(d, L, ds)
    lanes, T = 5, 24
    rng = np.random.default_rng(100 + d + ds)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    want = oracle.Model(w, d, L, ds, bf16=True).new_state(lanes).forward_chunk(tok)
    c = _codec(d, L, ds, lanes=lanes, w=w)
    c.reset_state(lanes)
    d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
    c.forward_chunk(torch.from_numpy(tok).cuda(), lanes, T, d_log)
    torch.cuda.synchronize()
    got = d_log.cpu().numpy().reshape(lanes, T, 256)
    scale = np.abs(want).max()
    err = np.abs(got - want).max()
    assert err <= TOL * scale, f"max |gpu - oracle| {err:.3g} > {TOL} x {scale:.3g}"
    c.reset_state(lanes)
    d_s = torch.zeros(lanes * 256, dtype=torch.float32, device="cuda")
    for t in range(T):
        c.step_batch(torch.from_numpy(np.ascontiguousarray(tok[:, t])).cuda(), lanes, d_s, True)
        st = d_s.cpu().numpy().reshape(lanes, 256)
        assert np.array_equal(st.view(np.uint32), got[:, t].view(np.uint32)), f"step {t}"


@pytest.mark.parametrize("d,L,ds,gen,n,chunk", [
    (64, 2, 16, "c1", 8 * 1000 + 11, 1000),
    (256, 2, 16, "c3", 6 * 800, 800),
    (512, 1, 32, "c5", 4 * 600 + 3, 600),
])
def test_bf16_round_trip_and_ratio(torch_dev, oracle, make_weights, d, L, ds, gen, n, chunk):
    w = make_weights(d, L, ds)
    data = {"c1": lambda: synth.gen_c1(), "c3": lambda: synth.gen_c3(4),
            "c5": lambda: synth.gen_c5(4096)}[gen]()[:n]
    c = _codec(d, L, ds, lanes=4, w=w)
    blob = c.compress(data, chunk_size=chunk)
    assert c.decompress(blob) == data
    ref = oracle.Model(w, d, L, ds, bf16=True).compress(data, chunk_size=chunk)
    assert abs(len(blob) / len(ref) - 1.0) < 5e-3, f"{len(blob)} vs oracle {len(ref)} bytes"


@pytest.mark.parametrize("d,L,ds", [(64, 2, 16), (256, 1, 16), (512, 1, 32)])
def test_bf16_many_lanes_step_equals_chunk_and_round_trip(torch_dev, make_weights, d, L, ds):
    """From 2048 lanes on the bf16 decode GEMMs run the many-lane forms (2 x 2
    tiles per wave, 64 x 64 LDS blocks, and 128 x 128 LDS blocks for in_proj
    and FF1 from d_model 128, a partial last block at 2100 lanes): step
    logits stay bit-identical to chunk logits, with the state streamed
    (cache budget 0) and through the caches (every layer), and a container
    of 2101 chunks (one decode batch) round-trips byte for byte."""
    torch = torch_dev
    w = make_weights(d, L, ds)
    lanes, T = 2100, 5
    rng = np.random.default_rng(7 + d)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    c = _codec(d, L, ds, lanes=2200, w=w)
    c.reset_state(lanes)
    d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
    c.forward_chunk(torch.from_numpy(tok).cuda(), lanes, T, d_log)
    torch.cuda.synchronize()
    got = d_log.cpu().numpy().reshape(lanes, T, 256)
    d_s = torch.zeros(lanes * 256, dtype=torch.float32, device="cuda")
    for budget, want_cached in [(0, 0), (1 << 40, L)]:
        c.set_state_cache_budget(budget)
        assert c.decode_plan(lanes)["cached_layers"] == want_cached
        c.reset_state(lanes)
        for t in range(T):
            c.step_batch(torch.from_numpy(np.ascontiguousarray(tok[:, t])).cuda(), lanes, d_s, True)
            st = d_s.cpu().numpy().reshape(lanes, 256)
            assert np.array_equal(st.view(np.uint32), got[:, t].view(np.uint32)), \
                f"budget {budget} step {t}"
    c.set_state_cache_budget(-1)
    data = synth.gen_c3(21)[:2100 * 40 + 7]
    blob = c.compress(data, chunk_size=40)
    assert c.decompress(blob) == data
