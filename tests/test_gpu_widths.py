"""GPU parity at d_model widths between the ones the kernels are built for.

The reference accepts any d_model (dt_rank = ceil(d / 16), boa.cpp:912-918,
gemm_gpu.hpp:38-66).  This build runs a model of width dn at the next built
width (64, 80, 128, 256, 512; bf16: 64, 128, 256, 512) with the extra
features zero and the LayerNorms dividing by dn.  Each case compares the
HIP library, through the C ABI, with the CPU oracle run at the model's own
width: fp32 logits bit for bit in chunk and step mode, BOA2 bytes and round
trips; bf16 within the bf16 tolerance, compress == decompress bits and the
round trip.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


def _codec(d, L, ds, lanes, w, prec="fp32"):
    import boa_hip
    import torch
    c = boa_hip.Codec(d, L, ds, lanes, 0, precision=prec)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w)
    return c


# widths below 64 (the persistent decode at width 64), between 64 and 80,
# between the power-of-two widths, and d_state 32 at width 384 (-> 512)
@pytest.mark.parametrize("d,L,ds", [(37, 2, 16), (72, 1, 16), (100, 2, 16), (200, 1, 16),
                                    (384, 1, 32)])
def test_odd_width_fp32_bit_exact(torch_dev, oracle, make_weights, d, L, ds):
    torch = torch_dev
    w = make_weights(d, L, ds)
    lanes, T = 5, 24
    rng = np.random.default_rng(d + 3 * L + ds)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    m = oracle.Model(w, d, L, ds)
    want = m.new_state(lanes).forward_chunk(tok)
    c = _codec(d, L, ds, lanes, w)
    c.reset_state(lanes)
    d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
    c.forward_chunk(torch.from_numpy(tok).cuda(), lanes, T, d_log)
    torch.cuda.synchronize()
    got = d_log.cpu().numpy().reshape(lanes, T, 256)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"d={d}: max |diff| {np.abs(got - want).max()}"
    c.reset_state(lanes)
    d_s = torch.zeros(lanes * 256, dtype=torch.float32, device="cuda")
    for t in range(T):
        c.step_batch(torch.from_numpy(np.ascontiguousarray(tok[:, t])).cuda(), lanes, d_s, True)
        st = d_s.cpu().numpy().reshape(lanes, 256)
        assert np.array_equal(st.view(np.uint32), want[:, t].view(np.uint32)), f"step {t}"
    # the codec: the oracle's container, and back
    data = rng.integers(0, 256, size=7 * 300 - 11, dtype=np.uint8).tobytes()
    c2 = _codec(d, L, ds, 7, w)
    blob = c2.compress(data, chunk_size=300)
    assert blob == m.compress(data, chunk_size=300)
    assert c2.decompress(blob) == data
    c.close()
    c2.close()


@pytest.mark.parametrize("d,ds", [(96, 16), (200, 32)])
def test_odd_width_bf16(torch_dev, oracle, make_weights, d, ds):
    torch = torch_dev
    w = make_weights(d, 1, ds)
    lanes, T = 4, 40
    rng = np.random.default_rng(d + ds)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    want = oracle.Model(w, d, 1, ds).new_state(lanes).forward_chunk(tok)
    c = _codec(d, 1, ds, lanes, w, "bf16")
    c.reset_state(lanes)
    d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
    c.forward_chunk(torch.from_numpy(tok).cuda(), lanes, T, d_log)
    torch.cuda.synchronize()
    got = d_log.cpu().numpy().reshape(lanes, T, 256)
    # the bf16 tolerance of the other bf16 tests: 2e-2 of the logit scale
    assert np.abs(got - want).max() <= 2e-2 * np.abs(want).max()
    c.reset_state(lanes)
    d_s = torch.zeros(lanes * 256, dtype=torch.float32, device="cuda")
    for t in range(T):
        c.step_batch(torch.from_numpy(np.ascontiguousarray(tok[:, t])).cuda(), lanes, d_s, True)
        assert np.array_equal(d_s.cpu().numpy().reshape(lanes, 256).view(np.uint32),
                              got[:, t].view(np.uint32)), f"step {t}"
    data = rng.integers(0, 256, size=5 * 200 - 7, dtype=np.uint8).tobytes()
    c2 = _codec(d, 1, ds, 5, w, "bf16")
    assert c2.decompress(c2.compress(data, chunk_size=200)) == data
    c.close()
    c2.close()

