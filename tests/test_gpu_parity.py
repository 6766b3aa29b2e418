"""GPU parity: the HIP path against the CPU oracle on the same seeded inputs.

Every comparison is exact (integer words, CDF integers, fp32 logit bits,
container bytes): the kernels evaluate the oracle's operation sequence, and
v_mfma_f32_16x16x4_f32 rounds as the K-ordered fma chain the oracle runs.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


def _codec(d, L, ds=16, lanes=64, tile=0, w=None):
    import boa_hip
    import torch
    c = boa_hip.Codec(d, L, ds, lanes, tile)
    # order the library's launches with torch's copies
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    if w is not None:
        c.load_weights(w)
    return c


def random_cdfs(rng, n, skew):
    """n strictly increasing 257-entry integer CDFs over 2^24 with every
    frequency >= 1; `skew` concentrates mass (forces long inverted runs)."""
    out = np.zeros((n, 257), np.uint32)
    for i in range(n):
        w = rng.random(256) ** skew
        w = np.maximum(w / w.sum() * ((1 << 24) - 256), 0).astype(np.int64) + 1
        w[rng.integers(256)] += (1 << 24) - int(w.sum())
        out[i, 1:] = np.cumsum(w)
    return out


@pytest.mark.parametrize("skew", [1.0, 8.0, 40.0])
def test_coder_bit_exact_given_cdfs(torch_dev, oracle, skew):
    torch = torch_dev
    rng = np.random.default_rng(7 + int(skew))
    lanes, n_sym = 19, 700
    cdf = random_cdfs(rng, lanes * n_sym, skew).reshape(lanes, n_sym, 257)
    syms = np.empty((lanes, n_sym), np.uint8)
    for b in range(lanes):
        for i in range(n_sym):
            # draw mostly likely symbols, sometimes the rarest one
            f = np.diff(cdf[b, i].astype(np.int64))
            syms[b, i] = np.argmin(f) if rng.random() < 0.05 else rng.choice(256, p=f / f.sum())
    want = [oracle.encode_cdf_stream(cdf[b], syms[b]) for b in range(lanes)]
    pitch = 2 * n_sym + 8
    c = _codec(64, 1)
    d_cdf = torch.from_numpy(cdf.reshape(-1)).cuda()
    d_syms = torch.from_numpy(syms.reshape(-1)).cuda()
    d_words = torch.zeros(lanes * pitch, dtype=torch.int32, device="cuda")
    d_sizes = torch.zeros(lanes, dtype=torch.int32, device="cuda")
    c.rc_encode_cdf(d_cdf, d_syms, n_sym, lanes, d_words, pitch, d_sizes)
    torch.cuda.synchronize()
    words = d_words.cpu().numpy().view(np.uint32).reshape(lanes, pitch)
    sizes = d_sizes.cpu().numpy()
    for b in range(lanes):
        assert sizes[b] == len(want[b]), f"lane {b}"
        assert np.array_equal(words[b, :sizes[b]], want[b]), f"lane {b} words differ"
    d_out = torch.zeros(lanes * n_sym, dtype=torch.uint8, device="cuda")
    c.rc_decode_cdf(d_cdf, n_sym, lanes, d_words, pitch, d_sizes, d_out)
    torch.cuda.synchronize()
    assert np.array_equal(d_out.cpu().numpy().reshape(lanes, n_sym), syms)


def test_cdf_from_logits_bit_exact(torch_dev, oracle):
    torch = torch_dev
    rng = np.random.default_rng(11)
    rows = 333
    # large scales underflow most exps and exercise the boundary fix-up
    scale = np.repeat([0.01, 1.0, 5.0, 30.0, 200.0, 300.0], rows // 6 + 1)[:rows, None]
    logits = (rng.standard_normal((rows, 256)) * scale).astype(np.float32)
    logits[0] = 0.0                     # uniform row
    logits[1, 17] = 1e4                 # one-hot row
    bias = rng.standard_normal(256).astype(np.float32)
    c = _codec(64, 1)
    for b in (None, bias):
        d_l = torch.from_numpy(logits).cuda()
        d_b = torch.from_numpy(b).cuda() if b is not None else None
        d_q = torch.zeros(rows * 257, dtype=torch.int32, device="cuda")
        c.cdf_from_logits(d_l, d_b, rows, d_q)
        torch.cuda.synchronize()
        got = d_q.cpu().numpy().view(np.uint32).reshape(rows, 257)
        for r in range(rows):
            want = oracle.cdf_quantize(oracle.cdf_build(logits[r], b))
            assert np.array_equal(got[r], want), f"row {r}"


def _forward_pair(torch, oracle, w, d, L, lanes, T, seed):
    rng = np.random.default_rng(seed)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    m = oracle.Model(w, d, L)
    want = m.new_state(lanes).forward_chunk(tok)
    c = _codec(d, L, lanes=lanes, w=w)
    c.reset_state(lanes)
    d_tok = torch.from_numpy(tok).cuda()
    d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
    c.forward_chunk(d_tok, lanes, T, d_log)
    torch.cuda.synchronize()
    got = d_log.cpu().numpy().reshape(lanes, T, 256)
    return tok, want, got, c


def test_forward_chunk_matches_oracle(torch_dev, oracle, w_c1):
    tok, want, got, _ = _forward_pair(torch_dev, oracle, w_c1, 64, 2, 5, 48, 3)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"max |diff| {np.abs(got - want).max()}"


def test_step_equals_chunk_on_gpu(torch_dev, w_c1):
    torch = torch_dev
    lanes, T = 6, 40
    rng = np.random.default_rng(5)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    c = _codec(64, 2, lanes=lanes, w=w_c1)
    c.reset_state(lanes)
    d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
    c.forward_chunk(torch.from_numpy(tok).cuda(), lanes, T, d_log)
    chunk = d_log.cpu().numpy().reshape(lanes, T, 256)
    c.reset_state(lanes)
    steps = []
    d_s = torch.zeros(lanes * 256, dtype=torch.float32, device="cuda")
    for t in range(T):
        c.step_batch(torch.from_numpy(np.ascontiguousarray(tok[:, t])).cuda(), lanes, d_s, True)
        steps.append(d_s.cpu().numpy().reshape(lanes, 256).copy())
    step = np.stack(steps, 1)
    assert np.array_equal(chunk.view(np.uint32), step.view(np.uint32))


def test_compress_container_matches_oracle(torch_dev, oracle, w_c1):
    import synth
    data = synth.gen_c1()[: 16 * 4096 + 1234]
    m = oracle.Model(w_c1, 64, 2)
    want = m.compress(data, chunk_size=4096)
    c = _codec(64, 2, lanes=8, tile=1000, w=w_c1)   # 3 batches, ragged tiles
    got = c.compress(data, chunk_size=4096)
    assert got == want
    assert c.decompress(got) == data
