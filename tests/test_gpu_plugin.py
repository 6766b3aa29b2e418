"""GPU side of the Python codec's CDF plug-in (boa_cdf_from_probs,
gpu_range_coder.py:57-79): bit-exact with the oracle's ref_cdf_from_probs
for softmax rows of several widths and for the degenerate rows that fall
back to the uniform CDF; the CDFs then code through boa_rc_encode_cdf into
the oracle coder's words (which tests/test_oracle_python_coder.py shows are
the Python codec coder's words)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def codec():
    import boa_hip
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = boa_hip.Codec(64, 2, 16, 8)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    return c


def _rows(K, n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        lg = rng.standard_normal(K) * (0.5, 4.0, 20.0)[i % 3]
        p = np.exp(lg - lg.max())
        out.append((p / p.sum()).astype(np.float32))
    rows = np.stack(out)
    rows[1] = 0.0                    # zero row -> uniform
    rows[2, 0] = np.nan              # NaN -> uniform
    rows[4] = 0.0
    rows[4, K // 2] = 3.0            # one-hot, unnormalised
    return rows


@pytest.mark.parametrize("K", [17, 256, 1024])
def test_cdf_from_probs_bit_exact(codec, oracle, K):
    import torch
    rows = _rows(K, 40, K)
    q = torch.zeros((len(rows), K + 1), dtype=torch.int32, device="cuda")
    codec.cdf_from_probs(torch.from_numpy(rows).cuda(), len(rows), K, q)
    torch.cuda.synchronize()
    got = q.cpu().numpy().view(np.uint32)
    want = np.stack([oracle.cdf_from_probs(r) for r in rows])
    assert np.array_equal(got, want)


def test_plugin_cdfs_code_like_the_oracle(codec, oracle):
    import torch
    rows = _rows(256, 64, 3)
    q = torch.zeros((64, 257), dtype=torch.int32, device="cuda")
    codec.cdf_from_probs(torch.from_numpy(rows).cuda(), 64, 256, q)
    rng = np.random.default_rng(4)
    n = 300
    idx = np.arange(n) % 64
    qc = q.cpu().numpy().view(np.uint32)[idx]
    syms = np.array([np.searchsorted(qc[i], rng.integers(0, 1 << 24), side="right") - 1
                     for i in range(n)], np.uint8)
    cdf = torch.from_numpy(qc.view(np.int32).copy()).cuda().reshape(1, n, 257)
    pitch = 2 * n + 8
    words = torch.zeros(pitch, dtype=torch.int32, device="cuda")
    sizes = torch.zeros(1, dtype=torch.int32, device="cuda")
    codec.rc_encode_cdf(cdf, torch.from_numpy(syms).cuda(), n, 1, words, pitch, sizes)
    torch.cuda.synchronize()
    nw = int(sizes.item())
    assert words[:nw].cpu().numpy().view(np.uint32).tolist() == \
        oracle.encode_cdf_stream(qc, syms).tolist()
