"""The Python GPU codec's coder path as an alternate CDF plug-in.

gpu_range_coder.py builds integer CDFs from probabilities (build_cdf_fast,
:57-79) and codes them with a 64-bit range coder (:84-182).  These tests
pin the oracle's ref_cdf_from_probs with closed forms and invariants, and
show that a restatement of that file's encoder and decoder produces and
reads exactly the streams of this build's coder (the C++ driver's,
range_coder_kernels.cu), so probabilities from elsewhere can be coded into
the Python codec's streams.
"""
import numpy as np
import pytest

TOTAL = 1 << 24
M64 = (1 << 64) - 1


def test_uniform_probs_closed_form(oracle):
    q = oracle.cdf_from_probs(np.full(256, 1 / 256, np.float32))
    assert np.array_equal(q, np.arange(257, dtype=np.uint32) * 65536)


@pytest.mark.parametrize("K,j", [(256, 0), (256, 77), (256, 255), (10, 3), (1, 0)])
def test_one_hot_closed_form(oracle, K, j):
    p = np.zeros(K, np.float32)
    p[j] = 1.0
    q = oracle.cdf_from_probs(p).astype(np.int64)
    want = np.arange(K + 1, dtype=np.int64)
    want[j + 1:] += TOTAL - K
    want[K] = TOTAL
    assert np.array_equal(q, want)


@pytest.mark.parametrize("row", [np.zeros(256), np.full(256, np.nan), np.r_[np.inf, np.ones(255)],
                                 -np.ones(256)])
def test_degenerate_rows_fall_back_to_uniform(oracle, row):
    q = oracle.cdf_from_probs(row.astype(np.float32))
    step = (TOTAL - 256) // 256 + 1
    want = np.arange(257, dtype=np.int64) * step
    want[256] = TOTAL
    assert np.array_equal(q.astype(np.int64), want)


def test_invariants_and_proportionality(oracle):
    rng = np.random.default_rng(5)
    for K in (2, 17, 256, 1024):
        for scale in (0.5, 3.0, 12.0):
            lg = rng.standard_normal(K) * scale
            p = np.exp(lg - lg.max()).astype(np.float32)
            p /= p.sum()
            q = oracle.cdf_from_probs(p).astype(np.int64)
            f = np.diff(q)
            assert q[0] == 0 and q[K] == TOTAL and f.min() >= 1
            ideal = 1 + p.astype(np.float64) / p.astype(np.float64).sum() * (TOTAL - K)
            assert np.abs(f - ideal).max() < 2.0
            # scaling the row by a power of two scales norm and running sums exactly
            assert np.array_equal(oracle.cdf_from_probs(p * 4).astype(np.int64), q)


# ---- restatement of gpu_range_coder.py:84-182 (encoder, finalize, decoder)
def py_encode(cdfs, syms, stats=None):
    lower, rng_, inv, first_inv, out = 0, M64, 0, 0, []
    runs = []
    for cdf, s in zip(cdfs, syms):
        s = int(s)
        left, prob = int(cdf[s]), int(cdf[s + 1]) - int(cdf[s])
        scale = rng_ >> 24
        rng_ = scale * prob
        old = lower
        lower = (lower + scale * left) & M64
        if inv > 0 and ((lower + rng_) & M64) > lower:
            first, rest = (first_inv + 1, 0) if lower < old else (first_inv, 0xFFFFFFFF)
            out.append(first & 0xFFFFFFFF)
            out.extend([rest] * (inv - 1))
            runs.append((inv, lower < old))
            inv = 0
        while rng_ < (1 << 32):
            word = lower >> 32
            lower = (lower << 32) & M64
            rng_ = (rng_ << 32) & M64
            if inv > 0:
                inv += 1
            elif ((lower + rng_) & M64) > lower:
                out.append(word)
            else:
                inv, first_inv = 1, word
    if stats is not None:
        stats["runs"] = runs
    if rng_ == M64:
        return []
    point = (lower + (1 << 32) - 1) & M64
    if inv > 0:
        first, rest = (first_inv + 1, 0) if point < lower else (first_inv, 0xFFFFFFFF)
        out.append(first & 0xFFFFFFFF)
        out.extend([rest] * (inv - 1))
    out.append(point >> 32)
    if ((lower + rng_) & M64) >> 32 == point >> 32:
        out.append(0)
    return out


def py_decode(cdfs, words):
    lower, rng_, point, rd = 0, M64, 0, 0
    for _ in range(2):
        point = ((point << 32) | (words[rd] if rd < len(words) else 0)) & M64
        rd += 1
    syms = []
    for cdf in cdfs:
        scale = rng_ >> 24
        q = min(((point - lower) & M64) // scale, TOTAL - 1)
        s = 1
        while s <= 256 and not (int(cdf[s]) > q):
            s += 1
        s = min(max(s - 1, 0), 255)
        syms.append(s)
        lower = (lower + scale * int(cdf[s])) & M64
        rng_ = scale * (int(cdf[s + 1]) - int(cdf[s]))
        while rng_ < (1 << 32):
            lower = (lower << 32) & M64
            rng_ = (rng_ << 32) & M64
            point = ((point << 32) | (words[rd] if rd < len(words) else 0)) & M64
            rd += 1
    return syms


@pytest.mark.parametrize("seed,skew", [(0, 0.5), (1, 6.0), (2, 30.0)])
def test_python_codec_coder_matches_this_coder(oracle, seed, skew):
    rng = np.random.default_rng(seed)
    n = 600
    cdfs = []
    for _ in range(8):
        lg = rng.standard_normal(256) * skew
        p = np.exp(lg - lg.max()).astype(np.float32)
        cdfs.append(oracle.cdf_from_probs(p / p.sum()))
    rows = np.stack([cdfs[i % 8] for i in range(n)])
    # symbols drawn mostly from the likely ones, some from the tails
    syms = np.array([np.searchsorted(rows[i], rng.integers(0, TOTAL), side="right") - 1
                     if i % 5 else rng.integers(0, 256) for i in range(n)], np.uint8)
    ours = oracle.encode_cdf_stream(rows, syms)
    assert ours.tolist() == py_encode(rows, syms)
    assert py_decode(rows, ours.tolist()) == syms.tolist()


def test_python_codec_coder_inverted_runs_and_carries(oracle):
    """Random symbols under a CDF with one dominant symbol at the top of the
    range drive lower + range across 2^64: the stream holds inverted runs
    resolved both with and without a carry, and both coders agree."""
    cdf = np.arange(257, dtype=np.uint32)
    cdf[256] = TOTAL
    rng = np.random.default_rng(11)
    found = None
    for trial in range(200):
        syms = np.where(rng.random(3000) < 0.9, 255, rng.integers(0, 255, 3000)).astype(np.uint8)
        rows = np.broadcast_to(cdf, (len(syms), 257))
        st = {}
        want = py_encode(rows, syms, st)
        if {c for _, c in st["runs"]} == {True, False}:
            found = (rows, syms, want)
            break
    assert found, "no stream with both kinds of inverted run"
    rows, syms, want = found
    ours = oracle.encode_cdf_stream(np.ascontiguousarray(rows), syms)
    assert ours.tolist() == want
    assert py_decode(rows, ours.tolist()) == syms.tolist()
