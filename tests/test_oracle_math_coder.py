"""CPU tests pinning the oracle's math, CDF quantiser and range coder.

The reference ships no test vectors for this path, so every check here is
against something the mathematics fixes: float64 library functions with ulp
bounds, closed forms (uniform logits, a one-symbol stream worked by hand),
invariants of the integer CDF, and an arbitrary-precision model of the
range coder that has no 64-bit window and therefore no carry / inverted-run
logic (the part of the coder most likely to hide a mistake).
"""
import struct
import zlib

import numpy as np
import pytest


def f32(x):
    return np.float32(x)


def ulp_err(got, want64):
    got = np.asarray(got, np.float64)
    want32 = np.asarray(want64, np.float64).astype(np.float32)
    spacing = np.abs(np.spacing(want32.astype(np.float32))).astype(np.float64)
    return np.abs(got - want64) / spacing


def vec(fn, xs):
    return np.array([fn(float(x)) for x in xs], np.float64)


# ------------------------------------------------------------------ math
def test_expf_ulp_bound(oracle):
    L = oracle.lib()
    xs = np.concatenate([np.linspace(-87.0, 88.7, 40001, dtype=np.float32),
                         np.linspace(-1, 1, 20001, dtype=np.float32)])
    got = vec(L.ref_expf, xs)
    err = ulp_err(got, np.exp(xs.astype(np.float64)))
    assert err.max() <= 2.0, f"max ulp error {err.max()}"
    assert L.ref_expf(0.0) == 1.0
    assert L.ref_expf(-87.5) == 0.0
    assert L.ref_expf(89.0) == float("inf")
    assert np.isnan(L.ref_expf(float("nan")))


def test_exp2_neg(oracle):
    """The scan's base-2 exp: within one ulp of float64 2^t on [-126, 0],
    exact at integers (2^0 = 1 and ldexp are exact), clamped below -126 and
    above 0, NaN mapped to 2^-126."""
    L = oracle.lib()
    ts = np.concatenate([np.linspace(-126.0, 0.0, 200001, dtype=np.float32),
                         -np.geomspace(1e-30, 126.0, 40001).astype(np.float32),
                         np.linspace(-0.5, 0.5, 20001, dtype=np.float32).clip(None, 0)])
    got = vec(L.ref_exp2_neg, ts)
    err = ulp_err(got, np.exp2(ts.astype(np.float64)))
    assert err.max() <= 1.0, f"max ulp error {err.max()}"
    for k in range(127):
        assert L.ref_exp2_neg(float(-k)) == 2.0 ** -k
    tiny = 2.0 ** -126
    for t in (-126.5, -200.0, float("-inf"), float("nan")):
        assert L.ref_exp2_neg(t) == tiny
    assert L.ref_exp2_neg(3.0) == 1.0 and L.ref_exp2_neg(-0.0) == 1.0


def test_scan_decay_against_float64(oracle):
    """exp(-exp(A_log) dt) taken as 2^(na2 dt): the three fp32 roundings
    before the exp (exp(A_log), the log2(e) product, the dt product) bound
    the error by a few ulp times |t|, against float64 exp(-exp(a) dt)."""
    L = oracle.lib()
    rng = np.random.default_rng(3)
    a = rng.uniform(-4, 4, 4000).astype(np.float32)
    dt = np.exp(rng.uniform(-8, 3, 4000)).astype(np.float32)
    got = np.array([L.ref_exp2_neg(np.float32(np.float32(L.ref_scan_na2(float(x))) * np.float32(d)))
                    for x, d in zip(a, dt)])
    x64 = -np.exp(a.astype(np.float64)) * dt.astype(np.float64)
    want = np.exp(x64)
    keep = x64 > -87.0
    t = np.abs(x64[keep]) / np.log(2.0)
    rel = np.abs(got[keep] - want[keep]) / want[keep]
    assert np.all(rel <= 2.0 ** -23 * (2.0 + 4.0 * t)), rel.max()
    # the decay coefficient itself: two fp32 roundings of -exp(a) log2(e)
    na2 = np.array([L.ref_scan_na2(float(x)) for x in a])
    want_na2 = -np.exp(a.astype(np.float64)) / np.log(2.0)
    assert np.all(np.abs(na2 - want_na2) <= 4 * 2.0 ** -24 * np.abs(want_na2))


def test_logf_ulp_bound(oracle):
    L = oracle.lib()
    xs = np.concatenate([np.geomspace(1e-30, 1e30, 40001).astype(np.float32),
                         np.linspace(0.5, 2.0, 20001, dtype=np.float32)])
    got = vec(L.ref_logf, xs)
    want = np.log(xs.astype(np.float64))
    err = np.abs(got - want) / np.maximum(np.abs(np.spacing(want.astype(np.float32))), 1e-45)
    assert err.max() <= 2.0, f"max ulp error {err.max()}"
    assert L.ref_logf(1.0) == 0.0
    assert L.ref_logf(float("inf")) == float("inf")


def test_activations_against_float64(oracle):
    L = oracle.lib()
    xs = np.linspace(-30, 30, 6001, dtype=np.float32)
    x64 = xs.astype(np.float64)
    # unthresholded float32 softplus: log(fl(1 + exp(x))), so 0 once exp(x) < 2^-24
    one_plus = (np.float32(1) + np.exp(x64).astype(np.float32)).astype(np.float64)
    np.testing.assert_allclose(vec(L.ref_softplus, xs), np.log(one_plus), rtol=3e-6, atol=1e-7)
    np.testing.assert_allclose(vec(L.ref_silu, xs), x64 / (1 + np.exp(-x64)), rtol=2e-6, atol=1e-12)
    gelu = 0.5 * x64 * (1 + np.tanh(np.sqrt(2 / np.pi) * (x64 + 0.044715 * x64 ** 3)))
    np.testing.assert_allclose(vec(L.ref_gelu, xs), gelu, rtol=2e-5, atol=2e-6)
    # the reference's own exp (activations.hpp:33-84) is a degree-6 Taylor
    # polynomial after a one-constant reduction: a few 1e-6 relative
    ys = np.linspace(-80, 80, 8001, dtype=np.float32)
    np.testing.assert_allclose(vec(L.ref_repro_exp, ys), np.exp(ys.astype(np.float64)), rtol=1e-5)


def test_half_widening_exhaustive(oracle):
    L = oracle.lib()
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([L.ref_half_to_float(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# -------------------------------------------------------------- CDF
def test_cdf_uniform_closed_form(oracle):
    q = oracle.cdf_quantize(oracle.cdf_build(np.zeros(256, np.float32)))
    # s_cdf[k] = k/256 exactly, so low_k = floor(k/256 (2^24-256)) + k = 65536 k
    assert np.array_equal(q[:256], np.arange(256, dtype=np.uint32) * 65536)
    assert q[256] == 1 << 24


def test_cdf_invariants_and_softmax(oracle):
    rng = np.random.default_rng(3)
    for scale in (0.1, 1.0, 4.0, 20.0, 100.0):
        for _ in range(20):
            lg = (rng.standard_normal(256) * scale).astype(np.float32)
            q = oracle.cdf_quantize(oracle.cdf_build(lg)).astype(np.int64)
            f = np.diff(q)
            assert q[0] == 0 and q[256] == 1 << 24
            assert (f >= 1).all()
            p = np.exp(lg.astype(np.float64) - lg.max())
            p /= p.sum()
            # freq_k = floor(c_{k+1} S) - floor(c_k S) + 1 with S = 2^24 - 256
            assert np.abs(f - (p * ((1 << 24) - 256) + 1)).max() <= 2.0


def test_cdf_fixup_sequential_vs_lockstep(oracle):
    """The reference's lock-step lane-boundary fix-up (mode 1) can leave a
    zero-frequency symbol when neighbouring lanes both shift (peaked
    distributions with underflowing exps); the oracle's lane-by-lane fix-up
    (mode 0) never does and equals mode 1 bit for bit whenever mode 1's
    result is monotone."""
    rng = np.random.default_rng(3)
    zero1 = 0
    compared = 0
    for scale in (20.0, 100.0, 300.0):
        for _ in range(400):
            lg = (rng.standard_normal(256) * scale).astype(np.float32)
            s0 = oracle.cdf_build(lg, mode=0)
            s1 = oracle.cdf_build(lg, mode=1)
            f0 = np.diff(oracle.cdf_quantize(s0).astype(np.int64))
            f1 = np.diff(oracle.cdf_quantize(s1).astype(np.int64))
            assert (f0 >= 1).all()
            zero1 += (f1 < 1).any()
            if (np.diff(s1[:256]) >= 0).all():
                assert np.array_equal(s0, s1)
                compared += 1
    assert zero1 > 0 and compared > 500


def test_cdf_one_hot_and_bias(oracle):
    lg = np.zeros(256, np.float32)
    lg[77] = 1e4
    q = oracle.cdf_quantize(oracle.cdf_build(lg)).astype(np.int64)
    f = np.diff(q)
    assert f[77] == (1 << 24) - 255 and (np.delete(f, 77) == 1).all()
    # bias is added before anything else (decoder path, range_coder_kernels.cu:668)
    rng = np.random.default_rng(1)
    a = rng.standard_normal(256).astype(np.float32)
    b = rng.standard_normal(256).astype(np.float32)
    assert np.array_equal(oracle.cdf_build(a, b), oracle.cdf_build(a + b))


def test_cdf_temperature_power_of_two(oracle):
    rng = np.random.default_rng(2)
    lg = rng.standard_normal(256).astype(np.float32)
    # (l - m) * 2 is exact, so inv_temperature = 2 equals doubled logits
    assert np.array_equal(oracle.cdf_build(lg, None, 2.0), oracle.cdf_build(lg * 2))


# ------------------------------------------------------------- coder
def bigint_words(cdf_rows, syms):
    """Arbitrary-precision model of the coder: no 64-bit window, so carries
    propagate by integer addition instead of inverted-run bookkeeping.
    Returns the expected word stream."""
    if len(syms) == 0:
        return []
    lo, rng, shifts = 0, (1 << 64) - 1, 0
    for row, s in zip(cdf_rows, syms):
        s = int(s)
        left, prob = int(row[s]), int(row[s + 1]) - int(row[s])
        prob = prob or 1
        scale = rng >> 24
        lo += scale * left
        rng = scale * prob
        while rng < (1 << 32):
            lo <<= 32
            rng <<= 32
            shifts += 1
    point = lo + (1 << 32) - 1
    n_words = shifts + 1
    top = point >> 32
    words = [(top >> (32 * (n_words - 1 - i))) & 0xFFFFFFFF for i in range(n_words)]
    # final window: low 64 bits of lower and of lower+range
    win_lo = lo & ((1 << 64) - 1)
    upper = (win_lo + rng) & ((1 << 64) - 1)
    point_w = (((win_lo + (1 << 32) - 1) & ((1 << 64) - 1)) >> 32)
    if (upper >> 32) == point_w:
        words.append(0)
    return words


def random_cdf(rng, skew):
    w = rng.random(256) ** skew
    w = np.maximum(w / w.sum() * ((1 << 24) - 256), 0).astype(np.int64) + 1
    w[rng.integers(256)] += (1 << 24) - int(w.sum())
    q = np.zeros(257, np.uint32)
    q[1:] = np.cumsum(w)
    return q


def test_coder_hand_worked_kat(oracle):
    # one symbol, left = 0, prob = 2^23: range' = (2^40-1) 2^23, no
    # renormalisation; finish emits point>>32 = 0 and no extra word because
    # upper>>32 = 0x7FFFFFFF
    cdf = np.zeros((1, 257), np.uint32)
    cdf[0, 1:] = 1 << 24
    cdf[0, 1] = 1 << 23
    assert list(oracle.encode_cdf_stream(cdf, np.array([0], np.uint8))) == [0]
    assert len(oracle.encode_cdf_stream(cdf[:0], np.array([], np.uint8))) == 0


@pytest.mark.parametrize("skew", [1.0, 6.0, 30.0])
def test_coder_matches_bigint_model_and_round_trips(oracle, skew):
    rng = np.random.default_rng(int(skew * 10))
    for trial in range(30):
        n = int(rng.integers(0, 300))
        cdf = np.stack([random_cdf(rng, skew) for _ in range(n)]) if n else np.zeros((0, 257), np.uint32)
        syms = np.array([rng.choice(256, p=np.diff(c.astype(np.int64)) / (1 << 24)) for c in cdf],
                        np.uint8)
        words = oracle.encode_cdf_stream(cdf, syms)
        assert list(words) == bigint_words(cdf, syms), f"trial {trial}"
        assert np.array_equal(oracle.decode_cdf_stream(cdf, n, words), syms)


def test_coder_carries_and_inverted_runs(oracle):
    """Symbols at the very top of the interval push `lower` towards 2^64 and
    force carries and long inverted runs; count them with the stepwise API."""
    import ctypes as C
    L = oracle.lib()
    rng = np.random.default_rng(9)
    saw_inverted = saw_long = 0
    for trial in range(40):
        n = 400
        cdf = np.zeros((n, 257), np.uint32)
        syms = np.zeros(n, np.uint8)
        for i in range(n):
            c = random_cdf(rng, 1.0)
            if rng.random() < 0.7:       # a near-certain top symbol
                c = np.arange(257, dtype=np.uint32)
                c[256] = 1 << 24
                c[255] = (1 << 24) - int(rng.integers(1, 4))
                syms[i] = 255 if rng.random() < 0.9 else rng.integers(255)
            else:
                syms[i] = rng.choice(256, p=np.diff(c.astype(np.int64)) / (1 << 24))
            cdf[i] = c
        st = oracle.RcEnc()
        L.ref_rc_enc_init(C.byref(st))
        buf = np.zeros(4 * n + 8, np.uint32)
        max_inv = 0
        for i in range(n):
            s = int(syms[i])
            L.ref_rc_enc_put(C.byref(st), int(cdf[i, s]), int(cdf[i, s + 1] - cdf[i, s]), buf)
            max_inv = max(max_inv, st.inverted_num)
        saw_inverted += max_inv > 0
        saw_long += max_inv > 2
        words = oracle.encode_cdf_stream(cdf, syms)
        assert list(words) == bigint_words(cdf, syms)
        assert np.array_equal(oracle.decode_cdf_stream(cdf, n, words), syms)
    assert saw_inverted > 0 and saw_long > 0


def test_coder_exhaustive_tiny_alphabet(oracle):
    """All messages of length <= 5 over a 3-symbol distribution."""
    import itertools
    base = np.zeros(257, np.uint32)
    freqs = np.ones(256, np.int64)
    freqs[[3, 100, 200]] = [(1 << 23), (1 << 22), 0]
    freqs[200] = (1 << 24) - int(freqs.sum()) + 0
    base[1:] = np.cumsum(freqs)
    assert base[256] == 1 << 24
    for n in range(6):
        for msg in itertools.product([3, 100, 200], repeat=n):
            cdf = np.tile(base, (n, 1))
            syms = np.array(msg, np.uint8)
            words = oracle.encode_cdf_stream(cdf, syms)
            assert list(words) == bigint_words(cdf, syms)
            assert np.array_equal(oracle.decode_cdf_stream(cdf, n, words), syms)


# --------------------------------------------------------- container
def test_crc32_and_leb128_kats(oracle):
    assert oracle.crc32(b"123456789") == 0xCBF43926
    blob = np.random.default_rng(0).integers(0, 256, 10000, dtype=np.uint8).tobytes()
    assert oracle.crc32(blob) == zlib.crc32(blob)
    assert oracle.uvarint(0) == b"\x00"
    assert oracle.uvarint(127) == b"\x7f"
    assert oracle.uvarint(128) == b"\x80\x01"
    assert oracle.uvarint(300) == b"\xac\x02"
    assert oracle.uvarint(2 ** 63) == b"\x80" * 9 + b"\x01"
