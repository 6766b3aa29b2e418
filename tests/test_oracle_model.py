"""CPU tests pinning the oracle's model forward, weight loader and container.

The model is checked against an independent float64 numpy restatement of
the mambav1 equations (Mamba selective scan, Gu & Dao; LayerNorm; tanh GELU;
Linear-ReLU-Linear head) written from the mathematics, not from the oracle's
code.  Chunk-mode and step-mode logits of the oracle must be bit-identical
(the decoder re-derives the encoder's CDFs from them).
"""
import os
import struct
import zlib

import numpy as np
import pytest

import synth


# ------------------------------------------------------ float64 restatement
def _ln(x, w, b):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + 1e-5) * w + b


def _softplus(x):
    return np.logaddexp(0.0, x)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _gelu_tanh(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def np_forward(tensors, tokens, d, L, ds):
    t = {k: v.astype(np.float64) for k, v in tensors}
    di, r = 2 * d, (d + 15) // 16
    x = t["embedding.weight"][tokens]
    T = len(tokens)
    for i in range(L):
        p = f"blocks.{i}."
        m = p + "mamba."
        h = _ln(x, t[p + "ln1.weight"], t[p + "ln1.bias"])
        xz = h @ t[m + "in_proj.weight"].T + t[m + "in_proj.bias"]
        xs, z = xz[:, :di], xz[:, di:]
        w = t[m + "conv1d.weight"][:, 0, :]               # [di, 4]
        xp = np.concatenate([np.zeros((3, di)), xs], 0)   # causal, zero history
        conv = t[m + "conv1d.bias"] + sum(w[:, k] * xp[k:k + T] for k in range(4))
        u = _silu(conv)
        dbc = u @ t[m + "x_proj.weight"].T
        dt = _softplus(dbc[:, :r] @ t[m + "dt_proj.weight"].T + t[m + "dt_proj.bias"])
        Bm, Cm = dbc[:, r:r + ds], dbc[:, r + ds:]
        A = -np.exp(t[m + "A_log"])                        # [di, ds]
        hs = np.zeros((di, ds))
        ys = np.empty((T, di))
        for s in range(T):
            hs = np.exp(dt[s][:, None] * A) * hs + (dt[s][:, None] * Bm[s][None, :]) * u[s][:, None]
            ys[s] = hs @ Cm[s] + t[m + "D"] * u[s]
        y = ys * (z * (1.0 / (1.0 + np.exp(-z))))
        out = y @ t[m + "out_proj.weight"].T + t[m + "out_proj.bias"]
        h2 = _ln(out, t[p + "ln2.weight"], t[p + "ln2.bias"])
        ff = _gelu_tanh(h2 @ t[p + "ff.0.weight"].T + t[p + "ff.0.bias"]) @ t[p + "ff.2.weight"].T
        x = x + ff + t[p + "ff.2.bias"]
    hh = np.maximum(0.0, x @ t["head.0.weight"].T + t["head.0.bias"])
    return hh @ t["head.2.weight"].T + t["head.2.bias"]


@pytest.mark.parametrize("d,L,ds", [(64, 2, 16), (32, 1, 32), (80, 1, 16), (256, 2, 16),
                                    (512, 1, 32), (100, 1, 16), (37, 1, 16), (200, 1, 32)])
def test_forward_matches_float64_restatement(oracle, weights_dir, d, L, ds):
    """Up to C2's width (K = 1024 in FF2) and C5's (d_model 512, d_state 32,
    K = 2048), d_model 80 (dt_rank 5, rows not a multiple of 32), and widths
    between the GPU kernels' built widths (100, 37 and 200, which the GPU runs
    zero-padded to 128, 64 and 256)."""
    tensors = synth.random_weight_tensors(d, L, ds, seed=1)
    path = weights_dir / f"np_{d}_{L}_{ds}.bin"
    synth.write_weights(str(path), tensors)
    rng = np.random.default_rng(4)
    tok = rng.integers(0, 256, size=(2, 30), dtype=np.uint8)
    m = oracle.Model(path, d, L, ds)
    got = m.new_state(2).forward_chunk(tok)
    for b in range(2):
        want = np_forward(tensors, tok[b], d, L, ds)
        np.testing.assert_allclose(got[b], want, rtol=1e-4, atol=1e-4 * np.abs(want).max())


def test_long_sequence_matches_float64_restatement(oracle, weights_dir):
    """C2's width over 2,048 tokens: with dt about 1e-3 .. 1e-1 the scan state
    carries hundreds to thousands of steps of history, so rounding drift in
    the recurrence would show here and not in 30-token runs."""
    d, L, ds, T = 256, 2, 16, 2048
    tensors = synth.random_weight_tensors(d, L, ds, seed=0)
    path = weights_dir / f"np_long_{d}_{L}_{ds}.bin"
    synth.write_weights(str(path), tensors)
    rng = np.random.default_rng(11)
    tok = rng.integers(0, 256, size=(2, T), dtype=np.uint8)
    got = oracle.Model(path, d, L, ds).new_state(2).forward_chunk(tok)
    for b in range(2):
        want = np_forward(tensors, tok[b], d, L, ds)
        np.testing.assert_allclose(got[b], want, rtol=1e-4, atol=1e-4 * np.abs(want).max())


def _scan_float32_reference_order(oracle, w_dt, b_dt, dd, a_log, delta, u, z, h, fused=False):
    """The reference's chunk scan (mamba_kernels.cu:414-470, every product
    and sum rounded on its own: dB = dt B; h = (dA h) + (dB u); y = y + h C;
    y = y + D u) followed by the gate (:130-151), in numpy float32, whose
    scalar + and * are single IEEE roundings.  The transcendentals (softplus,
    the base-2 decay, exp) are the oracle's own, pinned elsewhere.
    fused=True computes the fma form h = fma(dA, h, B (dt u)),
    y = fma(h, C, y) instead (float64 products then one rounding), the form
    the update must not take."""
    L = oracle.lib()
    f = np.float32
    r, ds = len(w_dt), len(a_log)
    na2 = [f(L.ref_scan_na2(float(a))) for a in a_log]
    h = [f(v) for v in h]
    ys = []
    for t in range(len(u)):
        # the dt inputs and weights are dyadic, so the K-order chain is exact
        acc = f(sum(float(delta[t, j]) * float(w_dt[j]) for j in range(r)))
        dt = f(L.ref_softplus(float(acc + f(b_dt))))
        ut, B, Cv = f(u[t]), delta[t, r:r + ds], delta[t, r + ds:]
        y = f(0.0)
        if fused:
            dtu = f(dt * ut)
        for n in range(ds):
            dA = f(L.ref_exp2_neg(float(na2[n] * dt)))
            if fused:
                h[n] = f(float(dA) * float(h[n]) + float(f(B[n] * dtu)))
                y = f(float(h[n]) * float(Cv[n]) + float(y))
            else:
                dB = dt * f(B[n])
                h[n] = dA * h[n] + dB * ut
                y = y + h[n] * f(Cv[n])
        y = y + f(dd) * ut
        sg = f(1.0) / (f(1.0) + f(L.ref_expf(float(-f(z[t])))))
        ys.append(y * (f(z[t]) * sg))
    return np.array(ys, np.float32), np.array(h, np.float32)


def test_scan_update_rounds_like_the_reference(oracle):
    """The oracle's scan rounds every product and sum of the state update on
    its own, as the reference's __fmul_rn / __fadd_rn lines do, bit for bit
    over 4,096 tokens; the fused (fma) form differs, so the check sees it."""
    rng = np.random.default_rng(21)
    r, ds, T = 16, 16, 4096
    w_dt = (rng.integers(-8, 9, size=r) / 64).astype(np.float32)
    a_log = np.log(np.arange(1, ds + 1)).astype(np.float32)
    delta = rng.standard_normal((T, r + 2 * ds)).astype(np.float32)
    delta[:, :r] = rng.integers(-8, 9, size=(T, r)) / 16
    u = rng.standard_normal(T).astype(np.float32)
    z = rng.standard_normal(T).astype(np.float32)
    h0 = (0.1 * rng.standard_normal(ds)).astype(np.float32)
    b_dt, dd = -4.5, 1.0
    y, h = oracle.scan_channel(w_dt, b_dt, dd, a_log, delta, u, z, h0)
    want_y, want_h = _scan_float32_reference_order(oracle, w_dt, b_dt, dd, a_log, delta, u, z, h0)
    assert np.array_equal(y.view(np.uint32), want_y.view(np.uint32))
    assert np.array_equal(h.view(np.uint32), want_h.view(np.uint32))
    fy, fh = _scan_float32_reference_order(oracle, w_dt, b_dt, dd, a_log, delta, u, z, h0, fused=True)
    assert not np.array_equal(fy.view(np.uint32), y.view(np.uint32))


def test_chunk_step_and_tile_bit_identity(oracle, w_c1):
    m = oracle.Model(w_c1, 64, 2)
    rng = np.random.default_rng(8)
    tok = rng.integers(0, 256, size=(3, 70), dtype=np.uint8)
    whole = m.new_state(3).forward_chunk(tok)
    st = m.new_state(3)
    parts = [st.forward_chunk(tok[:, a:b]) for a, b in ((0, 1), (1, 3), (3, 40), (40, 70))]
    tiled = np.concatenate(parts, 1)
    assert np.array_equal(whole.view(np.uint32), tiled.view(np.uint32))
    st = m.new_state(3)
    step = np.stack([st.step(tok[:, t]) for t in range(70)], 1)
    assert np.array_equal(whole.view(np.uint32), step.view(np.uint32))
    # without the head bias, adding it afterwards rounds the same way
    st = m.new_state(3)
    nob = np.stack([st.step(tok[:, t], add_bias=False) for t in range(5)], 1)
    tensors = dict(synth.random_weight_tensors(64, 2, 16, seed=0))
    assert np.array_equal((nob + tensors["head.2.bias"]).view(np.uint32), whole[:, :5].view(np.uint32))


def test_fp16_weights_equal_widened_fp32(oracle, weights_dir):
    tensors = synth.random_weight_tensors(64, 1, 16, seed=2)
    p16 = weights_dir / "w16.bin"
    p32 = weights_dir / "w16as32.bin"
    synth.write_weights(str(p16), tensors, fp16=True)
    synth.write_weights(str(p32), [(k, v.astype(np.float16).astype(np.float32)) for k, v in tensors])
    assert os.path.getsize(p16) == synth.expected_weight_bytes(64, 1, 16, fp16=True)
    tok = np.arange(40, dtype=np.uint8).reshape(2, 20)
    a = oracle.Model(p16, 64, 1).new_state(2).forward_chunk(tok)
    b = oracle.Model(p32, 64, 1).new_state(2).forward_chunk(tok)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_weight_sizes_and_loader_errors(oracle, w_c1, weights_dir):
    # sizes of the convert_boa_weights.py layout for the BASELINE configs
    assert synth.expected_weight_bytes(64, 2) == 679_172
    assert synth.expected_weight_bytes(256, 8) == 31_688_708
    assert synth.expected_weight_bytes(512, 12, 32) == 186_813_444
    assert oracle.lib().ref_model_expected_bytes(256, 8, 16, 0) == 31_688_708
    with pytest.raises(ValueError, match="expected"):
        oracle.Model(w_c1, 64, 3)
    # headerless legacy fp32 file (boa_gpu.hpp:1001-1005)
    raw = open(w_c1, "rb").read()
    legacy = weights_dir / "legacy.bin"
    legacy.write_bytes(raw[4:])
    tok = np.arange(20, dtype=np.uint8).reshape(1, 20)
    a = oracle.Model(w_c1, 64, 2).new_state(1).forward_chunk(tok)
    b = oracle.Model(legacy, 64, 2).new_state(1).forward_chunk(tok)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- container
def parse_boa2(blob):
    """Independent struct-level reader of the BOA2 layout (boa.cpp:538-581)."""
    magic, ver, flags, total, chunk, n, last, fp_len = struct.unpack_from("<4sIIQIIIB", blob, 0)
    assert magic == b"BOA2" and ver == 1
    p = 33 + fp_len
    idx = blob.rindex(b"IDX2", 0, len(blob) - 4)
    crc = struct.unpack_from("<I", blob, len(blob) - 4)[0]
    assert crc == zlib.crc32(blob[idx:len(blob) - 4])
    q = idx + 4
    first = blob[q:q + n]
    q += n
    lens = []
    for _ in range(n):
        v, shift = 0, 0
        while True:
            bt = blob[q]
            q += 1
            v |= (bt & 0x7F) << shift
            shift += 7
            if not bt & 0x80:
                break
        lens.append(v)
    assert q == len(blob) - 4
    streams, off = [], p
    for ln in lens:
        streams.append(blob[off:off + ln])
        off += ln
    assert off == idx
    return dict(flags=flags, total=total, chunk=chunk, n=n, last=last, first=first, streams=streams)


def test_container_layout_and_per_chunk_streams(oracle, w_c1):
    data = synth.gen_c1()[:5 * 1000 + 1]          # last chunk has one byte
    m = oracle.Model(w_c1, 64, 2)
    blob = m.compress(data, chunk_size=1000)
    c = parse_boa2(blob)
    assert (c["flags"], c["total"], c["chunk"], c["n"], c["last"]) == (0, len(data), 1000, 6, 1)
    assert c["first"] == bytes(data[i * 1000] for i in range(6))
    assert c["streams"][-1] == b""                 # a 1-byte chunk codes nothing
    for i in range(5):
        words = m.encode_chunk(data[i * 1000:(i + 1) * 1000])
        assert c["streams"][i] == words.tobytes()
    assert m.decompress(blob) == data
    # --max-chunks truncates (boa.cpp:296-299)
    blob3 = m.compress(data, chunk_size=1000, max_chunks=3)
    c3 = parse_boa2(blob3)
    assert (c3["n"], c3["total"], c3["last"]) == (3, 3000, 1000)
    assert m.decompress(blob3) == data[:3000]


def test_container_error_paths(oracle, w_c1):
    m = oracle.Model(w_c1, 64, 2)
    blob = m.compress(synth.gen_c1()[:3000], chunk_size=1000)
    assert oracle.boa2_parse(blob)[0] == 0
    assert oracle.boa2_parse(blob[:20])[0] == -1                      # too short
    assert oracle.boa2_parse(b"XOA2" + blob[4:])[0] == -2             # magic
    assert oracle.boa2_parse(blob[:4] + b"\x02" + blob[5:])[0] == -3  # version
    bad = bytearray(blob)
    bad[-6] ^= 0x55                                                    # index byte
    assert oracle.boa2_parse(bytes(bad))[0] == -6                     # CRC
    no_idx = blob.replace(b"IDX2", b"IDY2")
    assert oracle.boa2_parse(no_idx)[0] == -4
    # forge the last stream's length past the payload, with a valid CRC
    c = parse_boa2(blob)
    idx = blob.rindex(b"IDX2")
    lens = [len(x) for x in c["streams"]]
    lens[-1] += 1_000_000
    index = b"IDX2" + c["first"] + b"".join(oracle.uvarint(v) for v in lens)
    forged = blob[:idx] + index + struct.pack("<I", zlib.crc32(index))
    assert oracle.boa2_parse(forged)[0] == -8


REF_CKPT = "/root/reference/experiments/cms_experiment/cms_experiment_final_model_fp32_mambav1_64_2_20ep.pt"


@pytest.mark.skipif(not os.path.exists(REF_CKPT), reason="reference checkpoint not mounted")
def test_real_checkpoint_round_trip(oracle, weights_dir):
    """A trained mambav1 checkpoint from the reference (d64, 2 layers, the
    BASELINE config-1 shape, trained on CMS jet features that are not in the
    container), converted with this repo's writer: the oracle round-trips
    the config-1 input, and compresses a run of zero bytes."""
    import torch
    ck = torch.load(REF_CKPT, map_location="cpu", weights_only=True)
    sd = ck["state_dict"] if "state_dict" in ck else ck
    tensors, n_layers = synth.convert_state_dict(sd)
    assert n_layers == 2
    p = weights_dir / "ckpt_64_2.bin"
    synth.write_weights(str(p), tensors)
    m = oracle.Model(p, 64, 2)
    data = synth.gen_c1()[:16384]
    blob = m.compress(data, chunk_size=4096)
    assert m.decompress(blob) == data
    zeros = bytes(8192)
    zblob = m.compress(zeros, chunk_size=4096)
    assert m.decompress(zblob) == zeros
    assert len(zblob) * 1.3 < len(zeros)


def test_bf16_rounding_kats(oracle):
    to = oracle.lib().ref_f32_to_bf16
    f = lambda u: np.array([u], np.uint32).view(np.float32)[0]
    assert to(1.0) == 0x3F80
    assert to(f(0x3F808000)) == 0x3F80          # tie -> even
    assert to(f(0x3F818000)) == 0x3F82          # tie -> even (odd below)
    assert to(f(0x3F808001)) == 0x3F81          # above the tie
    assert to(f(0x7F7FFFFF)) == 0x7F80          # rounds up to +inf
    assert to(f(0x7FC00001)) & 0x7FC0 == 0x7FC0  # NaN stays NaN
    v = np.random.default_rng(3).standard_normal(10000).astype(np.float32)
    bits = np.array([to(float(x)) for x in v], np.uint32) << 16
    back = bits.view(np.float32)
    assert np.all(np.abs(back - v) <= np.abs(v) * 2.0 ** -8)


def test_bf16_model_close_to_fp32_and_chunk_equals_step(oracle, w_c1):
    tok = np.random.default_rng(9).integers(0, 256, size=(3, 50), dtype=np.uint8)
    a = oracle.Model(w_c1, 64, 2).new_state(3).forward_chunk(tok)
    m16 = oracle.Model(w_c1, 64, 2, bf16=True)
    b = m16.new_state(3).forward_chunk(tok)
    assert not np.array_equal(a, b)
    assert np.abs(a - b).max() <= 2e-2 * np.abs(a).max()
    st = m16.new_state(3)
    step = np.stack([st.step(tok[:, t]) for t in range(50)], 1)
    assert np.array_equal(b.view(np.uint32), step.view(np.uint32))
    data = synth.gen_c1()[:3000]
    blob = m16.compress(data, chunk_size=700)
    assert m16.decompress(blob) == data
