"""Seeded synthetic inputs and random-init weights for the codec benchmarks.

Weight files use the byte layout that ``convert_boa_weights.py`` writes and
``BoaPredictorGPU::load_weights`` reads (reference:
portability_solved_cpp/convert_boa_weights.py:153-241, boa_gpu.hpp:990-1029):
a 4-byte magic ``BOA\\x00`` (fp32) or ``BOA\\x01`` (fp16), then raw
little-endian tensors in PyTorch [out, in] order:

    embedding.weight [256, d]
    per block: ln1.w, ln1.b, in_proj.w [2di, d], in_proj.b [2di], conv1d.w
      [di, 1, 4], conv1d.b [di], x_proj.w [r+2ds, di], dt_proj.w [di, r],
      dt_proj.b [di], A_log [di, ds], D [di], out_proj.w [d, di],
      out_proj.b [d], ln2.w, ln2.b, ff.0.w [4d, d], ff.0.b [4d],
      ff.2.w [d, 4d], ff.2.b [d]
    head.0.w [d, d], head.0.b [d], head.2.w [256, d], head.2.b [256]

The file carries no dimensions: d_model and n_layers come from the command
line (boa.cpp:912-920); d_inner = 2 d, dt_rank = ceil(d/16).
"""
from __future__ import annotations

import math
import os

import numpy as np

VOCAB = 256


def dims(d_model: int, d_state: int = 16):
    di = 2 * d_model
    r = (d_model + 15) // 16
    return di, r, r + 2 * d_state


def expected_weight_bytes(d_model: int, n_layers: int, d_state: int = 16, fp16: bool = False) -> int:
    d = d_model
    di, r, R = dims(d, d_state)
    per_layer = (2 * d + 2 * di * d + 2 * di + di * 4 + di + R * di + di * r + di
                 + di * d_state + di + d * di + d + 2 * d + 4 * d * d + 4 * d + 4 * d * d + d)
    elems = VOCAB * d + n_layers * per_layer + d * d + d + VOCAB * d + VOCAB
    return 4 + elems * (2 if fp16 else 4)


def random_weight_tensors(d_model: int, n_layers: int, d_state: int = 16, seed: int = 0):
    """Mamba-style random init, drawn in file order from default_rng(seed).

    Linear W, b ~ U(+-1/sqrt(fan_in)) (in_proj/out_proj biases are zero, as
    the converter writes them); conv W, b ~ U(+-1/2); x_proj ~ U(+-1/sqrt(di));
    dt_proj.w ~ U(+-r^-1/2); dt_proj.b = softplus^-1(exp(U(ln 1e-3, ln 1e-1)));
    A_log[c, n] = ln(n+1); D = 1; LayerNorm w = 1, b = 0; embedding ~ N(0, 1).
    Returns a list of (name, float32 array) in file order.
    """
    rng = np.random.default_rng(seed)
    d = d_model
    di, r, R = dims(d, d_state)
    out = []

    def uni(shape, bound):
        return rng.uniform(-bound, bound, size=shape).astype(np.float32)

    out.append(("embedding.weight", rng.standard_normal((VOCAB, d)).astype(np.float32)))
    for i in range(n_layers):
        p = f"blocks.{i}."
        out.append((p + "ln1.weight", np.ones(d, np.float32)))
        out.append((p + "ln1.bias", np.zeros(d, np.float32)))
        out.append((p + "mamba.in_proj.weight", uni((2 * di, d), 1 / math.sqrt(d))))
        out.append((p + "mamba.in_proj.bias", np.zeros(2 * di, np.float32)))
        out.append((p + "mamba.conv1d.weight", uni((di, 1, 4), 0.5)))
        out.append((p + "mamba.conv1d.bias", uni((di,), 0.5)))
        out.append((p + "mamba.x_proj.weight", uni((R, di), 1 / math.sqrt(di))))
        out.append((p + "mamba.dt_proj.weight", uni((di, r), r ** -0.5)))
        dt = np.exp(rng.uniform(math.log(1e-3), math.log(1e-1), size=di))
        out.append((p + "mamba.dt_proj.bias", (dt + np.log(-np.expm1(-dt))).astype(np.float32)))
        out.append((p + "mamba.A_log", np.tile(np.log(np.arange(1, d_state + 1, dtype=np.float64)),
                                               (di, 1)).astype(np.float32)))
        out.append((p + "mamba.D", np.ones(di, np.float32)))
        out.append((p + "mamba.out_proj.weight", uni((d, di), 1 / math.sqrt(di))))
        out.append((p + "mamba.out_proj.bias", np.zeros(d, np.float32)))
        out.append((p + "ln2.weight", np.ones(d, np.float32)))
        out.append((p + "ln2.bias", np.zeros(d, np.float32)))
        out.append((p + "ff.0.weight", uni((4 * d, d), 1 / math.sqrt(d))))
        out.append((p + "ff.0.bias", uni((4 * d,), 1 / math.sqrt(d))))
        out.append((p + "ff.2.weight", uni((d, 4 * d), 1 / math.sqrt(4 * d))))
        out.append((p + "ff.2.bias", uni((d,), 1 / math.sqrt(4 * d))))
    out.append(("head.0.weight", uni((d, d), 1 / math.sqrt(d))))
    out.append(("head.0.bias", uni((d,), 1 / math.sqrt(d))))
    out.append(("head.2.weight", uni((VOCAB, d), 1 / math.sqrt(d))))
    out.append(("head.2.bias", uni((VOCAB,), 1 / math.sqrt(d))))
    return out


def write_weights(path: str, tensors, fp16: bool = False) -> int:
    """Write (name, array) pairs in the BOA weight layout; returns bytes written."""
    with open(path, "wb") as f:
        f.write(b"BOA\x01" if fp16 else b"BOA\x00")
        for _, t in tensors:
            a = np.ascontiguousarray(t, dtype=np.float16 if fp16 else np.float32)
            f.write(a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes())
    return os.path.getsize(path)


def write_random_weights(path: str, d_model: int, n_layers: int, d_state: int = 16,
                         seed: int = 0, fp16: bool = False) -> int:
    return write_weights(path, random_weight_tensors(d_model, n_layers, d_state, seed), fp16)


def convert_state_dict(sd, d_state: int = 16):
    """Order a mambav1 PyTorch state dict the way convert_boa_weights.py does
    (reference convert_boa_weights.py:186-239); missing in/out_proj biases
    become zeros.  `sd` maps names to array-likes."""
    def arr(k):
        v = sd[k]
        v = v.float().numpy() if hasattr(v, "numpy") else np.asarray(v)
        return np.asarray(v, dtype=np.float32)

    out = [("embedding.weight", arr("embedding.weight"))]
    i = 0
    while f"blocks.{i}.ln1.weight" in sd:
        p = f"blocks.{i}."
        m = p + "mamba."
        out.append((p + "ln1.weight", arr(p + "ln1.weight")))
        out.append((p + "ln1.bias", arr(p + "ln1.bias")))
        w_in = arr(m + "in_proj.weight")
        out.append((m + "in_proj.weight", w_in))
        out.append((m + "in_proj.bias", arr(m + "in_proj.bias") if m + "in_proj.bias" in sd
                    else np.zeros(w_in.shape[0], np.float32)))
        out.append((m + "conv1d.weight", arr(m + "conv1d.weight")))
        if m + "conv1d.bias" in sd:
            out.append((m + "conv1d.bias", arr(m + "conv1d.bias")))
        for k in ("x_proj.weight", "dt_proj.weight", "dt_proj.bias", "A_log", "D", "out_proj.weight"):
            out.append((m + k, arr(m + k)))
        w_out = arr(m + "out_proj.weight")
        out.append((m + "out_proj.bias", arr(m + "out_proj.bias") if m + "out_proj.bias" in sd
                    else np.zeros(w_out.shape[0], np.float32)))
        out.append((p + "ln2.weight", arr(p + "ln2.weight")))
        out.append((p + "ln2.bias", arr(p + "ln2.bias")))
        ff = p + "ff" if p + "ff.0.weight" in sd else p + "ff.net"
        for k in (".0.weight", ".0.bias", ".2.weight", ".2.bias"):
            out.append((ff + k, arr(ff + k)))
        i += 1
    for k in ("head.0.weight", "head.0.bias", "head.2.weight", "head.2.bias"):
        out.append((k, arr(k)))
    return out, i


# --------------------------------------------------------------------------
# Benchmark inputs (seeded), one generator per configuration.
# --------------------------------------------------------------------------
def gen_c1() -> bytes:
    """1 MiB of little-endian float32 N(0,1) values rounded to 3 decimals (seed 1)."""
    rng = np.random.default_rng(1)
    return np.round(rng.standard_normal(262144), 3).astype("<f4").tobytes()


def gen_c2(n_records: int = 2_097_152) -> bytes:
    """64 MiB of interleaved float32 records of 8 fields: 4 exponential(lambda=0.1)
    then 4 uniform(-pi, pi) (seed 2)."""
    rng = np.random.default_rng(2)
    a = rng.exponential(scale=10.0, size=(n_records, 4))
    b = rng.uniform(-math.pi, math.pi, size=(n_records, 4))
    return np.hstack([a, b]).astype("<f4").tobytes()


def gen_c3(n_blocks: int = 65536) -> bytes:
    """256 MiB of alternating 4 KiB blocks: int16 Poisson(20) counts and
    float32 N(0,1) values (seed 3)."""
    rng = np.random.default_rng(3)
    parts = []
    for i in range(n_blocks):
        if i % 2 == 0:
            parts.append(rng.poisson(20, size=2048).astype("<i2").tobytes())
        else:
            parts.append(rng.standard_normal(1024).astype("<f4").tobytes())
    return b"".join(parts)


def _markov_fill():
    """synth_markov_fill from libsynth.so (built next to this file), or None."""
    import ctypes as C
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsynth.so")
    if not os.path.exists(path):
        return None
    fn = C.CDLL(path).synth_markov_fill
    fn.restype = C.c_int
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_void_p]
    return fn


def gen_c4(n: int = 268_435_456, block: int = 1 << 24) -> bytes:
    """First-order Markov bytes: rows of a 256x256 transition matrix are
    Dirichlet(0.05) draws (seed 4), x0 = 0; x_{t+1} is the inverse-CDF draw
    of row x_t at u_t, the uniforms taken from the same generator in blocks
    (the same stream as one rng.random(n) call)."""
    rng = np.random.default_rng(4)
    P = rng.dirichlet(np.full(256, 0.05), size=256)
    cum = np.ascontiguousarray(np.cumsum(P, axis=1))
    out = np.empty(n, np.uint8)
    fill = _markov_fill()
    x = 0
    for s in range(0, n, block):
        u = rng.random(min(block, n - s))
        if fill is not None:
            x = fill(cum.ctypes.data, u.ctypes.data, len(u), x, out[s:].ctypes.data)
            continue
        for t in range(len(u)):
            out[s + t] = x
            x = min(int(np.searchsorted(cum[x], u[t])), 255)
    return out.tobytes()


def gen_c5(n: int = 268_435_456) -> bytes:
    """1 GiB of float32 Gaussian-mixture values (seed 5)."""
    rng = np.random.default_rng(5)
    c = rng.choice(3, p=[0.5, 0.3, 0.2], size=n)
    x = rng.normal(loc=np.array([0.0, 5.0, -3.0])[c], scale=np.array([1.0, 0.5, 2.0])[c])
    return x.astype("<f4").tobytes()


# model shape, precision, chunk count, input generator
CONFIGS = {
    "c1": dict(d_model=64, n_layers=2, d_state=16, precision="fp32", chunks=64, gen=gen_c1),
    "c2": dict(d_model=256, n_layers=8, d_state=16, precision="fp32", chunks=1000, gen=gen_c2),
    "c3": dict(d_model=256, n_layers=8, d_state=16, precision="bf16", chunks=8192, gen=gen_c3),
    "c4": dict(d_model=256, n_layers=8, d_state=16, precision="fp32", chunks=4096, gen=gen_c4),
    "c5": dict(d_model=512, n_layers=12, d_state=32, precision="bf16", chunks=16384, gen=gen_c5),
}


def chunk_size_for(n_bytes: int, chunks: int) -> int:
    return (n_bytes + chunks - 1) // chunks
