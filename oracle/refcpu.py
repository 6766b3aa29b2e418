"""ctypes binding of the CPU oracle (oracle/librefcpu.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, and only as the checker / CPU baseline.  The
product path never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# Two builds of the same source: x86-64-v3 (AVX2 + FMA; the tests' default)
# and x86-64-v4 (AVX-512), chosen with REFCPU_ISA=v4 before the first load.
# Neither reassociates nor contracts floating-point operations
# (-ffp-contract=off, no -ffast-math), so both compute the same bits.
ISA_LIBS = {"v3": "librefcpu.so", "v4": "librefcpu_v4.so"}
ISA = os.environ.get("REFCPU_ISA", "v3")
LIB_PATH = os.path.join(HERE, ISA_LIBS.get(ISA, ISA_LIBS["v3"]))


def host_has_avx512() -> bool:
    """AVX-512 F/BW/CD/DQ/VL, the x86-64-v4 level, on this host."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= fl
    except OSError:
        pass
    return False


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


class RcEnc(C.Structure):
    _fields_ = [("lower", C.c_uint64), ("range", C.c_uint64), ("inverted_num", C.c_int32),
                ("first_inv_lower_word", C.c_uint32), ("write_idx_words", C.c_int32),
                ("pad_", C.c_int32)]


class RcDec(C.Structure):
    _fields_ = [("lower", C.c_uint64), ("range", C.c_uint64), ("point", C.c_uint64),
                ("read_idx_words", C.c_int32), ("pad_", C.c_int32)]


class CodecOpts(C.Structure):
    _fields_ = [("chunk_size", C.c_int64), ("gpu_batch", C.c_int32), ("tile", C.c_int32),
                ("max_chunks", C.c_int32), ("n_threads", C.c_int32), ("temperature", C.c_float),
                ("warm_start", C.c_int32)]


class Boa2Info(C.Structure):
    _fields_ = [("total_size", C.c_uint64), ("chunk_len", C.c_uint32), ("n_chunks", C.c_uint32),
                ("last_chunk_len", C.c_uint32), ("flags", C.c_uint32),
                ("interleave_batch", C.c_uint32), ("payload_off", C.c_int64),
                ("idx_off", C.c_int64), ("idx_version", C.c_int32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C")
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C")
        u32p = np.ctypeslib.ndpointer(np.uint32, flags="C")
        u8p = np.ctypeslib.ndpointer(np.uint8, flags="C")
        sig = {
            "ref_expf": (C.c_float, [C.c_float]),
            "ref_exp2_neg": (C.c_float, [C.c_float]),
            "ref_scan_na2": (C.c_float, [C.c_float]),
            "ref_logf": (C.c_float, [C.c_float]),
            "ref_repro_exp": (C.c_float, [C.c_float]),
            "ref_repro_tanh": (C.c_float, [C.c_float]),
            "ref_gelu": (C.c_float, [C.c_float]),
            "ref_silu": (C.c_float, [C.c_float]),
            "ref_softplus": (C.c_float, [C.c_float]),
            "ref_scan_channel": (None, [f32p, C.c_float, C.c_float, f32p, C.c_int32, C.c_int32,
                                        C.c_int32, f32p, f32p, f32p, f32p, f32p]),
            "ref_half_to_float": (C.c_float, [C.c_uint16]),
            "ref_rc_enc_init": (None, [C.POINTER(RcEnc)]),
            "ref_rc_enc_put": (None, [C.POINTER(RcEnc), C.c_uint32, C.c_uint32, u32p]),
            "ref_rc_enc_finish": (C.c_int32, [C.POINTER(RcEnc), u32p]),
            "ref_rc_dec_init": (None, [C.POINTER(RcDec), u32p, C.c_int32]),
            "ref_rc_dec_target": (C.c_uint32, [C.POINTER(RcDec)]),
            "ref_rc_dec_advance": (None, [C.POINTER(RcDec), C.c_uint32, C.c_uint32, u32p, C.c_int32]),
            "ref_rc_encode_cdf_stream": (C.c_int32, [u32p, u8p, C.c_int32, u32p]),
            "ref_rc_decode_cdf_stream": (None, [u32p, C.c_int32, u32p, C.c_int32, u8p]),
            "ref_cdf_build": (None, [f32p, P, C.c_float, f64p]),
            "ref_cdf_build_mode": (None, [f32p, P, C.c_float, f64p, C.c_int32]),
            "ref_cdf_interval": (None, [f64p, C.c_int32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
            "ref_cdf_quantize": (None, [f64p, u32p]),
            "ref_cdf_from_probs": (None, [f32p, C.c_int32, u32p]),
            "ref_cdf_search": (C.c_int32, [f64p, C.c_uint32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
            "ref_model_load": (P, [C.c_char_p, C.c_int32, C.c_int32, C.c_int32, C.c_char_p, C.c_int32]),
            "ref_model_set_bf16": (C.c_int32, [P]),
            "ref_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "ref_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "ref_model_free": (None, [P]),
            "ref_model_expected_bytes": (C.c_int64, [C.c_int32, C.c_int32, C.c_int32, C.c_int32]),
            "ref_state_new": (P, [P, C.c_int32]),
            "ref_state_reset": (None, [P]),
            "ref_state_free": (None, [P]),
            "ref_forward_chunk": (None, [P, P, u8p, C.c_int32, C.c_int32, f32p, C.c_int32]),
            "ref_step": (None, [P, P, u8p, C.c_int32, f32p, C.c_int32, C.c_int32]),
            "ref_compress": (C.c_int32, [P, P, C.c_int64, C.POINTER(CodecOpts), C.POINTER(P),
                                         C.POINTER(C.c_int64)]),
            "ref_decompress": (C.c_int32, [P, P, C.c_int64, C.POINTER(CodecOpts), C.POINTER(P),
                                           C.POINTER(C.c_int64)]),
            "ref_free": (None, [P]),
            "ref_encode_chunk": (C.c_int32, [P, u8p, C.c_int32, C.c_int32, C.c_float, u32p, C.c_int32]),
            "ref_crc32": (C.c_uint32, [P, C.c_int64]),
            "ref_uvarint_encode": (C.c_int32, [C.c_uint64, u8p]),
            "ref_boa2_parse": (C.c_int32, [P, C.c_int64, C.POINTER(Boa2Info), P, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


# ----------------------------------------------------------------- helpers
def cdf_build(logits, bias=None, inv_temperature=1.0, mode=0):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty(257, np.float64)
    b = None
    if bias is not None:
        b = np.ascontiguousarray(bias, dtype=np.float32)
    lib().ref_cdf_build_mode(lg, b.ctypes.data if b is not None else None, inv_temperature, out,
                             mode)
    return out


def cdf_quantize(s_cdf):
    q = np.empty(257, np.uint32)
    lib().ref_cdf_quantize(np.ascontiguousarray(s_cdf, dtype=np.float64), q)
    return q


def cdf_from_probs(probs):
    p = np.ascontiguousarray(probs, dtype=np.float32)
    out = np.empty(len(p) + 1, np.uint32)
    lib().ref_cdf_from_probs(p, len(p), out)
    return out


def encode_cdf_stream(cdf, syms):
    cdf = np.ascontiguousarray(cdf, dtype=np.uint32).reshape(-1, 257)
    syms = np.ascontiguousarray(syms, dtype=np.uint8)
    out = np.zeros(4 * len(syms) + 8, np.uint32)
    n = lib().ref_rc_encode_cdf_stream(cdf, syms, len(syms), out)
    return out[:n].copy()


def decode_cdf_stream(cdf, n_sym, words):
    cdf = np.ascontiguousarray(cdf, dtype=np.uint32).reshape(-1, 257)
    w = np.ascontiguousarray(words, dtype=np.uint32)
    if w.size == 0:
        w = np.zeros(1, np.uint32)
        nw = 0
    else:
        nw = len(words)
    out = np.zeros(n_sym, np.uint8)
    lib().ref_rc_decode_cdf_stream(cdf, n_sym, w, nw, out)
    return out


def scan_channel(w_dt, b_dt, dd, a_log, delta, u, z, h):
    """One channel's chunk-mode scan over T tokens (ref_scan_channel):
    returns (y [T], new state [ds])."""
    w_dt = np.ascontiguousarray(w_dt, dtype=np.float32)
    a_log = np.ascontiguousarray(a_log, dtype=np.float32)
    delta = np.ascontiguousarray(delta, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    z = np.ascontiguousarray(z, dtype=np.float32)
    hs = np.array(h, dtype=np.float32)
    T, ds, r = len(u), len(a_log), len(w_dt)
    assert delta.shape == (T, r + 2 * ds) and ds <= 64
    y = np.empty(T, np.float32)
    lib().ref_scan_channel(w_dt, float(b_dt), float(dd), a_log, r, ds, T, delta, u, z, hs, y)
    return y, hs


class Model:
    def __init__(self, path, d_model, n_layers, d_state=16, bf16=False):
        err = C.create_string_buffer(512)
        h = lib().ref_model_load(str(path).encode(), d_model, n_layers, d_state, err, 512)
        if not h:
            raise ValueError(err.value.decode())
        self.h = h
        self.d_model, self.n_layers, self.d_state = d_model, n_layers, d_state
        if bf16:
            lib().ref_model_set_bf16(h)

    def close(self):
        if self.h:
            lib().ref_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def new_state(self, lanes):
        return State(self, lanes)

    def compress(self, data: bytes, chunk_size=4096, tile=0, max_chunks=0, n_threads=0,
                 temperature=1.0, warm_start=False, gpu_batch=64) -> bytes:
        """boa.cpp compress_v2; warm_start interleaves chunks over gpu_batch lanes."""
        o = CodecOpts(chunk_size, gpu_batch, tile, max_chunks, n_threads, temperature,
                      1 if warm_start else 0)
        out = C.c_void_p()
        n = C.c_int64()
        buf = np.frombuffer(data, np.uint8)
        rc = lib().ref_compress(self.h, buf.ctypes.data, len(data), C.byref(o), C.byref(out), C.byref(n))
        if rc:
            raise RuntimeError(f"ref_compress failed: {rc}")
        res = C.string_at(out, n.value)
        lib().ref_free(out)
        return res

    def decompress(self, blob: bytes, n_threads=0, temperature=1.0) -> bytes:
        o = CodecOpts(0, 64, 0, 0, n_threads, temperature, 0)
        out = C.c_void_p()
        n = C.c_int64()
        buf = np.frombuffer(blob, np.uint8)
        rc = lib().ref_decompress(self.h, buf.ctypes.data, len(blob), C.byref(o), C.byref(out), C.byref(n))
        if rc:
            raise RuntimeError(f"ref_decompress failed: {rc}")
        res = C.string_at(out, n.value)
        lib().ref_free(out)
        return res

    def encode_chunk(self, chunk: bytes, tile=0, temperature=1.0):
        buf = np.frombuffer(chunk, np.uint8).copy()
        cap = (len(chunk) * 10 + 4096 + 3) // 4
        out = np.zeros(cap, np.uint32)
        n = lib().ref_encode_chunk(self.h, buf, len(chunk), tile, temperature, out, cap)
        if n < 0:
            raise RuntimeError("encode_chunk overflow")
        return out[:n].copy()


class State:
    def __init__(self, model: Model, lanes: int):
        self.model = model
        self.lanes = lanes
        self.h = lib().ref_state_new(model.h, lanes)

    def reset(self):
        lib().ref_state_reset(self.h)

    def __del__(self):
        try:
            lib().ref_state_free(self.h)
        except Exception:
            pass

    def forward_chunk(self, tokens, n_threads=0):
        tok = np.ascontiguousarray(tokens, dtype=np.uint8)
        lanes, T = tok.shape
        out = np.empty((lanes, T, 256), np.float32)
        lib().ref_forward_chunk(self.model.h, self.h, tok, lanes, T, out, n_threads)
        return out

    def step(self, tokens, add_bias=True, n_threads=0):
        tok = np.ascontiguousarray(tokens, dtype=np.uint8)
        out = np.empty((len(tok), 256), np.float32)
        lib().ref_step(self.model.h, self.h, tok, len(tok), out, 1 if add_bias else 0, n_threads)
        return out


def crc32(data: bytes) -> int:
    buf = np.frombuffer(data, np.uint8)
    return lib().ref_crc32(buf.ctypes.data if len(data) else None, len(data))


def uvarint(x: int) -> bytes:
    out = np.zeros(10, np.uint8)
    n = lib().ref_uvarint_encode(x, out)
    return out[:n].tobytes()


def boa2_parse(blob: bytes):
    info = Boa2Info()
    buf = np.frombuffer(blob, np.uint8)
    rc = lib().ref_boa2_parse(buf.ctypes.data, len(blob), C.byref(info), None, None, None)
    if rc:
        return rc, None
    nc = info.n_chunks
    first = np.zeros(max(nc, 1), np.uint8)
    offs = np.zeros(max(nc, 1), np.uint64)
    lens = np.zeros(max(nc, 1), np.uint64)
    rc = lib().ref_boa2_parse(buf.ctypes.data, len(blob), C.byref(info), first.ctypes.data,
                              offs.ctypes.data, lens.ctypes.data)
    return rc, dict(info=info, first=first[:nc], offsets=offs[:nc], lengths=lens[:nc])
