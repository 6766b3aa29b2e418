"""Python binding of the MI355X codec library (libboa_hip.so, C ABI in
include/boa_hip.h).

This is plumbing for tests, the benchmark and smoke(): the product is the C
ABI and the `boa` CLI.  Device buffers are passed as raw pointers (torch
tensors' data_ptr() or hipMalloc'd memory).  Importing the module never
falls back to anything: if the library is missing or fails to load, every
entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libboa_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "boa_hip.h")

BOA_OK = 0
(K_GEMM, K_SCAN, K_CONV, K_LN, K_CDF, K_CODER, K_DECODE, K_GEMM_SMALL, K_DEC_GEMM,
 K_DEC_SCAN, K_HEAD_CDF, K_DEC_LNGEMM) = range(12)
K_NAMES = ["gemm", "scan", "conv", "ln", "cdf", "coder", "decode", "gemm_small", "dec_gemm",
           "dec_scan", "head_cdf", "dec_lngemm"]
BOA_E_ARG, BOA_E_HIP, BOA_E_IO, BOA_E_FORMAT, BOA_E_STATE, BOA_E_NOMEM = -1, -2, -3, -4, -5, -6

# void (*)(void* user, int32_t phase, int64_t done_bytes, int64_t total_bytes)
PROGRESS_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int32, C.c_int64, C.c_int64)


class BoaError(RuntimeError):
    def __init__(self, msg, rc=None):
        super().__init__(msg)
        self.rc = rc


class Config(C.Structure):
    _fields_ = [("d_model", C.c_int32), ("n_layers", C.c_int32), ("d_state", C.c_int32),
                ("max_lanes", C.c_int32), ("tile", C.c_int32), ("precision", C.c_int32),
                ("temperature", C.c_float)]


def build(clean: bool = False) -> str:
    """Compile libboa_hip.so and the boa CLI for gfx950 (hipcc)."""
    if clean:
        subprocess.run(["make", "-s", "-C", HERE, "clean"], check=True)
    subprocess.run(["make", "-s", "-C", HERE, "-j4"], check=True)
    return LIB_PATH


def declared_symbols() -> list[str]:
    """Function names declared in include/boa_hip.h."""
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(boa_[a-z0-9_]+)\s*\(", txt)))


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise BoaError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        P, i32, i64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float
        sig = {
            "boa_create": (C.c_int, [C.POINTER(Config), C.POINTER(P)]),
            "boa_destroy": (None, [P]),
            "boa_last_error": (C.c_char_p, [P]),
            "boa_set_stream": (C.c_int, [P, P]),
            "boa_use_own_stream": (C.c_int, [P]),
            "boa_set_temperature": (C.c_int, [P, f32]),
            "boa_set_warm_start": (C.c_int, [P, i32]),
            "boa_set_progress": (C.c_int, [P, PROGRESS_FN, P]),
            "boa_decode_plan": (C.c_int, [P, i32, C.POINTER(i32), C.POINTER(i32)]),
            "boa_set_state_cache_budget": (C.c_int, [P, i64]),
            "boa_last_timings": (C.c_int, [P, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                           C.POINTER(C.c_double)]),
            "boa_load_weights": (C.c_int, [P, C.c_char_p]),
            "boa_load_weights_mem": (C.c_int, [P, P, C.c_size_t]),
            "boa_weight_file_bytes": (i64, [i32, i32, i32, i32]),
            "boa_estimate_memory": (i64, [C.POINTER(Config), i64, i32]),
            "boa_reset_state": (C.c_int, [P, i32]),
            "boa_forward_chunk": (C.c_int, [P, P, i32, i32, P]),
            "boa_step_batch": (C.c_int, [P, P, i32, P, i32]),
            "boa_forward_chunk_noalloc": (C.c_int, [P, P, i32, i32, P]),
            "boa_cdf_from_logits": (C.c_int, [P, P, P, i32, P]),
            "boa_cdf_from_probs": (C.c_int, [P, P, i32, i32, P]),
            "boa_rc_encode_cdf": (C.c_int, [P, P, P, i32, i32, P, i64, P]),
            "boa_rc_decode_cdf": (C.c_int, [P, P, i32, i32, P, i64, P, P]),
            "boa_compress_device": (C.c_int, [P, P, i64, i64, i32, P, i64, P, P, P]),
            "boa_num_chunks": (i64, [i64, i64, i32]),
            "boa_payload_bound_words": (i64, [i64, i64, i32]),
            "boa_decompress_device": (C.c_int, [P, P, P, P, P, i32, i64, i64, P]),
            "boa_compress_buffer": (C.c_int, [P, P, i64, i64, i32, C.POINTER(P), C.POINTER(i64)]),
            "boa_decompress_buffer": (C.c_int, [P, P, i64, C.POINTER(P), C.POINTER(i64)]),
            "boa_compress_file": (C.c_int, [P, C.c_char_p, C.c_char_p, i64, i32]),
            "boa_decompress_file": (C.c_int, [P, C.c_char_p, C.c_char_p]),
            "boa_free": (None, [P]),
            "boa_crc32": (C.c_uint32, [P, i64]),
            "boa_profile_enable": (C.c_int, [P, i32]),
            "boa_profile_reset": (C.c_int, [P]),
            "boa_profile_read": (C.c_int, [P, i32, C.POINTER(C.c_double), C.POINTER(i64),
                                           C.POINTER(C.c_double)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


class Codec:
    """One context: weights, recurrent state and work buffers on one GPU."""

    def __init__(self, d_model, n_layers, d_state=16, max_lanes=64, tile=0, temperature=1.0,
                 precision="fp32"):
        prec = {"fp32": 0, "bf16": 1}[precision]
        self.cfg = Config(d_model, n_layers, d_state, max_lanes, tile, prec, temperature)
        h = C.c_void_p()
        rc = lib().boa_create(C.byref(self.cfg), C.byref(h))
        if rc != BOA_OK:
            raise BoaError(f"boa_create failed ({rc})")
        self.h = h

    def _check(self, rc, what):
        if rc != BOA_OK:
            raise BoaError(f"{what} failed ({rc}): {lib().boa_last_error(self.h).decode()}", rc)

    def close(self):
        if getattr(self, "h", None):
            lib().boa_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load_weights(self, path):
        self._check(lib().boa_load_weights(self.h, str(path).encode()), "load_weights")

    def set_stream(self, stream_ptr):
        self._check(lib().boa_set_stream(self.h, stream_ptr), "set_stream")

    def reset_state(self, lanes):
        self._check(lib().boa_reset_state(self.h, lanes), "reset_state")

    def forward_chunk(self, d_tokens, lanes, T, d_logits):
        self._check(lib().boa_forward_chunk(self.h, _ptr(d_tokens), lanes, T, _ptr(d_logits)),
                    "forward_chunk")

    def forward_chunk_noalloc(self, d_tokens, lanes, T, d_logits):
        """boa_forward_chunk with its activations in the library's fixed
        per-GPU scratch array (no device allocation during the call)."""
        self._check(lib().boa_forward_chunk_noalloc(self.h, _ptr(d_tokens), lanes, T,
                                                    _ptr(d_logits)), "forward_chunk_noalloc")

    def step_batch(self, d_tokens, lanes, d_logits, add_bias=True):
        self._check(lib().boa_step_batch(self.h, _ptr(d_tokens), lanes, _ptr(d_logits),
                                         1 if add_bias else 0), "step_batch")

    def cdf_from_logits(self, d_logits, d_bias, rows, d_qcdf):
        self._check(lib().boa_cdf_from_logits(self.h, _ptr(d_logits), _ptr(d_bias), rows,
                                              _ptr(d_qcdf)), "cdf_from_logits")

    def cdf_from_probs(self, d_probs, rows, K, d_qcdf):
        self._check(lib().boa_cdf_from_probs(self.h, _ptr(d_probs), rows, K, _ptr(d_qcdf)),
                    "cdf_from_probs")

    def rc_encode_cdf(self, d_cdf, d_syms, n_sym, lanes, d_words, pitch_words, d_sizes):
        self._check(lib().boa_rc_encode_cdf(self.h, _ptr(d_cdf), _ptr(d_syms), n_sym, lanes,
                                            _ptr(d_words), pitch_words, _ptr(d_sizes)),
                    "rc_encode_cdf")

    def rc_decode_cdf(self, d_cdf, n_sym, lanes, d_words, pitch_words, d_sizes, d_syms):
        self._check(lib().boa_rc_decode_cdf(self.h, _ptr(d_cdf), n_sym, lanes, _ptr(d_words),
                                            pitch_words, _ptr(d_sizes), _ptr(d_syms)),
                    "rc_decode_cdf")

    def compress_device(self, d_data, n, chunk_size, d_payload, cap_words, max_chunks=0):
        import numpy as np
        nc = lib().boa_num_chunks(n, chunk_size, max_chunks)
        lens = np.zeros(max(nc, 1), np.uint64)
        first = np.zeros(max(nc, 1), np.uint8)
        words = C.c_int64()
        self._check(lib().boa_compress_device(self.h, _ptr(d_data), n, chunk_size, max_chunks,
                                              _ptr(d_payload), cap_words, lens.ctypes.data,
                                              first.ctypes.data, C.byref(words)),
                    "compress_device")
        return lens[:nc], first[:nc], words.value

    def decompress_device(self, d_payload, offsets_words, stream_bytes, first, chunk_len,
                          last_len, d_out):
        import numpy as np
        offs = np.ascontiguousarray(offsets_words, np.uint64)
        lens = np.ascontiguousarray(stream_bytes, np.uint64)
        fb = np.ascontiguousarray(first, np.uint8)
        self._check(lib().boa_decompress_device(self.h, _ptr(d_payload), offs.ctypes.data,
                                                lens.ctypes.data, fb.ctypes.data, len(fb),
                                                chunk_len, last_len, _ptr(d_out)),
                    "decompress_device")

    def set_progress(self, fn):
        """fn(phase, done_bytes, total_bytes) during compress (phase 0) and
        decompress (phase 1); None turns the reports off."""
        if fn is None:
            self._progress = None
            self._check(lib().boa_set_progress(self.h, PROGRESS_FN(), None), "set_progress")
            return
        self._progress = PROGRESS_FN(lambda _u, ph, done, total: fn(ph, done, total))
        self._check(lib().boa_set_progress(self.h, self._progress, None), "set_progress")

    def decode_plan(self, lanes):
        """The decode step's schedule at `lanes` lanes: dict(cached_layers,
        fused_ln, persistent, fused_xproj, fused_head)."""
        a, f = C.c_int32(), C.c_int32()
        self._check(lib().boa_decode_plan(self.h, lanes, C.byref(a), C.byref(f)), "decode_plan")
        return dict(cached_layers=a.value, fused_ln=bool(f.value & 1),
                    persistent=bool(f.value & 2), fused_xproj=bool(f.value & 4),
                    fused_head=bool(f.value & 8))

    def last_timings(self):
        """(h2d_s, compute_s, d2h_s) of the last compress()/decompress() call."""
        a, b, c = C.c_double(), C.c_double(), C.c_double()
        self._check(lib().boa_last_timings(self.h, C.byref(a), C.byref(b), C.byref(c)),
                    "last_timings")
        return a.value, b.value, c.value

    def set_state_cache_budget(self, nbytes):
        self._check(lib().boa_set_state_cache_budget(self.h, int(nbytes)), "set_state_cache_budget")

    def set_warm_start(self, interleave_batch):
        """--warm-start (boa.cpp:310-319): 0 turns it off."""
        self._check(lib().boa_set_warm_start(self.h, int(interleave_batch)), "set_warm_start")

    def compress(self, data: bytes, chunk_size=4096, max_chunks=0) -> bytes:
        import numpy as np
        buf = np.frombuffer(data, np.uint8)
        out = C.c_void_p()
        n = C.c_int64()
        self._check(lib().boa_compress_buffer(self.h, buf.ctypes.data if len(data) else None,
                                              len(data), chunk_size, max_chunks, C.byref(out),
                                              C.byref(n)), "compress_buffer")
        res = C.string_at(out, n.value)
        lib().boa_free(out)
        return res

    def decompress(self, blob: bytes) -> bytes:
        import numpy as np
        buf = np.frombuffer(blob, np.uint8)
        out = C.c_void_p()
        n = C.c_int64()
        self._check(lib().boa_decompress_buffer(self.h, buf.ctypes.data, len(blob), C.byref(out),
                                                C.byref(n)), "decompress_buffer")
        res = C.string_at(out, n.value)
        lib().boa_free(out)
        return res

    def profile(self, on=True):
        self._check(lib().boa_profile_enable(self.h, 1 if on else 0), "profile_enable")

    def profile_reset(self):
        self._check(lib().boa_profile_reset(self.h), "profile_reset")

    def profile_read(self):
        out = {}
        for k, name in enumerate(K_NAMES):
            ms = C.c_double()
            n = C.c_int64()
            w = C.c_double()
            self._check(lib().boa_profile_read(self.h, k, C.byref(ms), C.byref(n), C.byref(w)),
                        "profile_read")
            out[name] = dict(ms=ms.value, launches=n.value, work=w.value)
        return out


def payload_bound_words(n, chunk_size, max_chunks=0):
    return lib().boa_payload_bound_words(n, chunk_size, max_chunks)
