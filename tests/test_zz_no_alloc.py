"""The allocation-free entry point boa_forward_chunk_noalloc (activations in
the library's fixed per-GPU scratch array) gives the bits of
boa_forward_chunk, through the C ABI, on two calls in a row -- the second
smaller, so it runs on what the first left in the array -- and rejects a
request beyond the array's limit with BOA_E_ARG.  On a fresh context (no
activation buffers allocated yet) it is captured into a HIP graph in global
capture mode, where any device allocation would fail the capture, and the
graph's replays give boa_forward_chunk's bits."""
import ctypes

import numpy as np
import pytest

import boa_hip

pytestmark = pytest.mark.gpu

MAX_ROWS_C2 = (64 * 2 ** 20 - 7 * 256) // (4 * (14 * 256 + 16 + 32))


def _forward(lib, h, fn, tok, lanes, T, torch):
    d_tok = torch.from_numpy(np.ascontiguousarray(tok)).cuda()
    d_log = torch.full((lanes * T * 256,), float("nan"), dtype=torch.float32, device="cuda")
    assert lib.boa_reset_state(h, lanes) == 0
    rc = fn(h, ctypes.c_void_p(d_tok.data_ptr()), lanes, T, ctypes.c_void_p(d_log.data_ptr()))
    torch.cuda.synchronize()
    return rc, d_log.cpu().numpy()


@pytest.mark.parametrize("d,L,ds,prec,shapes", [
    (256, 2, 16, 0, [(40, 100), (7, 33)]),
    (512, 1, 32, 1, [(16, 64), (3, 10)]),
])
def test_noalloc_forward_matches_forward_chunk(make_weights, d, L, ds, prec, shapes):
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    lib = boa_hip.lib()
    w = make_weights(d, L, ds)
    cfg = boa_hip.Config(d, L, ds, 64, 0, prec, 1.0)
    h = ctypes.c_void_p()
    assert lib.boa_create(ctypes.byref(cfg), ctypes.byref(h)) == 0
    try:
        assert lib.boa_set_stream(h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
        assert lib.boa_load_weights(h, str(w).encode()) == 0
        rng = np.random.default_rng(d + ds)
        for lanes, T in shapes:  # the second call is smaller than the first
            tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
            rc, want = _forward(lib, h, lib.boa_forward_chunk, tok, lanes, T, torch)
            assert rc == 0
            rc, got = _forward(lib, h, lib.boa_forward_chunk_noalloc, tok, lanes, T, torch)
            assert rc == 0, lib.boa_last_error(h)
            assert not np.isnan(got).any()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (lanes, T)
    finally:
        lib.boa_destroy(h)


def test_noalloc_rejects_rows_beyond_the_scratch(make_weights):
    import torch
    assert torch.cuda.is_available()
    lib = boa_hip.lib()
    w = make_weights(256, 2)
    cfg = boa_hip.Config(256, 2, 16, 64, 0, 0, 1.0)
    h = ctypes.c_void_p()
    assert lib.boa_create(ctypes.byref(cfg), ctypes.byref(h)) == 0
    try:
        assert lib.boa_load_weights(h, str(w).encode()) == 0
        T = MAX_ROWS_C2 // 64 + 1  # 64 lanes x T rows > the limit
        d_tok = torch.zeros(64 * T, dtype=torch.uint8, device="cuda")
        # buffers of the full request's size, so that even a missed check
        # would stay in bounds
        d_log = torch.zeros(64 * T * 256, dtype=torch.float32, device="cuda")
        rc = lib.boa_forward_chunk_noalloc(h, ctypes.c_void_p(d_tok.data_ptr()), 64, T,
                                           ctypes.c_void_p(d_log.data_ptr()))
        assert rc == boa_hip.BOA_E_ARG
        assert b"exceeds" in lib.boa_last_error(h)
    finally:
        lib.boa_destroy(h)


def _hip():
    h = ctypes.CDLL("libamdhip64.so")
    vp, P = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
    for name, args in [("hipStreamCreateWithFlags", [P, ctypes.c_uint]),
                       ("hipStreamBeginCapture", [vp, ctypes.c_int]),
                       ("hipStreamEndCapture", [vp, P]),
                       ("hipGraphInstantiate", [P, vp, vp, vp, ctypes.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]), ("hipStreamSynchronize", [vp]),
                       ("hipGraphExecDestroy", [vp]), ("hipGraphDestroy", [vp]),
                       ("hipStreamDestroy", [vp])]:
        getattr(h, name).argtypes = args
        getattr(h, name).restype = ctypes.c_int
    return h


def test_noalloc_captured_in_a_graph_on_a_fresh_context(make_weights):
    import torch
    assert torch.cuda.is_available()
    lib, hip = boa_hip.lib(), _hip()
    w = make_weights(256, 2)
    cfg = boa_hip.Config(256, 2, 16, 64, 0, 0, 1.0)
    h = ctypes.c_void_p()
    assert lib.boa_create(ctypes.byref(cfg), ctypes.byref(h)) == 0
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    try:
        assert hip.hipStreamCreateWithFlags(ctypes.byref(stream), 1) == 0  # non-blocking
        assert lib.boa_set_stream(h, stream) == 0
        assert lib.boa_load_weights(h, str(w).encode()) == 0
        lanes, T = 12, 70
        tok = np.random.default_rng(5).integers(0, 256, size=(lanes, T), dtype=np.uint8)
        d_tok = torch.from_numpy(tok).cuda()
        d_log = torch.full((lanes * T * 256,), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        assert lib.boa_reset_state(h, lanes) == 0
        assert hip.hipStreamSynchronize(stream) == 0
        # capture the first forward this context runs: it must neither
        # allocate nor synchronise
        assert hip.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
        rc = lib.boa_forward_chunk_noalloc(h, ctypes.c_void_p(d_tok.data_ptr()), lanes, T,
                                           ctypes.c_void_p(d_log.data_ptr()))
        ec = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
        assert rc == 0, lib.boa_last_error(h)
        assert ec == 0
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        # the eager reference afterwards, on the same context
        d_want = torch.empty_like(d_log)
        assert lib.boa_reset_state(h, lanes) == 0
        assert lib.boa_forward_chunk(h, ctypes.c_void_p(d_tok.data_ptr()), lanes, T,
                                     ctypes.c_void_p(d_want.data_ptr())) == 0
        assert hip.hipStreamSynchronize(stream) == 0
        want = d_want.cpu().numpy()
        for _ in range(3):  # replays, with eager work and synchronisations between
            d_log.fill_(float("nan"))
            torch.cuda.synchronize()
            assert lib.boa_reset_state(h, lanes) == 0
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            got = d_log.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        lib.boa_destroy(h)
        if stream.value:
            hip.hipStreamDestroy(stream)
