"""ftx_down_axpy_noalloc (no counterpart in the reference: ftx_down_axpy for
callers that cannot allocate) against ftx_down_axpy through the C ABI, on
device buffers.  Both run the same kernels in the same order, so the outputs
are bit-identical; two calls in a row (the second on a smaller input) show
that the shared scratch array keeps no state a later call depends on.  The
error paths (host buffers, a shape above the scratch limit) return their
codes without launching anything.  Captured into a HIP graph on a stream of
the caller's, the call records its kernels only (no allocation, memset or
synchronisation), and every replay of the graph gives the eager result."""
import ctypes

import numpy as np
import pytest

import pyoracle as P
from builders import q_rows

pytestmark = pytest.mark.gpu


def _device(gctx, a):
    a = np.ascontiguousarray(a, np.float32)
    b = gctx.buffer(a.nbytes)
    b.write(a)
    return b


@pytest.mark.parametrize("dt", [P.Q4_K, P.Q8_0])
def test_down_axpy_noalloc_matches(gctx, orc, dt):
    rng = np.random.default_rng(17)
    lib, h = gctx.lib, gctx.h
    for M, n_in, N in ((8, 2048, 1024), (3, 512, 512)):  # the second input is smaller
        w = q_rows(orc, rng, n_in, N, dt)
        W = gctx.upload(w["raw"], dt, (N, n_in))
        x = (rng.standard_normal((M, n_in)) * 0.5).astype(np.float32)
        y0 = rng.standard_normal((M, N)).astype(np.float32)
        bx, b1, b2 = _device(gctx, x), _device(gctx, y0), _device(gctx, y0)
        assert lib.ftx_down_axpy(h, bx.ptr, M, n_in, W.handle, b1.ptr) == 0
        rc = lib.ftx_down_axpy_noalloc(h, bx.ptr, M, n_in, W.handle, b2.ptr)
        assert rc == 0, gctx.error()
        got = b2.read(np.float32, M * N).reshape(M, N)
        want = b1.read(np.float32, M * N).reshape(M, N)
        assert np.array_equal(got, want), (M, n_in, N)
        assert not np.array_equal(got, y0)
        for b in (bx, b1, b2):
            b.free()
        W.free()


def test_down_axpy_noalloc_errors(gctx):
    lib, h = gctx.lib, gctx.h
    # 256 rows of 32768 outputs: one split of partials is 8 Mi floats, above
    # the 4 Mi-float scratch array
    W = gctx.alloc(P.Q8_0, (32768, 64))
    bx = gctx.buffer(256 * 64 * 4)
    by = gctx.buffer(256 * 32768 * 4)
    assert lib.ftx_down_axpy_noalloc(h, bx.ptr, 256, 64, W.handle, by.ptr) == -5  # FTX_E_RANGE
    assert "scratch" in gctx.error()
    # host buffers are refused (staging them would allocate)
    xh = np.zeros((2, 64), np.float32)
    yh = np.zeros((2, 32768), np.float32)
    assert lib.ftx_down_axpy_noalloc(h, xh.ctypes.data, 2, 64, W.handle,
                                     yh.ctypes.data) == -1  # FTX_E_INVALID
    # a row count that is not the weight's
    assert lib.ftx_down_axpy_noalloc(h, bx.ptr, 2, 32, W.handle, by.ptr) == -1
    for o in (bx, by, W):
        o.free()


def _hip():
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    for name, args in (("hipStreamCreate", [ctypes.POINTER(vp)]),
                       ("hipStreamDestroy", [vp]),
                       ("hipStreamSynchronize", [vp]),
                       ("hipStreamBeginCapture", [vp, ctypes.c_int]),
                       ("hipStreamEndCapture", [vp, ctypes.POINTER(vp)]),
                       ("hipGraphInstantiate", [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]),
                       ("hipGraphExecDestroy", [vp]),
                       ("hipGraphDestroy", [vp])):
        f = getattr(hip, name)
        f.restype = ctypes.c_int
        f.argtypes = args
    return hip


def test_down_axpy_noalloc_graph_capture(gctx, orc):
    lib, h = gctx.lib, gctx.h
    hip = _hip()
    rng = np.random.default_rng(23)
    M, n_in, N = 8, 2048, 1024
    w = q_rows(orc, rng, n_in, N, P.Q4_K)
    W = gctx.upload(w["raw"], P.Q4_K, (N, n_in))
    x = (rng.standard_normal((M, n_in)) * 0.5).astype(np.float32)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    bx, bw, by = _device(gctx, x), _device(gctx, y0), _device(gctx, y0)
    assert lib.ftx_down_axpy(h, bx.ptr, M, n_in, W.handle, bw.ptr) == 0
    want = bw.read(np.float32, M * N).reshape(M, N)
    # one eager call first: the scratch array's address is looked up then
    assert lib.ftx_down_axpy_noalloc(h, bx.ptr, M, n_in, W.handle, by.ptr) == 0, gctx.error()
    gctx.sync()
    assert np.array_equal(by.read(np.float32, M * N).reshape(M, N), want)
    st, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(st)) == 0
    try:
        gctx.set_stream(st.value)
        assert hip.hipStreamBeginCapture(st, 2) == 0  # relaxed mode
        rc = lib.ftx_down_axpy_noalloc(h, bx.ptr, M, n_in, W.handle, by.ptr)
        assert hip.hipStreamEndCapture(st, ctypes.byref(graph)) == 0
        assert rc == 0, gctx.error()
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep in range(3):
            # eager work and a synchronisation between the replays
            by.write(y0)
            assert lib.ftx_down_axpy(h, bx.ptr, M, n_in, W.handle, bw.ptr) == 0
            gctx.sync()
            assert hip.hipGraphLaunch(exe, st) == 0
            assert hip.hipStreamSynchronize(st) == 0
            got = by.read(np.float32, M * N).reshape(M, N)
            assert np.array_equal(got, want), rep
    finally:
        gctx.set_stream(None)
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        hip.hipStreamSynchronize(st)
        hip.hipStreamDestroy(st)
    for b in (bx, bw, by, W):
        b.free()
