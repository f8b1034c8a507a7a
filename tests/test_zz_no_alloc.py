"""ftx_down_axpy_noalloc (no counterpart in the reference: ftx_down_axpy for
callers that cannot allocate) against ftx_down_axpy through the C ABI, on
device buffers.  Both run the same kernels in the same order, so the outputs
are bit-identical; two calls in a row (the second on a smaller input) show
that the shared scratch array keeps no state a later call depends on.  The
error paths (host buffers, a shape above the scratch limit) return their
codes without launching anything."""
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
