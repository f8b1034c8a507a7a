"""GPU parity of the kernels behind the IBackend-level entry points, through
the C ABI, against the CPU oracle on the same inputs.

Dequantisation is bit-exact (every fp16 bit pattern; random blocks of every
dtype).  Products use fp32 accumulation in a different order from the
oracle's sequential sums, so they are compared with a relative tolerance of
1e-4 of the largest output magnitude per row (TOL below).
"""
import numpy as np
import pytest

import pyoracle as P
from xwfes_amd import ftx

pytestmark = pytest.mark.gpu

TOL = 1e-4  # max|gpu - oracle| / max|oracle| per output row


def rel_err_rows(a, b):
    a = np.atleast_2d(a).astype(np.float64)
    b = np.atleast_2d(b).astype(np.float64)
    return (np.abs(a - b).max(axis=1) / np.maximum(np.abs(b).max(axis=1), 1e-30)).max()


def random_blocks(rng, dtype, rows, cols):
    """Random bytes with finite, moderate fp16 scale fields."""
    be, bb = P.BLOCK[dtype]
    nb = rows * P.row_bytes(dtype, cols)
    raw = rng.integers(0, 256, nb, dtype=np.uint8)
    if dtype == P.F32:
        return rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8).copy()
    if dtype in (P.F16, P.BF16):
        hi = raw[1::2]
        raw[1::2] = (0x20 + (hi & 0x1F)) | (hi & 0x80) if dtype == P.F16 else \
            (0x3C + (hi & 0x03)) | (hi & 0x80)
        return raw
    hdr = {P.Q4_0: [0], P.Q8_0: [0], P.Q4_1: [0, 2], P.Q4_K: [0, 2], P.Q6_K: [208]}[dtype]
    nblk = nb // bb
    for off in hdr:
        idx = np.arange(nblk) * bb + off + 1
        raw[idx] = 0x20 + (raw[idx] & 0x1F)
    return raw


def test_device_info(gctx):
    info = gctx.info()
    assert info["compute_units"] > 0 and info["mem_bytes"] > 0
    assert "gfx950" in info["name"]


def test_half_to_float_exhaustive(gctx, orc):
    """Every fp16 bit pattern through the F16 dequant path."""
    hs = np.arange(65536, dtype=np.uint16)
    t = gctx.upload(hs.view(np.uint8), ftx.F16, (65536, 1))
    got = gctx.dequant(t)[0]
    t.free()
    want = orc.dequant(hs.view(np.uint8), P.F16, 65536)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype", [P.F32, P.F16, P.BF16, P.Q4_0, P.Q4_1, P.Q8_0, P.Q4_K, P.Q6_K])
def test_dequant_bit_exact(gctx, orc, dtype):
    rng = np.random.default_rng(100 + dtype)
    rows, cols = 37, 1024
    raw = random_blocks(rng, dtype, rows, cols)
    t = gctx.upload(raw, dtype, (cols, rows))
    got = gctx.dequant(t)
    t.free()
    want = orc.dequant(raw, dtype, cols, rows=rows)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", [P.Q4_0, P.Q8_0])
def test_dequant_ragged_row(gctx, orc, dtype):
    """Rows whose length is not a whole number of blocks (the reference
    truncates the last block, include/ft/quant.h:31-60)."""
    rng = np.random.default_rng(7)
    rows, cols = 5, 100
    raw = random_blocks(rng, dtype, rows, cols)
    t = gctx.upload(raw, dtype, (cols, rows))
    got = gctx.dequant(t)
    t.free()
    want = orc.dequant(raw, dtype, cols, rows=rows)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def rand_weight(orc, rng, rows, cols, dtype, std=0.02):
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    return orc.quantize(w, dtype)


@pytest.mark.parametrize("dtype", [P.Q4_K, P.Q6_K, P.Q4_0, P.Q8_0, P.F16, P.F32, P.BF16, P.Q4_1])
@pytest.mark.parametrize("M", [1, 3, 8, 13])
def test_matmul_vs_oracle(gctx, orc, dtype, M):
    rng = np.random.default_rng(dtype * 31 + M)
    K, N = 1024, 96
    raw = rand_weight(orc, rng, N, K, dtype)
    t = gctx.upload(raw, dtype, (K, N))
    x = rng.standard_normal((M, K)).astype(np.float32)
    got = gctx.matmul(x, t)
    t.free()
    want = orc.matmul(x, raw, dtype, N)
    assert rel_err_rows(got, want) < TOL


@pytest.mark.parametrize("M", [1, 2, 5, 8])
@pytest.mark.parametrize("N", [96, 1000, 4128])
def test_matmul_mfma_q4k_vs_oracle(gctx, orc, M, N):
    """K = 4096 Q4_K takes the int8-MFMA row-dot path (split sums over the
    contraction for small N, ragged last tile for N = 96)."""
    rng = np.random.default_rng(M * 1000 + N)
    K = 4096
    raw = rand_weight(orc, rng, N, K, P.Q4_K)
    t = gctx.upload(raw, P.Q4_K, (K, N))
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[-1, :7] *= 40.0   # outliers in the first 256-element block of the last row
    got = gctx.matmul(x, t)
    t.free()
    want = orc.matmul(x, raw, P.Q4_K, N)
    assert rel_err_rows(got[:-1], want[:-1]) < TOL if M > 1 else True
    # the activation limbs are relative to each block's maximum: a block with
    # 40x outliers carries its other values 40x more coarsely
    assert rel_err_rows(got[-1:], want[-1:]) < 3 * TOL


@pytest.mark.parametrize("M", [1, 3, 8])
@pytest.mark.parametrize("N", [64, 1000])
def test_matmul_mfma_q6k_vs_oracle(gctx, orc, M, N):
    """K = 4096 Q6_K: planar device layout, int8-MFMA over 16-element
    sub-blocks."""
    rng = np.random.default_rng(M * 77 + N)
    K = 4096
    raw = rand_weight(orc, rng, N, K, P.Q6_K)
    t = gctx.upload(raw, P.Q6_K, (K, N))
    x = rng.standard_normal((M, K)).astype(np.float32)
    got = gctx.matmul(x, t)
    t.free()
    want = orc.matmul(x, raw, P.Q6_K, N)
    assert rel_err_rows(got, want) < TOL


def test_q6k_device_layout_roundtrip(gctx, orc):
    """The planar Q6_K layout dequantises bit-exactly, including rows whose
    super-block count is odd (padded rows)."""
    rng = np.random.default_rng(12)
    for cols in (256, 768, 4096):
        raw = random_blocks(rng, P.Q6_K, 9, cols)
        t = gctx.upload(raw, P.Q6_K, (cols, 9))
        got = gctx.dequant(t)
        t.free()
        want = orc.dequant(raw, P.Q6_K, cols, rows=9)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), cols


def test_matmul_mfma_zero_row(gctx, orc):
    """An all-zero activation row gives zeros (row scale 0)."""
    rng = np.random.default_rng(3)
    K, N = 4096, 64
    raw = rand_weight(orc, rng, N, K, P.Q4_K)
    t = gctx.upload(raw, P.Q4_K, (K, N))
    x = rng.standard_normal((3, K)).astype(np.float32)
    x[1] = 0.0
    got = gctx.matmul(x, t)
    t.free()
    assert np.all(got[1] == 0.0)
    want = orc.matmul(x, raw, P.Q4_K, N)
    assert rel_err_rows(got[[0, 2]], want[[0, 2]]) < TOL


def test_matmul_rows_are_independent(gctx, orc):
    """An M-row product equals M single-row products (the reference's M-sum
    behaviour, src/cpu_backend.cpp:98-101, is not reproduced)."""
    rng = np.random.default_rng(5)
    K, N = 512, 40
    raw = rand_weight(orc, rng, N, K, P.Q4_K)
    t = gctx.upload(raw, P.Q4_K, (K, N))
    x = rng.standard_normal((6, K)).astype(np.float32)
    y = gctx.matmul(x, t)
    for m in range(6):
        assert np.array_equal(gctx.matmul(x[m:m + 1], t)[0], y[m])
    t.free()


@pytest.mark.parametrize("dtype", [P.Q4_K, P.Q6_K, P.Q4_0, P.Q8_0, P.F32])
@pytest.mark.parametrize("M", [1, 8, 11])
def test_down_axpy_vs_oracle(gctx, orc, dtype, M):
    rng = np.random.default_rng(dtype * 7 + M)
    n_in, N = 768, 512
    raw = rand_weight(orc, rng, n_in, N, dtype)
    t = gctx.upload(raw, dtype, (N, n_in))
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    x[:, ::5] = 0.0
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    got = gctx.down_axpy(x, t, y0)
    t.free()
    want = orc.down_axpy(x, raw, dtype, N, y0)
    assert rel_err_rows(got - y0, want - y0) < TOL


def test_expert_chunk_equals_direct_ffn(gctx, orc):
    """run_expert_chunk semantics (src/cpu_backend.cpp:106-149): SwiGLU of a
    window of IC neurons, then the down rows accumulated into out; chunked ==
    direct (the reference test_chunker, src/tests/test_core.cpp:307-346)."""
    rng = np.random.default_rng(9)
    M, K, FF, C = 3, 256, 96, 32
    dt = P.Q8_0
    g = rand_weight(orc, rng, FF, K, dt)
    u = rand_weight(orc, rng, FF, K, dt)
    dn = rand_weight(orc, rng, FF, K, dt)
    tg, tu, td = (gctx.upload(r, dt, (K, FF)) for r in (g, u, dn))
    x = rng.standard_normal((M, K)).astype(np.float32)
    rb = P.row_bytes(dt, K)
    out = np.zeros((M, K), np.float32)
    for i0 in range(0, FF, C):
        out = gctx.expert_chunk(x, tg.ptr + i0 * rb, tu.ptr + i0 * rb, td.ptr + i0 * rb, out,
                                dt, C)
    hg = orc.matmul(x, g, dt, FF)
    hu = orc.matmul(x, u, dt, FF)
    h = (hg / (1.0 + np.exp(-hg.astype(np.float64)))).astype(np.float32) * hu
    want = orc.down_axpy(h, dn, dt, K)
    for t in (tg, tu, td):
        t.free()
    assert rel_err_rows(out, want) < 1e-4


def test_quantize_roundtrip_on_device(gctx, orc):
    """ftx_quantize output dequantises close to its input (builder sanity)."""
    rng = np.random.default_rng(11)
    src = gctx.buffer(16 * 1024 * 4)
    for dt, tol in ((P.Q4_K, 0.07), (P.Q6_K, 0.03), (P.Q4_0, 0.09), (P.Q8_0, 0.006)):
        w = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float32)
        src.write(w)
        t = gctx.alloc(dt, (1024, 16))
        gctx.quantize(src.ptr, t)
        got = gctx.dequant(t)
        t.free()
        assert np.abs(got - w).max() / np.abs(w).max() < tol
    src.free()


def test_fill_normal_moments(gctx):
    n = 1 << 20
    b = gctx.buffer(n * 4)
    gctx.fill_normal(b.ptr, n, seed=3, std=0.02)
    x = b.read(np.float32, n).astype(np.float64)
    assert abs(x.mean()) < 1e-4 and abs(x.std() - 0.02) < 2e-4
    # same seed, same values; f16 output is the rounded f32 stream
    gctx.fill_normal(b.ptr, n // 2, seed=3, std=0.02, dtype=ftx.F16)
    h = b.read(np.float16, n // 2)
    assert np.array_equal(h, x[: n // 2].astype(np.float32).astype(np.float16))
    b.free()


def test_errors_are_reported(gctx):
    rng = np.random.default_rng(1)
    raw = rand_weight(P.Oracle(), rng, 8, 64, P.Q8_0)
    t = gctx.upload(raw, P.Q8_0, (64, 8))
    with pytest.raises(ftx.FtxError) as e:
        gctx.matmul(np.zeros((2, 32), np.float32), t)
    assert e.value.code == -1 and "K must equal" in str(e.value)
    t.free()
