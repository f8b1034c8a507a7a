"""Pins of the oracle's scalar and block formats.

fp16/bf16: exhaustive against IEEE (numpy) and, where built, against the
reference's own functions.  Reference block types (Q4_0 interleaved, Q8_0,
Q4_1, F16, BF16, F32): bit-exact against the reference's dequant_row /
dot_row_f32 plus hand-computed known answers.  Q4_K / Q6_K (absent from the
reference): hand-computed known answers and layout probes (flipping one
stored field changes exactly the elements the ggml layout assigns to it),
plus a quantise/dequantise round-trip bound.
"""
import struct

import numpy as np
import pytest

import pyoracle as P


def f32bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_half_to_float_exhaustive_ieee(orc):
    hs = np.arange(65536, dtype=np.uint16)
    want = hs.view(np.float16).astype(np.float32)
    got = np.array([orc.half_to_float(int(h)) for h in hs], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_half_to_float_exhaustive_reference(orc, ref):
    for h in range(65536):
        a, b = orc.half_to_float(h), ref.lib.ref_half_to_float(h)
        assert f32bits(a) == f32bits(b), hex(h)


def test_float_to_half_rne(orc):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    # focus half the sample on the half range, including subnormals
    bits[:100000] = (bits[:100000] & 0x807FFFFF) | ((rng.integers(100, 145, 100000) << 23)
                                                  .astype(np.uint32))
    xs = bits.view(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    for x, w in zip(xs, want):
        g = orc.float_to_half(float(x))
        if np.isnan(x):
            assert (g & 0x7C00) == 0x7C00 and (g & 0x3FF)
        else:
            assert g == w, (x, hex(g), hex(w))
    # edges: max half, overflow, tie to even, smallest subnormal, underflow
    for x, w in [(65504.0, 0x7BFF), (65520.0, 0x7C00), (1.0 + 2**-11, 0x3C00),
                 (1.0 + 3 * 2**-11, 0x3C02), (2**-24, 0x0001), (2**-26, 0x0000),
                 (-0.0, 0x8000), (float("inf"), 0x7C00)]:
        assert orc.float_to_half(x) == w, x


def test_float_to_half_vs_reference(orc, ref):
    """Agrees with the reference everywhere except where the reference drops
    the rounding carry (odd exponent, mantissa rounds up to 0x400)."""
    rng = np.random.default_rng(1)
    bits = (rng.integers(0, 2**23, 50000) | (rng.integers(100, 143, 50000) << 23)).astype(np.uint32)
    bits[:200] = (0x3FFFF000 + np.arange(200)).astype(np.uint32)   # just below 2.0
    for b in bits:
        x = float(np.uint32(b).view(np.float32))
        g, r = orc.float_to_half(x), ref.lib.ref_float_to_half(x)
        if g != r:
            # the only allowed difference: a carry into an odd exponent
            e = ((int(b) >> 23) & 0xFF) - 112
            assert e % 2 == 1 and g == r + 0x400 and (r & 0x3FF) == 0, (x, hex(g), hex(r))


def test_bf16(orc):
    for b in (0x0000, 0x3F80, 0xBF80, 0x7F80, 0x0001, 0x4049):
        want = np.array([b << 16], np.uint32).view(np.float32)[0]
        assert f32bits(orc.bf16_to_float(b)) == f32bits(want)


def blk(d16, payload):
    return np.frombuffer(struct.pack("<H", d16) + bytes(payload), np.uint8).copy()


def test_q4_0_known_answers(orc):
    # d = 1.0, byte j holds element 2j (low nibble) and 2j+1 (high nibble)
    payload = [(2 * j) % 16 | (((2 * j + 1) % 16) << 4) for j in range(16)]
    y = orc.dequant(blk(0x3C00, payload), P.Q4_0, 32)
    assert y.tolist() == [float((j % 16) - 8) for j in range(32)]
    assert np.all(orc.dequant(blk(0x0000, [0x88] * 16), P.Q4_0, 32) == 0)
    # d = -2.0: nibble 0 -> 16, nibble 15 -> -14
    y = orc.dequant(blk(0xC000, [0xF0] * 16), P.Q4_0, 32)
    assert y[0] == 16.0 and y[1] == -14.0
    # subnormal d = 2^-24: nibble 9 -> 2^-24
    y = orc.dequant(blk(0x0001, [0x99] * 16), P.Q4_0, 32)
    assert y[0] == 2.0 ** -24


def test_q8_0_known_answers(orc):
    q = [(j * 9 - 128) & 0xFF for j in range(32)]
    y = orc.dequant(blk(0x3800, q), P.Q8_0, 32)   # d = 0.5
    assert y.tolist() == [0.5 * float(np.int8(np.uint8(v))) for v in q]


def random_blocks(rng, dtype, nblocks):
    be, bb = P.BLOCK[dtype]
    raw = rng.integers(0, 256, nblocks * bb, dtype=np.uint8)
    # keep the fp16 fields finite and moderate: exponent byte in [0x20, 0x3F]
    hdr = {P.Q4_0: [0], P.Q8_0: [0], P.Q4_1: [0, 2], P.Q4_K: [0, 2], P.Q6_K: [208]}.get(dtype, [])
    for b in range(nblocks):
        for off in hdr:
            raw[b * bb + off + 1] = 0x20 + (raw[b * bb + off + 1] & 0x1F)
    if dtype in (P.F16,):
        raw[1::2] = 0x20 + (raw[1::2] & 0x1F)
    if dtype == P.F32:
        raw = rng.standard_normal(nblocks).astype(np.float32).view(np.uint8).copy()
    return raw


@pytest.mark.parametrize("dtype", [P.F32, P.F16, P.BF16, P.Q8_0, P.Q4_0, P.Q4_1])
def test_dequant_and_dot_match_reference(orc, ref, dtype):
    rng = np.random.default_rng(dtype)
    n = 4096 + 96 if dtype not in (P.F32, P.F16, P.BF16) else 3000
    be, bb = P.BLOCK[dtype]
    raw = random_blocks(rng, dtype, (n + be - 1) // be * (be if be == 1 else 1)) \
        if be == 1 else random_blocks(rng, dtype, (n + be - 1) // be)
    if be == 1:
        raw = raw[: n * bb] if raw.size >= n * bb else np.resize(raw, n * bb)
    a, b = orc.dequant(raw, dtype, n), ref.dequant(raw, dtype, n)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    x = rng.standard_normal(n).astype(np.float32)
    assert f32bits(orc.dot(x, raw, dtype, n)) == f32bits(ref.dot(x, raw, dtype, n))


def q4k_block(d16, m16, scales, qs):
    return np.frombuffer(struct.pack("<HH", d16, m16) + bytes(scales) + bytes(qs), np.uint8).copy()


def test_q4_k_known_answers(orc):
    # d = 1, dmin = 0.5; (sc, m) = (j + 1, 2j) for j < 4 and (j + 1, 2j) for j >= 4
    sc = [j + 1 for j in range(8)]
    mn = [2 * j for j in range(8)]
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] |= sc[j]
            s[j + 4] |= mn[j]
        else:
            s[j + 4] = (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    qs = [(l % 16) | ((15 - l % 16) << 4) for l in range(32)] * 4
    y = orc.dequant(q4k_block(0x3C00, 0x3800, s, qs), P.Q4_K, 256)
    # element 64g + l (low nibble, sub-block 2g) and 64g + 32 + l (high, 2g+1)
    assert y[0] == 1 * 0 - 0.0              # g=0 l=0: sc 1, q 0, m 0
    assert y[5] == 1 * 5 - 0.0              # sc 1, q 5
    assert y[32] == 2 * 15 - 0.5 * 2        # sub-block 1: sc 2, q 15, m 2
    assert y[64 + 3] == 3 * 3 - 0.5 * 4     # sub-block 2
    assert y[255] == 8 * (15 - 15) - 0.5 * 14   # sub-block 7, l = 31 -> q = 15-15


def test_q4_k_layout_probes(orc):
    rng = np.random.default_rng(7)
    base = random_blocks(rng, P.Q4_K, 1)
    y0 = orc.dequant(base, P.Q4_K, 256)
    for g in range(4):
        for l in (0, 17, 31):
            b = base.copy()
            b[16 + 32 * g + l] ^= 0x11          # flip one low and one high bit
            changed = np.nonzero(orc.dequant(b, P.Q4_K, 256) != y0)[0].tolist()
            assert set(changed) <= {64 * g + l, 64 * g + 32 + l}
    # scales byte j < 4 carries sub-block j's 6-bit scale (low bits)
    for j in range(4):
        b = base.copy()
        b[4 + j] ^= 0x01
        changed = set(np.nonzero(orc.dequant(b, P.Q4_K, 256) != y0)[0] // 32)
        assert changed <= {j}
    # high two bits of byte j < 4 belong to sub-block j + 4's scale
    for j in range(4):
        b = base.copy()
        b[4 + j] ^= 0x40
        changed = set(np.nonzero(orc.dequant(b, P.Q4_K, 256) != y0)[0] // 32)
        assert changed <= {j + 4}


def test_q6_k_known_answers(orc):
    ql = [0] * 128
    qh = [0] * 64
    # element 0: q6 = 63 (low nibble 15, high bits 3) -> 31; element 32: q6 = 0 -> -32
    ql[0] = 0x0F
    qh[0] = 0x03
    sc = [1] * 16
    sc[2] = -3
    raw = np.frombuffer(bytes(ql) + bytes(qh) + bytes([v & 0xFF for v in sc]) +
                        struct.pack("<H", 0x3C00), np.uint8).copy()
    y = orc.dequant(raw, P.Q6_K, 256)
    assert y[0] == 31.0            # sub-block 0, sc 1
    assert y[32] == -3.0 * -32     # element 32 is in sub-block 2 (sc -3)
    assert y[16] == -32.0          # sub-block 1, q6 0


def test_q6_k_layout_probes(orc):
    rng = np.random.default_rng(8)
    base = random_blocks(rng, P.Q6_K, 1)
    y0 = orc.dequant(base, P.Q6_K, 256)
    for c in range(2):
        for l in (0, 13, 31):
            b = base.copy()
            b[64 * c + l] ^= 0x11               # ql byte: elements k = 0 and 2
            ch = set(np.nonzero(orc.dequant(b, P.Q6_K, 256) != y0)[0].tolist())
            assert ch <= {128 * c + l, 128 * c + l + 64}
            b = base.copy()
            b[128 + 32 * c + l] ^= 0xFF         # qh byte: all four k
            ch = set(np.nonzero(orc.dequant(b, P.Q6_K, 256) != y0)[0].tolist())
            assert ch <= {128 * c + l + 32 * k for k in range(4)}
    for j in (0, 5, 15):
        b = base.copy()
        b[192 + j] ^= 0x01
        ch = set(np.nonzero(orc.dequant(b, P.Q6_K, 256) != y0)[0] // 16)
        assert ch <= {j}


@pytest.mark.parametrize("dtype,tol", [(P.Q8_0, 0.006), (P.Q4_0, 0.09), (P.Q4_K, 0.07),
                                       (P.Q6_K, 0.03), (P.F16, 0.0005), (P.Q4_1, 0.07)])
def test_quantise_roundtrip(orc, dtype, tol):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
    raw = orc.quantize(x, dtype)
    y = orc.dequant(raw, dtype, 1024, rows=8)
    err = np.abs(y - x).max() / np.abs(x).max()
    assert err < tol, err
    # reference test_quant style: dot against fp32 within a loose tolerance
    xs = rng.standard_normal(1024).astype(np.float32)
    rb = P.row_bytes(dtype, 1024)
    d = orc.dot(xs, raw[:rb], dtype, 1024)
    want = float(np.dot(xs.astype(np.float64), x[0].astype(np.float64)))
    assert abs(d - want) <= 0.35 * abs(want) + 5 * tol * np.abs(x[0]).sum() * 0.1
