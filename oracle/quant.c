/*
 * quant.c -- scalar and block formats of the CPU oracle (test infrastructure;
 * see ftx_oracle.h).  Compiled with -ffp-contract=off so that the operation
 * order written here is the one executed: the HIP dequant export is checked
 * bit-exactly against these functions.
 */
#include "ftx_oracle.h"

#include <math.h>
#include <string.h>

/* IEEE half -> float by bit manipulation, subnormals normalised.
 * Follows include/ft/types.h:60-82. */
float orc_half_to_float(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            /* value = m * 2^-24; normalise so the leading one becomes the
             * implicit bit */
            int p = 9;
            while (!(m & (1u << p))) --p;
            bits = sign | ((uint32_t)(103 + p) << 23) |
                   ((m << (23 - p)) & 0x7FFFFFu);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* float -> IEEE half, round to nearest even; NaN becomes a quiet NaN with
 * the payload dropped, overflow becomes infinity.
 * Follows include/ft/types.h:84-110 except for one fix: the reference ORs
 * the rounded mantissa into the exponent field (types.h:109), so a round-up
 * that carries out of the mantissa is lost when the exponent is odd (e.g.
 * 1.99995f -> 1.0).  Here the carry is added, which is IEEE RNE.  The
 * reference only calls this from its test quantisers
 * (src/tests/test_core.cpp:250-279), never on the verify path. */
uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t fe = (x >> 23) & 0xFFu;
    uint32_t m = x & 0x7FFFFFu;
    if (fe == 0xFF) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
    int32_t e = (int32_t)fe - 112; /* re-biased exponent for half */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000u;
        int sh = 14 - e;
        uint32_t q = m >> sh;
        uint32_t r = m & ((1u << sh) - 1u);
        uint32_t halfway = 1u << (sh - 1);
        if (r > halfway || (r == halfway && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = m >> 13;
    uint32_t r = m & 0x1FFFu;
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) ++q; /* may carry into e */
    return (uint16_t)(sign | ((uint32_t)e << 10)) + (uint16_t)q;
}

/* include/ft/types.h:112-117 */
float orc_bf16_to_float(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* block geometry: include/ft/types.h:31-58 for the reference types; ggml
 * block_q4_K (144 B / 256) and block_q6_K (210 B / 256) for the K-quants */
int64_t orc_block_elems(int dt) {
    switch (dt) {
        case ORC_Q4_0: case ORC_Q4_1: case ORC_Q8_0: return 32;
        case ORC_Q4_K: case ORC_Q6_K: return 256;
        case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
        default: return 0;
    }
}

int64_t orc_block_bytes(int dt) {
    switch (dt) {
        case ORC_F32: return 4;
        case ORC_F16: case ORC_BF16: return 2;
        case ORC_Q4_0: return 18;
        case ORC_Q4_1: return 20;
        case ORC_Q8_0: return 34;
        case ORC_Q4_K: return 144;
        case ORC_Q6_K: return 210;
        default: return 0;
    }
}

int64_t orc_row_bytes(int dt, int64_t n) {
    int64_t be = orc_block_elems(dt);
    if (be == 0) return 0;
    return (n + be - 1) / be * orc_block_bytes(dt);
}

/* Q4_K 6-bit (scale, min) pair j of a super-block; ggml get_scale_min_k4 */
static void q4k_scale_min(int j, const uint8_t* s, uint8_t* sc, uint8_t* mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/*
 * Row dequantisation.  F32/F16/BF16/Q8_0/Q4_0/Q4_1 follow
 * include/ft/quant.h:10-84, including the reference's interleaved Q4_0
 * nibble order (element j is nibble j&1 of byte j/2) and its Q4_1 field
 * roles (first fp16 is added, second multiplies the nibble).
 * Q4_K / Q6_K follow the public ggml dequantize_row_q4_K / _q6_K layouts with
 * this fixed operation order (no contraction):
 *   Q4_K: y = (d*sc)*q - (dmin*m)
 *   Q6_K: y = (d*sc)*(q6 - 32)
 */
int orc_dequant_row(float* dst, const uint8_t* src, int dt, int64_t n) {
    switch (dt) {
        case ORC_F32:
            memcpy(dst, src, (size_t)n * 4);
            return 0;
        case ORC_F16:
            for (int64_t i = 0; i < n; ++i) dst[i] = orc_half_to_float(rd16(src + 2 * i));
            return 0;
        case ORC_BF16:
            for (int64_t i = 0; i < n; ++i) dst[i] = orc_bf16_to_float(rd16(src + 2 * i));
            return 0;
        case ORC_Q8_0:
            for (int64_t b = 0; b * 32 < n; ++b) {
                const uint8_t* p = src + b * 34;
                float d = orc_half_to_float(rd16(p));
                for (int64_t j = 0; j < 32 && b * 32 + j < n; ++j)
                    dst[b * 32 + j] = d * (float)(int8_t)p[2 + j];
            }
            return 0;
        case ORC_Q4_0:
            for (int64_t b = 0; b * 32 < n; ++b) {
                const uint8_t* p = src + b * 18;
                float d = orc_half_to_float(rd16(p));
                for (int64_t j = 0; j < 32 && b * 32 + j < n; ++j) {
                    uint8_t byte = p[2 + (j >> 1)];
                    int nib = (j & 1) ? (byte >> 4) : (byte & 0xF);
                    dst[b * 32 + j] = d * (float)(nib - 8);
                }
            }
            return 0;
        case ORC_Q4_1:
            for (int64_t b = 0; b * 32 < n; ++b) {
                const uint8_t* p = src + b * 20;
                float first = orc_half_to_float(rd16(p));
                float second = orc_half_to_float(rd16(p + 2));
                for (int64_t j = 0; j < 32 && b * 32 + j < n; ++j) {
                    uint8_t byte = p[4 + (j >> 1)];
                    int nib = (j & 1) ? (byte >> 4) : (byte & 0xF);
                    dst[b * 32 + j] = first + second * (float)nib;
                }
            }
            return 0;
        case ORC_Q4_K:
            for (int64_t b = 0; b * 256 < n; ++b) {
                const uint8_t* p = src + b * 144;
                float d = orc_half_to_float(rd16(p));
                float dmin = orc_half_to_float(rd16(p + 2));
                const uint8_t* sc = p + 4;
                const uint8_t* qs = p + 16;
                for (int g = 0; g < 4; ++g) {
                    uint8_t s0, m0, s1, m1;
                    q4k_scale_min(2 * g, sc, &s0, &m0);
                    q4k_scale_min(2 * g + 1, sc, &s1, &m1);
                    float d0 = d * (float)s0, n0 = dmin * (float)m0;
                    float d1 = d * (float)s1, n1 = dmin * (float)m1;
                    for (int l = 0; l < 32; ++l) {
                        int64_t e0 = b * 256 + 64 * g + l, e1 = e0 + 32;
                        float t0 = d0 * (float)(qs[32 * g + l] & 0xF);
                        float t1 = d1 * (float)(qs[32 * g + l] >> 4);
                        if (e0 < n) dst[e0] = t0 - n0;
                        if (e1 < n) dst[e1] = t1 - n1;
                    }
                }
            }
            return 0;
        case ORC_Q6_K:
            for (int64_t b = 0; b * 256 < n; ++b) {
                const uint8_t* p = src + b * 210;
                const uint8_t* ql = p;
                const uint8_t* qh = p + 128;
                const int8_t* sc = (const int8_t*)(p + 192);
                float d = orc_half_to_float(rd16(p + 208));
                for (int e = 0; e < 256; ++e) {
                    int c = e / 128, r = e % 128, l = r % 32, k = r / 32;
                    uint8_t lb = ql[64 * c + l + 32 * (k & 1)];
                    int lo = (k >> 1) ? (lb >> 4) : (lb & 0xF);
                    int hi = (qh[32 * c + l] >> (2 * k)) & 3;
                    int q = (lo | (hi << 4)) - 32;
                    float ds = d * (float)sc[e / 16];
                    if (b * 256 + e < n) dst[b * 256 + e] = ds * (float)q;
                }
            }
            return 0;
        default:
            return -1;
    }
}

/* x . dequant(w): fp32 sequential accumulation over dequantised chunks of
 * 2048 elements; include/ft/quant.h:86-103 */
float orc_dot_row_f32(const float* x, const uint8_t* w, int dt, int64_t n) {
    if (dt == ORC_F32) {
        const float* wf = (const float*)w;
        float acc = 0.f;
        for (int64_t i = 0; i < n; ++i) acc += x[i] * wf[i];
        return acc;
    }
    float buf[2048];
    float acc = 0.f;
    for (int64_t i = 0; i < n; i += 2048) {
        int64_t c = n - i < 2048 ? n - i : 2048;
        orc_dequant_row(buf, w + orc_row_bytes(dt, i), dt, c);
        for (int64_t j = 0; j < c; ++j) acc += x[i + j] * buf[j];
    }
    return acc;
}

/* ---------------- test-data quantisers ---------------- */

static int iround(float v) { return (int)lrintf(v); }
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void quant_q8_0(uint8_t* dst, const float* x) {
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    float d = amax / 127.f;
    float id = d > 0.f ? 1.f / d : 0.f;
    wr16(dst, orc_float_to_half(d));
    for (int j = 0; j < 32; ++j) dst[2 + j] = (uint8_t)(int8_t)clampi(iround(x[j] * id), -127, 127);
}

/* reference nibble order (include/ft/quant.h:54-57) */
static void quant_q4_0(uint8_t* dst, const float* x) {
    float amax = 0.f, vmax = 0.f;
    for (int j = 0; j < 32; ++j)
        if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); vmax = x[j]; }
    float d = vmax / -8.f;
    float id = d != 0.f ? 1.f / d : 0.f;
    wr16(dst, orc_float_to_half(d));
    memset(dst + 2, 0, 16);
    for (int j = 0; j < 32; ++j) {
        int q = clampi((int)(x[j] * id + 8.5f), 0, 15);
        dst[2 + j / 2] |= (uint8_t)(q << (4 * (j & 1)));
    }
}

static void quant_q4_1(uint8_t* dst, const float* x) {
    float lo = x[0], hi = x[0];
    for (int j = 1; j < 32; ++j) { lo = fminf(lo, x[j]); hi = fmaxf(hi, x[j]); }
    float s = (hi - lo) / 15.f;
    float is = s > 0.f ? 1.f / s : 0.f;
    wr16(dst, orc_float_to_half(lo));
    wr16(dst + 2, orc_float_to_half(s));
    memset(dst + 4, 0, 16);
    for (int j = 0; j < 32; ++j) {
        int q = clampi(iround((x[j] - lo) * is), 0, 15);
        dst[4 + j / 2] |= (uint8_t)(q << (4 * (j & 1)));
    }
}

/* Q4_K: per 32-element sub-block an affine (scale, -min) fit, both coded as
 * 6-bit multiples of the fp16 super-block d / dmin. */
static void quant_q4_k(uint8_t* dst, const float* x) {
    float scale[8], mins[8];
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int l = 1; l < 32; ++l) { lo = fminf(lo, x[32 * j + l]); hi = fmaxf(hi, x[32 * j + l]); }
        if (lo > 0.f) lo = 0.f;
        scale[j] = (hi - lo) / 15.f;
        mins[j] = -lo;
    }
    float smax = 0.f, mmax = 0.f;
    for (int j = 0; j < 8; ++j) { smax = fmaxf(smax, scale[j]); mmax = fmaxf(mmax, mins[j]); }
    uint16_t dh = orc_float_to_half(smax / 63.f), mh = orc_float_to_half(mmax / 63.f);
    float d = orc_half_to_float(dh), dmin = orc_half_to_float(mh);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = (uint8_t)(d > 0.f ? clampi(iround(scale[j] / d), 0, 63) : 0);
        mn[j] = (uint8_t)(dmin > 0.f ? clampi(iround(mins[j] / dmin), 0, 63) : 0);
    }
    wr16(dst, dh);
    wr16(dst + 2, mh);
    uint8_t* s = dst + 4;
    memset(s, 0, 12);
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            s[j] |= sc[j] & 63;
            s[j + 4] |= mn[j] & 63;
        } else {
            s[j + 4] = (uint8_t)((sc[j] & 0xF) | ((mn[j] & 0xF) << 4));
            s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
            s[j] |= (uint8_t)((mn[j] >> 4) << 6);
        }
    }
    uint8_t q[256];
    for (int j = 0; j < 8; ++j) {
        float ds = d * (float)sc[j], dm = dmin * (float)mn[j];
        for (int l = 0; l < 32; ++l)
            q[32 * j + l] = (uint8_t)(ds > 0.f ? clampi(iround((x[32 * j + l] + dm) / ds), 0, 15) : 0);
    }
    uint8_t* qs = dst + 16;
    for (int g = 0; g < 4; ++g)
        for (int l = 0; l < 32; ++l)
            qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
}

/* Q6_K: per 16-element sub-block a symmetric scale coded as an int8
 * multiple of the fp16 super-block d; values coded as q6 - 32. */
static void quant_q6_k(uint8_t* dst, const float* x) {
    float s[16], smax = 0.f, sabs = 0.f;
    for (int j = 0; j < 16; ++j) {
        float amax = 0.f, v = 0.f;
        for (int l = 0; l < 16; ++l)
            if (fabsf(x[16 * j + l]) > amax) { amax = fabsf(x[16 * j + l]); v = x[16 * j + l]; }
        s[j] = v / -32.f;
        if (fabsf(s[j]) > sabs) { sabs = fabsf(s[j]); smax = s[j]; }
    }
    uint16_t dh = orc_float_to_half(smax / -128.f);
    float d = orc_half_to_float(dh);
    int8_t sc[16];
    for (int j = 0; j < 16; ++j) sc[j] = (int8_t)(d != 0.f ? clampi(iround(s[j] / d), -128, 127) : 0);
    uint8_t q[256];
    for (int e = 0; e < 256; ++e) {
        float ds = d * (float)sc[e / 16];
        int v = ds != 0.f ? clampi(iround(x[e] / ds), -32, 31) : 0;
        q[e] = (uint8_t)(v + 32);
    }
    uint8_t* ql = dst;
    uint8_t* qh = dst + 128;
    memset(dst, 0, 210);
    for (int c = 0; c < 2; ++c)
        for (int l = 0; l < 32; ++l) {
            uint8_t q1 = q[128 * c + l], q2 = q[128 * c + l + 32];
            uint8_t q3 = q[128 * c + l + 64], q4 = q[128 * c + l + 96];
            ql[64 * c + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
            ql[64 * c + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
            qh[32 * c + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    memcpy(dst + 192, sc, 16);
    wr16(dst + 208, dh);
}

int orc_quantize_row(uint8_t* dst, const float* src, int dt, int64_t n) {
    int64_t be = orc_block_elems(dt), bb = orc_block_bytes(dt);
    if (be == 0) return -1;
    if (be > 1 && n % be) return -1;
    switch (dt) {
        case ORC_F32: memcpy(dst, src, (size_t)n * 4); return 0;
        case ORC_F16:
            for (int64_t i = 0; i < n; ++i) wr16(dst + 2 * i, orc_float_to_half(src[i]));
            return 0;
        case ORC_BF16:
            for (int64_t i = 0; i < n; ++i) {
                uint32_t u;
                memcpy(&u, &src[i], 4);
                if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) u |= 0x400000u;
                else u += 0x7FFFu + ((u >> 16) & 1u);
                wr16(dst + 2 * i, (uint16_t)(u >> 16));
            }
            return 0;
        default: break;
    }
    for (int64_t b = 0; b < n / be; ++b) {
        uint8_t* o = dst + b * bb;
        const float* x = src + b * be;
        switch (dt) {
            case ORC_Q8_0: quant_q8_0(o, x); break;
            case ORC_Q4_0: quant_q4_0(o, x); break;
            case ORC_Q4_1: quant_q4_1(o, x); break;
            case ORC_Q4_K: quant_q4_k(o, x); break;
            case ORC_Q6_K: quant_q6_k(o, x); break;
            default: return -1;
        }
    }
    return 0;
}
