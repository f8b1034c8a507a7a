// quant_dev.h -- device-side GGUF block formats.
//
// dq8() returns 8 consecutive dequantised elements of a row, bit-exact with
// dequant_row (include/ft/quant.h:10-84) for the reference types and with the
// ggml Q4_K / Q6_K layouts under a fixed operation order:
//   Q4_K: y = (d*sc)*q - (dmin*m)      Q6_K: y = (d*sc)*(q6 - 32)
// Contraction is switched off inside these functions so that the rounding
// steps are the ones written.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ftx.h"

// Internal planar layouts of Q8_0 / Q4_0 rows (same bytes as the GGUF row,
// reordered): the row's fp16 scales first, then its quants, so that 8
// elements are one aligned 8-byte (Q8_0) or 4-byte (Q4_0) load when the
// row holds a multiple of 4 blocks.  Never seen outside the library.
constexpr int FTX_Q8_0_PLANAR = 108;
constexpr int FTX_Q4_0_PLANAR = 102;
// Q8_0 / Q4_0 re-tiled for the one-pass GEMM (k_gemm.hip): per 16-row tile
// and 256-element step, every lane's bytes of the step contiguous
constexpr int FTX_Q8_0_MMT = 118;
constexpr int FTX_Q4_0_MMT = 112;
constexpr int FTX_Q6_K_MMT = 114;  // from the planar Q6_K rows below

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ float bf2f(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

__device__ __forceinline__ uint16_t ld16(const uint8_t* p) {
    return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

// Q4_K 6-bit (scale, min) of sub-block j (ggml get_scale_min_k4 layout)
__device__ __forceinline__ void q4k_sc_m(int j, const uint8_t* s, int& sc, int& m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

__host__ __device__ constexpr int64_t blk_elems(int dt) {
    return (dt == FTX_Q4_0 || dt == FTX_Q4_1 || dt == FTX_Q8_0) ? 32
           : (dt == FTX_Q4_K || dt == FTX_Q6_K)                 ? 256
                                                                : 1;
}

__host__ __device__ constexpr int64_t blk_bytes(int dt) {
    return dt == FTX_F32    ? 4
           : dt == FTX_F16  ? 2
           : dt == FTX_BF16 ? 2
           : dt == FTX_Q4_0 ? 18
           : dt == FTX_Q4_1 ? 20
           : dt == FTX_Q8_0 ? 34
           : dt == FTX_Q4_K ? 144
           : dt == FTX_Q6_K ? 210
                            : 0;
}

// ---- Q6_K device layout ----
// GGUF Q6_K super-blocks are 210 bytes, so inside a row they sit at 2-byte
// alignment only.  On the device a Q6_K row is stored as planes, each
// 16-byte aligned, with the same bytes permuted:
//   QL plane  [nsb][128]: GGUF ql byte 64c + 32a + 16b + 8g + t  ->  64g + 32c + 16a + 8b + t
//   QH plane  [nsb][64] : GGUF qh byte 32c + 16b + 8g + t        ->  32g + 16c + 8b + t
//   SC plane  [nsb][16] : the 16 int8 sub-block scales
//   D  plane  [nsb][2]  : the fp16 super-block scale
// and the row padded to a multiple of 16 bytes.  g is the half of a
// 16-element sub-block an MFMA lane group reads, so each lane group's bytes
// are contiguous.
__host__ __device__ constexpr int64_t q6k_dev_row_bytes(int64_t ncols) {
    return ((ncols + 255) / 256 * 210 + 15) / 16 * 16;
}
__host__ __device__ inline int q6k_ql_dev(int i) {  // GGUF ql index -> plane index
    const int c = i >> 6, a = (i >> 5) & 1, b = (i >> 4) & 1, g = (i >> 3) & 1, t = i & 7;
    return 64 * g + 32 * c + 16 * a + 8 * b + t;
}
__host__ __device__ inline int q6k_qh_dev(int i) {
    const int c = i >> 5, b = (i >> 4) & 1, g = (i >> 3) & 1, t = i & 7;
    return 32 * g + 16 * c + 8 * b + t;
}

// Elements e0 .. e0+7 of `row` (e0 % 8 == 0); elements at or past n are 0.
__device__ inline void dq8(const uint8_t* __restrict__ row, int dt, int64_t e0, int64_t n,
                           float* __restrict__ o) {
#pragma clang fp contract(off)
    switch (dt) {
        case FTX_F32: {
            const float* r = (const float*)row;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                o[i] = 0.f;
                if (e0 + i < n) o[i] = r[e0 + i];
            }
            return;
        }
        case FTX_F16: {
            const uint16_t* r = (const uint16_t*)row;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                o[i] = 0.f;
                if (e0 + i < n) o[i] = h2f(r[e0 + i]);
            }
            return;
        }
        case FTX_BF16: {
            const uint16_t* r = (const uint16_t*)row;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                o[i] = 0.f;
                if (e0 + i < n) o[i] = bf2f(r[e0 + i]);
            }
            return;
        }
        case FTX_Q8_0: {
            const uint8_t* p = row + (e0 >> 5) * 34;
            const float d = h2f(ld16(p));
            const int j0 = (int)(e0 & 31);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                o[i] = e0 + i < n ? d * (float)(int8_t)p[2 + j0 + i] : 0.f;
            return;
        }
        case FTX_Q4_0: {
            const uint8_t* p = row + (e0 >> 5) * 18;
            const float d = h2f(ld16(p));
            const int j0 = (int)(e0 & 31);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int j = j0 + i;
                const uint8_t b = p[2 + (j >> 1)];
                const int nib = (j & 1) ? (b >> 4) : (b & 0xF);
                o[i] = e0 + i < n ? d * (float)(nib - 8) : 0.f;
            }
            return;
        }
        case FTX_Q8_0_PLANAR: {
            const float d = h2f(((const uint16_t*)row)[e0 >> 5]);
            const uint2 q = *(const uint2*)(row + 2 * (n >> 5) + e0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t wd = i < 4 ? q.x : q.y;
                o[i] = e0 + i < n ? d * (float)(int8_t)((wd >> (8 * (i & 3))) & 0xFF) : 0.f;
            }
            return;
        }
        case FTX_Q4_0_PLANAR: {
            const float d = h2f(((const uint16_t*)row)[e0 >> 5]);
            const uint32_t q = *(const uint32_t*)(row + 2 * (n >> 5) + (e0 >> 1));
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                // element j: nibble (j & 1) of byte j / 2 (reference order)
                const int nib = (int)((q >> (8 * (i >> 1) + 4 * (i & 1))) & 0xF);
                o[i] = e0 + i < n ? d * (float)(nib - 8) : 0.f;
            }
            return;
        }
        case FTX_Q4_1: {
            const uint8_t* p = row + (e0 >> 5) * 20;
            const float first = h2f(ld16(p));
            const float second = h2f(ld16(p + 2));
            const int j0 = (int)(e0 & 31);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int j = j0 + i;
                const uint8_t b = p[4 + (j >> 1)];
                const int nib = (j & 1) ? (b >> 4) : (b & 0xF);
                o[i] = e0 + i < n ? first + second * (float)nib : 0.f;
            }
            return;
        }
        case FTX_Q4_K: {
            const uint8_t* p = row + (e0 >> 8) * 144;
            const float d = h2f(ld16(p));
            const float dmin = h2f(ld16(p + 2));
            const int r = (int)(e0 & 255);
            const int j = r >> 5, l0 = r & 31, g = j >> 1;
            int sc, m;
            q4k_sc_m(j, p + 4, sc, m);
            const float ds = d * (float)sc;
            const float dm = dmin * (float)m;
            const uint8_t* qs = p + 16 + 32 * g + l0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int q = (j & 1) ? (qs[i] >> 4) : (qs[i] & 0xF);
                const float t = ds * (float)q;
                o[i] = e0 + i < n ? t - dm : 0.f;
            }
            return;
        }
        case FTX_Q6_K: {  // device planar layout (above)
            const int64_t nsb = (n + 255) / 256, sb = e0 >> 8;
            const int r = (int)(e0 & 255);
            const int c = r >> 7, rr = r & 127, k = rr >> 5, l0 = rr & 31;
            const float d = h2f(ld16(row + nsb * 208 + sb * 2));
            const float ds = d * (float)(int8_t)row[nsb * 192 + sb * 16 + (r >> 4)];
            // 8 consecutive l share (b, g): contiguous in both planes
            const uint8_t* ql = row + sb * 128 + q6k_ql_dev(64 * c + 32 * (k & 1) + l0);
            const uint8_t* qh = row + nsb * 128 + sb * 64 + q6k_qh_dev(32 * c + l0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int lo = (k >> 1) ? (ql[i] >> 4) : (ql[i] & 0xF);
                const int hi = (qh[i] >> (2 * k)) & 3;
                o[i] = e0 + i < n ? ds * (float)((lo | (hi << 4)) - 32) : 0.f;
            }
            return;
        }
        default:
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = 0.f;
            return;
    }
}
