// k_quant.hip -- bit-exact block dequantisation (the export behind
// ftx_dequant) and the synthetic-model quantiser behind ftx_quantize.
#include "ftx_internal.h"
#include "quant_dev.h"

// One thread per 8 output elements; rows are independent.
__global__ void __launch_bounds__(256) k_dequant(const uint8_t* __restrict__ W, int dt,
                                                 int64_t row_bytes, int64_t ncols,
                                                 int64_t groups_per_row, int64_t total,
                                                 float* __restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int64_t r = t / groups_per_row;
    const int64_t e0 = (t % groups_per_row) * 8;
    float v[8];
    dq8(W + r * row_bytes, dt, e0, ncols, v);
    float* o = out + r * ncols + e0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (e0 + i < ncols) o[i] = v[i];
}

hipError_t launch_dequant(hipStream_t st, const uint8_t* W, int dt, int64_t row_bytes,
                          int64_t ncols, int64_t nrows, float* out) {
    const int64_t gpr = (ncols + 7) / 8;
    const int64_t total = gpr * nrows;
    if (total == 0) return hipSuccess;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)blocks), dim3(256), 0, st, W, dt, row_bytes,
                       ncols, gpr, total, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------- quantiser

__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ void st16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
__device__ __forceinline__ int clampi(int v, int lo, int hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

__device__ void q_q8_0(uint8_t* o, const float* x) {
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.f;
    const float id = d > 0.f ? 1.f / d : 0.f;
    st16(o, f2h(d));
    for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)(int8_t)clampi((int)rintf(x[j] * id), -127, 127);
}

// reference nibble order: element j is nibble j&1 of byte j/2
__device__ void q_q4_0(uint8_t* o, const float* x) {
    float amax = 0.f, vmax = 0.f;
    for (int j = 0; j < 32; ++j)
        if (fabsf(x[j]) > amax) {
            amax = fabsf(x[j]);
            vmax = x[j];
        }
    const float d = vmax / -8.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    st16(o, f2h(d));
    for (int j = 0; j < 16; ++j) {
        const int a = clampi((int)(x[2 * j] * id + 8.5f), 0, 15);
        const int b = clampi((int)(x[2 * j + 1] * id + 8.5f), 0, 15);
        o[2 + j] = (uint8_t)(a | (b << 4));
    }
}

__device__ void q_q4_1(uint8_t* o, const float* x) {
    float lo = x[0], hi = x[0];
    for (int j = 1; j < 32; ++j) {
        lo = fminf(lo, x[j]);
        hi = fmaxf(hi, x[j]);
    }
    const float s = (hi - lo) / 15.f;
    const float is = s > 0.f ? 1.f / s : 0.f;
    st16(o, f2h(lo));
    st16(o + 2, f2h(s));
    for (int j = 0; j < 16; ++j) {
        const int a = clampi((int)rintf((x[2 * j] - lo) * is), 0, 15);
        const int b = clampi((int)rintf((x[2 * j + 1] - lo) * is), 0, 15);
        o[4 + j] = (uint8_t)(a | (b << 4));
    }
}

// per 32-element sub-block an affine (scale, -min) fit coded as 6-bit
// multiples of the fp16 super-block d / dmin
__device__ void q_q4_k(uint8_t* o, const float* x) {
    float scale[8], mins[8];
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int l = 1; l < 32; ++l) {
            lo = fminf(lo, x[32 * j + l]);
            hi = fmaxf(hi, x[32 * j + l]);
        }
        if (lo > 0.f) lo = 0.f;
        scale[j] = (hi - lo) / 15.f;
        mins[j] = -lo;
    }
    float smax = 0.f, mmax = 0.f;
    for (int j = 0; j < 8; ++j) {
        smax = fmaxf(smax, scale[j]);
        mmax = fmaxf(mmax, mins[j]);
    }
    const uint16_t dh = f2h(smax / 63.f), mh = f2h(mmax / 63.f);
    const float d = h2f(dh), dmin = h2f(mh);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = (uint8_t)(d > 0.f ? clampi((int)rintf(scale[j] / d), 0, 63) : 0);
        mn[j] = (uint8_t)(dmin > 0.f ? clampi((int)rintf(mins[j] / dmin), 0, 63) : 0);
    }
    st16(o, dh);
    st16(o + 2, mh);
    uint8_t* s = o + 4;
    for (int j = 0; j < 12; ++j) s[j] = 0;
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
    uint8_t* qs = o + 16;
    for (int g = 0; g < 4; ++g) {
        const float ds0 = d * (float)sc[2 * g], dm0 = dmin * (float)mn[2 * g];
        const float ds1 = d * (float)sc[2 * g + 1], dm1 = dmin * (float)mn[2 * g + 1];
        for (int l = 0; l < 32; ++l) {
            const int a = ds0 > 0.f ? clampi((int)rintf((x[64 * g + l] + dm0) / ds0), 0, 15) : 0;
            const int b =
                ds1 > 0.f ? clampi((int)rintf((x[64 * g + 32 + l] + dm1) / ds1), 0, 15) : 0;
            qs[32 * g + l] = (uint8_t)(a | (b << 4));
        }
    }
}

// per 16-element sub-block a symmetric int8 multiple of the fp16 super-block d
__device__ void q_q6_k(uint8_t* o, const float* x) {
    float s[16], smax = 0.f, sabs = 0.f;
    for (int j = 0; j < 16; ++j) {
        float amax = 0.f, v = 0.f;
        for (int l = 0; l < 16; ++l)
            if (fabsf(x[16 * j + l]) > amax) {
                amax = fabsf(x[16 * j + l]);
                v = x[16 * j + l];
            }
        s[j] = v / -32.f;
        if (fabsf(s[j]) > sabs) {
            sabs = fabsf(s[j]);
            smax = s[j];
        }
    }
    const uint16_t dh = f2h(smax / -128.f);
    const float d = h2f(dh);
    int8_t sc[16];
    for (int j = 0; j < 16; ++j)
        sc[j] = (int8_t)(d != 0.f ? clampi((int)rintf(s[j] / d), -128, 127) : 0);
    uint8_t* ql = o;
    uint8_t* qh = o + 128;
    for (int c = 0; c < 2; ++c)
        for (int l = 0; l < 32; ++l) {
            uint8_t q[4];
            for (int k = 0; k < 4; ++k) {
                const int e = 128 * c + 32 * k + l;
                const float ds = d * (float)sc[e / 16];
                const int v = ds != 0.f ? clampi((int)rintf(x[e] / ds), -32, 31) : 0;
                q[k] = (uint8_t)(v + 32);
            }
            ql[64 * c + l] = (uint8_t)((q[0] & 0xF) | ((q[2] & 0xF) << 4));
            ql[64 * c + l + 32] = (uint8_t)((q[1] & 0xF) | ((q[3] & 0xF) << 4));
            qh[32 * c + l] = (uint8_t)((q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) |
                                       ((q[3] >> 4) << 6));
        }
    for (int j = 0; j < 16; ++j) o[192 + j] = (uint8_t)sc[j];
    st16(o + 208, dh);
}

// place one GGUF Q6_K block into the device planes of its row
__device__ void q6k_scatter(uint8_t* row, int64_t nsb, int64_t sb, const uint8_t* blk) {
    for (int i = 0; i < 128; ++i) row[sb * 128 + q6k_ql_dev(i)] = blk[i];
    for (int i = 0; i < 64; ++i) row[nsb * 128 + sb * 64 + q6k_qh_dev(i)] = blk[128 + i];
    for (int i = 0; i < 16; ++i) row[nsb * 192 + sb * 16 + i] = blk[192 + i];
    row[nsb * 208 + sb * 2] = blk[208];
    row[nsb * 208 + sb * 2 + 1] = blk[209];
}

// GGUF Q6_K rows -> device planar rows, one thread per block
__global__ void __launch_bounds__(256) k_q6k_repack(const uint8_t* __restrict__ src,
                                                    int64_t src_row_bytes, int64_t nsb,
                                                    int64_t total, int64_t dst_row_bytes,
                                                    uint8_t* __restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int64_t r = t / nsb, sb = t % nsb;
    uint8_t blk[210];
    const uint8_t* s = src + r * src_row_bytes + sb * 210;
    for (int i = 0; i < 210; ++i) blk[i] = s[i];
    q6k_scatter(dst + r * dst_row_bytes, nsb, sb, blk);
}

hipError_t launch_q6k_repack(hipStream_t st, const uint8_t* src, int64_t src_row_bytes,
                             int64_t ncols, int64_t nrows, int64_t dst_row_bytes, uint8_t* dst) {
    const int64_t nsb = (ncols + 255) / 256, total = nsb * nrows;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_q6k_repack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, src,
                       src_row_bytes, nsb, total, dst_row_bytes, dst);
    return hipGetLastError();
}

// one thread per block (per element for the plain types)
__global__ void __launch_bounds__(256) k_quantize(const float* __restrict__ src, int dt,
                                                  int64_t ncols, int64_t nblk_row,
                                                  int64_t total, int64_t row_bytes,
                                                  uint8_t* __restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int64_t r = t / nblk_row, b = t % nblk_row;
    const int64_t be = blk_elems(dt), bb = blk_bytes(dt);
    const float* x = src + r * ncols + b * be;
    uint8_t* o = dst + r * row_bytes + b * bb;
    switch (dt) {
        case FTX_F32: *(float*)o = x[0]; break;
        case FTX_F16: st16(o, f2h(x[0])); break;
        case FTX_BF16: {
            uint32_t u = __float_as_uint(x[0]);
            if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) u |= 0x400000u;
            else u += 0x7FFFu + ((u >> 16) & 1u);
            st16(o, (uint16_t)(u >> 16));
            break;
        }
        case FTX_Q8_0: q_q8_0(o, x); break;
        case FTX_Q4_0: q_q4_0(o, x); break;
        case FTX_Q4_1: q_q4_1(o, x); break;
        case FTX_Q4_K: q_q4_k(o, x); break;
        case FTX_Q6_K: {
            uint8_t blk[210];
            q_q6_k(blk, x);
            q6k_scatter(dst + r * row_bytes, nblk_row, b, blk);
            break;
        }
        default: break;
    }
}

hipError_t launch_quantize(hipStream_t st, const float* src, int dt, int64_t ncols,
                           int64_t nrows, int64_t row_bytes, uint8_t* dst) {
    const int64_t nb = ncols / blk_elems(dt);
    const int64_t total = nb * nrows;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, src,
                       dt, ncols, nb, total, row_bytes, dst);
    return hipGetLastError();
}

// ---------------------------------------------------------------- N(0, 1)
// Counter-based normal generator: two SplitMix64 outputs of (seed, i) give
// two uniforms, Box-Muller gives one normal.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void __launch_bounds__(256) k_fill_normal(void* __restrict__ dst, int f16, int64_t n,
                                                     uint64_t seed, float std) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t base = seed * 0x9E3779B97F4A7C15ull + (uint64_t)i * 2ull;
    const uint64_t a = mix64(base + 0x632BE59BD9B4E019ull), b = mix64(base + 0x8CB92BA72F3D8DD7ull);
    const float u1 = ((float)(a >> 40) + 0.5f) * (1.f / 16777216.f);
    const float u2 = (float)(b >> 40) * (1.f / 16777216.f);
    const float z = sqrtf(-2.f * logf(u1)) * cospif(2.f * u2);
    const float v = z * std;
    if (f16) ((_Float16*)dst)[i] = (_Float16)v;
    else ((float*)dst)[i] = v;
}

hipError_t launch_fill_normal(hipStream_t st, void* dst, int f16, int64_t n, uint64_t seed,
                              float std) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_normal, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dst,
                       f16, n, seed, std);
    return hipGetLastError();
}
