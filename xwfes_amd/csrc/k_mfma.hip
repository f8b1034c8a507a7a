// k_mfma.hip -- int8-MFMA quantised GEMV for small M (M <= 8), row-dot form
// (y = x W^T with the quantisation blocks along the contraction), the
// layout of every verify-step projection except ffn_down.
//
// Math.  Activations are split per row m and 256-element block into two
// int8 limbs with a block scale s = max|x_block| / 127:  x ~= s*(a + b/256),
// |a|,|b| <= 127, so x is carried to ~1/65000 of its block maximum.  Weights
// enter the MFMA as their raw quantised integers, so every MFMA product and
// sum is exact integer arithmetic; the block scales are applied on the MFMA
// outputs:
//   Q4_K  w = d*sc_j*q - dmin*m_j  (q in 0..15, sub-block j of 32)
//     y = sum_sb s_sb * [ d * sum_j sc_j * (A_j . q_j) - dmin * sum_j m_j * X_j ]
//   where X_j is the sum of the activation limb over sub-block j, formed by
//   a second MFMA whose B operand is the eight m_j of the super-block.
// Shapes.  v_mfma_i32_32x32x32_i8: A rows 0..7 = limb a of m = 0..7, rows
// 8..15 = limb b, rows 16..31 zero; B columns = 32 weight rows; K = 32 = one
// Q4_K sub-block.  Lane l holds A[l%32][16*(l/32) + s], B[16*(l/32) + s][l%32]
// and C[8*(r/4) + 4*(l/32) + r%4][l%32] (checked on gfx950).
#include "ftx_internal.h"
#include "quant_dev.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i ld16g(const void* p) { return *(const v4i*)p; }

// ---------------------------------------------------------------- prep
// One wave per (256-element super-block sb, activation row m < 8); rows
// m >= M are written as zeros.  Optional RMSNorm (src/engine.cpp:23-41) in
// front: each wave reduces the sum of squares of its whole row (L2 hits).
// Lane l quantises elements 4l .. 4l+3 of the super-block.
__global__ void __launch_bounds__(64) k_xq_prep(const float* __restrict__ x, int64_t ldx,
                                                const float* __restrict__ normw, float eps,
                                                int64_t K, int M, int8_t* __restrict__ frag,
                                                int8_t* __restrict__ xs32,
                                                int8_t* __restrict__ xs16,
                                                float* __restrict__ scale) {
#pragma clang fp contract(off)
    const int64_t sb = blockIdx.x;
    const int m = blockIdx.y, l = threadIdx.x;
    const bool live = m < M;
    const float* row = x + (int64_t)m * ldx;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (live) {
        const float4 t = *(const float4*)(row + sb * 256 + 4 * l);
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
        if (normw) {
            float ss = 0.f;
            for (int64_t k = 4 * l; k < K; k += 256) {
                const float4 u = *(const float4*)(row + k);
                ss += u.x * u.x;
                ss += u.y * u.y;
                ss += u.z * u.z;
                ss += u.w * u.w;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            const float inv = 1.f / sqrtf(ss / (float)K + eps);
            const float4 w4 = *(const float4*)(normw + sb * 256 + 4 * l);
            v[0] = v[0] * inv * w4.x;
            v[1] = v[1] * inv * w4.y;
            v[2] = v[2] * inv * w4.z;
            v[3] = v[3] * inv * w4.w;
        }
    }
    float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float q = mx > 0.f ? 127.f / mx : 0.f;
    if (l == 0) scale[sb * 8 + m] = mx > 0.f ? mx / 127.f : 0.f;
    int sa = 0, sbb = 0;
    uint32_t pa = 0, pb = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float y = v[t] * q;
        const float a = rintf(y);
        float bf = rintf((y - a) * 256.f);
        bf = fminf(fmaxf(bf, -127.f), 127.f);
        const int ai = (int)a, bi = (int)bf;
        sa += ai;
        sbb += bi;
        pa |= (uint32_t)(ai & 0xFF) << (8 * t);
        pb |= (uint32_t)(bi & 0xFF) << (8 * t);
    }
    // fragment bytes: element 4l+t of the super-block sits in 32-block
    // kb = 8 sb + l/8, half (l%8)/4, byte 4(l%4) + t
    const int64_t kb = sb * 8 + (l >> 3);
    const int half = (l & 7) >> 2, byte = 4 * (l & 3);
    *(uint32_t*)(frag + ((kb * 2 + half) * 16 + m) * 16 + byte) = pa;
    *(uint32_t*)(frag + ((kb * 2 + half) * 16 + 8 + m) * 16 + byte) = pb;
    // 16-element sums (4 lanes), split into 6-bit lo / signed hi
#pragma unroll
    for (int o = 1; o < 4; o <<= 1) {
        sa += __shfl_xor(sa, o, 64);
        sbb += __shfl_xor(sbb, o, 64);
    }
    if ((l & 3) == 0) {
        const int s16 = l >> 2;
        xs16[(sb * 32 + m) * 16 + s16] = (int8_t)(sa & 63);
        xs16[(sb * 32 + 16 + m) * 16 + s16] = (int8_t)(sa >> 6);
        xs16[(sb * 32 + 8 + m) * 16 + s16] = (int8_t)(sbb & 63);
        xs16[(sb * 32 + 24 + m) * 16 + s16] = (int8_t)(sbb >> 6);
    }
    // 32-element sums (8 lanes)
    sa += __shfl_xor(sa, 4, 64);
    sbb += __shfl_xor(sbb, 4, 64);
    if ((l & 7) == 0) {
        const int j = l >> 3;
        xs32[(sb * 32 + m) * 8 + j] = (int8_t)(sa & 63);
        xs32[(sb * 32 + 16 + m) * 8 + j] = (int8_t)(sa >> 6);
        xs32[(sb * 32 + 8 + m) * 8 + j] = (int8_t)(sbb & 63);
        xs32[(sb * 32 + 24 + m) * 8 + j] = (int8_t)(sbb >> 6);
    }
}

// ---------------------------------------------------------------- Q4_K

struct MvSeg {
    const uint8_t* W;
    int64_t row_bytes;
    int64_t N;
    int64_t tile0;  // first global tile of the segment
    int64_t row0;   // first global row of the segment
    int dt;
};

struct MvArgs {
    MvSeg seg[3];
    int nseg;
    int64_t tiles;
    int64_t rows;       // global rows (sum of N)
    int sb_per_split;
    int nsb;            // super-blocks per row
    const int8_t* frag;
    const int8_t* xs32;
    const int8_t* xs16;
    const float* scale;
    float* part;        // [S][8][rows]
};

// Q6_K  w = d*sc_s*(q - 32)  (q in 0..63, sub-block s of 16)
//   y = sum_sb s_sb * d * [ sum_s sc_s * (A_s . q_s)  -  32 * sum_s sc_s * X_s ]
// with v_mfma_i32_32x32x16_i8 per sub-block (lane l holds 8 slots
// 8*(l/32) + t) and the second sum as one 32x32x32 MFMA whose B operand is
// the 16 int8 scales.
__global__ void __launch_bounds__(256) k_mv_q6k(MvArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t T = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (T >= a.tiles) return;
    int si = 0;
    while (si + 1 < a.nseg && T >= a.seg[si + 1].tile0) ++si;
    const MvSeg sg = a.seg[si];
    if (sg.dt != FTX_Q6_K) return;
    const int col = lane & 31, g = lane >> 5;
    const int64_t n_raw = (T - sg.tile0) * 32 + col;
    const int64_t n = n_raw < sg.N ? n_raw : sg.N - 1;
    const uint8_t* wrow = sg.W + n * sg.row_bytes;
    const int64_t nsb = a.nsb;
    const int sp = blockIdx.y;
    const int sb0 = sp * a.sb_per_split, sb1 = sb0 + a.sb_per_split;
    const bool arow = col < 16;
    float acc[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = 0.f;
    const v4i zero4 = {0, 0, 0, 0};
    const v16i zero16 = {};
    for (int sb = sb0; sb < sb1; ++sb) {
        v4i ql[4], qh[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) ql[i] = ld16g(wrow + (int64_t)sb * 128 + 64 * g + 16 * i);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            qh[i] = ld16g(wrow + nsb * 128 + (int64_t)sb * 64 + 32 * g + 16 * i);
        const v4i scv = ld16g(wrow + nsb * 192 + (int64_t)sb * 16);
        const float d = h2f(*(const uint16_t*)(wrow + nsb * 208 + (int64_t)sb * 2));
        const uint32_t* qlw = (const uint32_t*)ql;  // 16 dwords: [c][a][b][2]
        const uint32_t* qhw = (const uint32_t*)qh;  // 8 dwords: [c][b][2]
        const uint32_t* scw = (const uint32_t*)&scv;
        int ai[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) ai[r] = 0;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int c = s >> 3, k = (s & 7) >> 1, b = s & 1;
            long af = 0;
            if (arow)
                af = *(const long*)(a.frag +
                                    ((((int64_t)sb * 8 + (s >> 1)) * 2 + b) * 16 + col) * 16 +
                                    8 * g);
            uint32_t v[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t L = qlw[8 * c + 4 * (k & 1) + 2 * b + h];
                const uint32_t H = qhw[4 * c + 2 * b + h];
                const uint32_t lo = (k >> 1) ? (L >> 4) & 0x0F0F0F0Fu : L & 0x0F0F0F0Fu;
                const uint32_t hi = ((H >> (2 * k)) & 0x03030303u) << 4;
                v[h] = lo | hi;
            }
            const long bf = (long)((uint64_t)v[0] | ((uint64_t)v[1] << 32));
            const v16i cm = __builtin_amdgcn_mfma_i32_32x32x16_i8(af, bf, zero16, 0, 0, 0);
            const int sc = (int)(int8_t)((scw[s >> 2] >> (8 * (s & 3))) & 0xFF);
#pragma unroll
            for (int r = 0; r < 8; ++r) ai[r] += sc * cm[r];
            // keep at most two sub-blocks in flight (bounds the accumulators)
            if (s & 1) __builtin_amdgcn_sched_barrier(0);
        }
        v4i ax = zero4, bs = zero4;
        if (g == 0) {
            ax = ld16g(a.xs16 + ((int64_t)sb * 32 + col) * 16);
            bs = scv;
        }
        const v16i dm = __builtin_amdgcn_mfma_i32_32x32x32_i8(ax, bs, zero16, 0, 0, 0);
        const float4 s4 = *(const float4*)(a.scale + (int64_t)sb * 8 + 4 * g);
        const float sm[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int corr = dm[r] + 64 * dm[r + 8];
            acc[r] += sm[r & 3] * (d * (float)(ai[r] - 32 * corr));
        }
    }
    float* out = a.part + (int64_t)sp * 8 * a.rows + sg.row0;
    if (n_raw < sg.N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            out[(int64_t)m * a.rows + n_raw] = acc[r] + acc[r + 4] * (1.f / 256.f);
        }
    }
}

__global__ void __launch_bounds__(256) k_mv_q4k(MvArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t T = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (T >= a.tiles) return;
    int si = 0;
    while (si + 1 < a.nseg && T >= a.seg[si + 1].tile0) ++si;
    const MvSeg sg = a.seg[si];
    if (sg.dt != FTX_Q4_K) return;
    const int col = lane & 31, g = lane >> 5;
    const int64_t n_raw = (T - sg.tile0) * 32 + col;
    const int64_t n = n_raw < sg.N ? n_raw : sg.N - 1;
    const uint8_t* wrow = sg.W + n * sg.row_bytes;
    const int sp = blockIdx.y;
    const int sb0 = sp * a.sb_per_split, sb1 = sb0 + a.sb_per_split;
    const bool arow = col < 16;
    float acc[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = 0.f;
    const v4i zero4 = {0, 0, 0, 0};
    const v16i zero16 = {};
    for (int sb = sb0; sb < sb1; ++sb) {
        const uint8_t* blk = wrow + (int64_t)sb * 144;
        const v4i hdr = ld16g(blk);
        v4i qs[4];
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) qs[gg] = ld16g(blk + 16 + 32 * gg + 16 * g);
        v4i af[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            af[j] = arow ? ld16g(a.frag + ((((int64_t)sb * 8 + j) * 2 + g) * 16 + col) * 16)
                         : zero4;
        v4i ax = zero4;
        if (g == 0) {
            const int2 t = *(const int2*)(a.xs32 + ((int64_t)sb * 32 + col) * 8);
            ax.x = t.x;
            ax.y = t.y;
        }
        const uint32_t S0 = (uint32_t)hdr.y, S1 = (uint32_t)hdr.z, S2 = (uint32_t)hdr.w;
        const uint32_t sc_lo = S0 & 0x3F3F3F3Fu;
        const uint32_t mn_lo = S1 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
        int ai[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) ai[r] = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const v4i w = qs[j >> 1];
            v4i b;
            if (j & 1) {
                b.x = (int)(((uint32_t)w.x >> 4) & 0x0F0F0F0Fu);
                b.y = (int)(((uint32_t)w.y >> 4) & 0x0F0F0F0Fu);
                b.z = (int)(((uint32_t)w.z >> 4) & 0x0F0F0F0Fu);
                b.w = (int)(((uint32_t)w.w >> 4) & 0x0F0F0F0Fu);
            } else {
                b.x = (int)((uint32_t)w.x & 0x0F0F0F0Fu);
                b.y = (int)((uint32_t)w.y & 0x0F0F0F0Fu);
                b.z = (int)((uint32_t)w.z & 0x0F0F0F0Fu);
                b.w = (int)((uint32_t)w.w & 0x0F0F0F0Fu);
            }
            const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[j], b, zero16, 0, 0, 0);
            const int sc = (int)(((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3))) & 0xFF);
#pragma unroll
            for (int r = 0; r < 8; ++r) ai[r] += sc * c[r];
        }
        v4i bm = zero4;
        if (g == 0) {
            bm.x = (int)mn_lo;
            bm.y = (int)mn_hi;
        }
        const v16i dm = __builtin_amdgcn_mfma_i32_32x32x32_i8(ax, bm, zero16, 0, 0, 0);
        const float d = h2f((uint16_t)((uint32_t)hdr.x & 0xFFFF));
        const float dmin = h2f((uint16_t)((uint32_t)hdr.x >> 16));
        // activation scales of this super-block for m = 4g .. 4g+3
        const float4 s4 = *(const float4*)(a.scale + (int64_t)sb * 8 + 4 * g);
        const float sm[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int mins = dm[r] + 64 * dm[r + 8];
            acc[r] += sm[r & 3] * (d * (float)ai[r] - dmin * (float)mins);
        }
    }
    // rows 4g+r (limb a, r < 4) and 8+4g+r (limb b) of activation m = 4g + r
    float* out = a.part + (int64_t)sp * 8 * a.rows + sg.row0;
    if (n_raw < sg.N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            out[(int64_t)m * a.rows + n_raw] = acc[r] + acc[r + 4] * (1.f / 256.f);
        }
    }
}

// Sum the S split partials in order and apply the epilogue.
struct RedSeg {
    float* y;
    int64_t ldy;
    int64_t row0, N;
};
struct RedArgs {
    const float* part;
    int S;
    int64_t rows;
    int M;
    int epi;  // EPI_STORE, EPI_ACCUM, or 2 = SwiGLU (seg 0 gate, seg 1 up -> seg 0 y)
    RedSeg seg[3];
    int nseg;
};

__global__ void __launch_bounds__(256) k_mv_reduce(RedArgs a) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int m = blockIdx.y;
    if (m >= a.M) return;
    if (a.epi == 2) {
        const int64_t N = a.seg[0].N;
        if (t >= N) return;
        float g = 0.f, u = 0.f;
        for (int s = 0; s < a.S; ++s) {
            const float* p = a.part + ((int64_t)s * 8 + m) * a.rows;
            g += p[a.seg[0].row0 + t];
            u += p[a.seg[1].row0 + t];
        }
        // src/engine.cpp:271-273: g / (1 + exp(-g)) * u
        a.seg[0].y[(int64_t)m * a.seg[0].ldy + t] = g / (1.f + expf(-g)) * u;
        return;
    }
    if (t >= a.rows) return;
    int si = 0;
    while (si + 1 < a.nseg && t >= a.seg[si + 1].row0) ++si;
    float v = 0.f;
    for (int s = 0; s < a.S; ++s) v += a.part[((int64_t)s * 8 + m) * a.rows + t];
    float* yp = a.seg[si].y + (int64_t)m * a.seg[si].ldy + (t - a.seg[si].row0);
    *yp = a.epi == EPI_ACCUM ? *yp + v : v;
}

}  // namespace

// fragments K*16 | xs32 K | xs16 2K | scales (K/256)*8 floats
size_t xq_bytes(int64_t K) { return (size_t)(K * 16 + K + K * 2 + K / 8 + 64); }

hipError_t launch_xq_prep(hipStream_t st, const float* x, int64_t ldx, const float* normw,
                          float eps, int64_t K, int64_t M, int8_t* xq) {
    if (K % 4096 || K > 16384) return hipErrorInvalidValue;
    int8_t* frag = xq;
    int8_t* xs32 = xq + K * 16;
    int8_t* xs16 = xs32 + K;
    float* scale = (float*)(xs16 + K * 2);
    hipLaunchKernelGGL(k_xq_prep, dim3((unsigned)(K / 256), 8), dim3(64), 0, st, x, ldx, normw, eps,
                       K, (int)M, frag, xs32, xs16, scale);
    return hipGetLastError();
}

bool mv_supported(int dt, int64_t K, int64_t M) {
    return (dt == FTX_Q4_K || dt == FTX_Q6_K) && M >= 1 && M <= 8 && K % 4096 == 0 &&
           K <= 16384;
}

// y[m*ldy + n] += sum_s part[s][m][n] for n < N, m < M (part rows of 8)
hipError_t launch_part_reduce(hipStream_t st, const float* part, int S, int64_t N, int64_t M,
                              float* y, int64_t ldy) {
    RedArgs r{};
    r.part = part;
    r.S = S;
    r.rows = N;
    r.M = (int)M;
    r.epi = EPI_ACCUM;
    r.nseg = 1;
    r.seg[0] = RedSeg{y, ldy, 0, N};
    hipLaunchKernelGGL(k_mv_reduce, dim3((unsigned)((N + 255) / 256), (unsigned)M), dim3(256), 0,
                       st, r);
    return hipGetLastError();
}

// contraction splits: double until ~8 waves per CU or one super-block each
static int mv_splits(int64_t tiles, int nsb, int cu_count) {
    int S = 1;
    const int64_t want = (int64_t)(cu_count > 0 ? cu_count : 256) * 8;
    while (S < nsb && tiles * S < want && nsb % (S * 2) == 0) S *= 2;
    return S;
}

size_t mv_part_floats(int64_t rows, int64_t K, int cu_count) {
    const int64_t tiles = (rows + 31) / 32;
    return (size_t)mv_splits(tiles, (int)(K / 256), cu_count) * 8 * (size_t)rows;
}

// segs: up to 3 same-K Q4_K weight segments; epi as in RedArgs
hipError_t launch_mv(hipStream_t st, const GemvSeg* segs, int nseg, const int8_t* xq, int64_t K,
                     int64_t M, int epi, float* part, int cu_count) {
    MvArgs a{};
    a.nseg = nseg;
    int64_t tiles = 0, rows = 0;
    bool has4 = false, has6 = false;
    for (int i = 0; i < nseg; ++i) {
        a.seg[i].W = segs[i].W;
        a.seg[i].row_bytes = segs[i].row_bytes;
        a.seg[i].N = segs[i].N;
        a.seg[i].tile0 = tiles;
        a.seg[i].row0 = rows;
        a.seg[i].dt = segs[i].dt;
        has4 |= segs[i].dt == FTX_Q4_K;
        has6 |= segs[i].dt == FTX_Q6_K;
        tiles += (segs[i].N + 31) / 32;
        rows += segs[i].N;
    }
    a.tiles = tiles;
    a.rows = rows;
    const int nsb = (int)(K / 256);
    const int S = mv_splits(tiles, nsb, cu_count);
    a.sb_per_split = nsb / S;
    a.nsb = nsb;
    a.frag = xq;
    a.xs32 = xq + K * 16;
    a.xs16 = xq + K * 16 + K;
    a.scale = (const float*)(xq + K * 16 + K + K * 2);
    a.part = part;
    // each kernel takes the tiles of its dtype; both write disjoint rows
    const dim3 grid((unsigned)((tiles + 3) / 4), (unsigned)S);
    if (has4) hipLaunchKernelGGL(k_mv_q4k, grid, dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (has6) hipLaunchKernelGGL(k_mv_q6k, grid, dim3(256), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    RedArgs r{};
    r.part = part;
    r.S = S;
    r.rows = rows;
    r.M = (int)M;
    r.epi = epi;
    r.nseg = nseg;
    for (int i = 0; i < nseg; ++i) r.seg[i] = RedSeg{segs[i].y, segs[i].ldy, a.seg[i].row0, segs[i].N};
    const int64_t span = epi == 2 ? segs[0].N : rows;
    hipLaunchKernelGGL(k_mv_reduce, dim3((unsigned)((span + 255) / 256), (unsigned)M), dim3(256), 0,
                       st, r);
    return hipGetLastError();
}
