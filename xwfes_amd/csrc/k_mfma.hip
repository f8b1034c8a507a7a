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
//   Q6_K  w = d*sc_s*(q - 32)  (q in 0..63, sub-block s of 16)
//     y = sum_sb s_sb * d * [ sum_s sc_s * (A_s . q_s)  -  32 * sum_s sc_s * X_s ]
// Shapes.  v_mfma_i32_32x32x32_i8: lane l holds A[l%32][16*(l/32) + s],
// B[16*(l/32) + s][l%32] and C[8*(r/4) + 4*(l/32) + r%4][l%32] (checked on
// gfx950).  B columns = 32 weight rows.  A rows 0..7 = limb a of m = 0..7,
// rows 8..15 = limb b.
//   Q4_K: K = 32 = one sub-block; A rows 16..31 only feed C rows 16..31,
//   which are never read, so those lanes load rows 0..15 again.
//   Q6_K: K = 32 = two sub-blocks 2p, 2p+1 made block-diagonal: A rows 0..15
//   carry sub-block 2p on the K slots of 2p and zeros elsewhere, rows 16..31
//   carry sub-block 2p+1, so C rows 0..15 and 16..31 are the two sub-block
//   dot products and every output register is used.
// Work split.  A workgroup owns one output unit (a tile of 16 or 32 weight
// rows; for SwiGLU a gate tile and its up tile) over the whole contraction,
// its W waves splitting the super-blocks into W contiguous ranges (W is
// chosen so the launch holds up to ~8 waves per CU).  Each wave walks its
// (super-block, tile) items with the next item's weights in flight during
// the current one's arithmetic.  With W > 1 the wave partials are added in
// wave order in LDS, so the result is deterministic; the epilogue (store,
// accumulate, or SwiGLU) follows.
#include "ftx_internal.h"
#include "quant_dev.h"
#include "xq_dev.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i ld16g(const void* p) { return *(const v4i*)p; }

// Materialise eight running sums here and fence the scheduler: keeps the
// compiler from re-associating a chain of integer multiply-adds into a tree
// that holds every MFMA result live at once, or from hoisting the operand
// unpacking of later sub-blocks (both spill).  Emits no instruction.
__device__ __forceinline__ void reg_fence8(int* v) {
#pragma unroll
    for (int r = 0; r < 8; ++r) asm volatile("" : "+v"(v[r]));
    __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------- prep
// One workgroup of 256 threads per (256-element super-block sb, activation
// row m < 8); rows m >= M are written as zeros.  Thread t forms element t:
//  - fold (part != null): x += sum_s part[s][m][.] over the S split
//    partials of the previous ffn_down, added in split order (loads issued
//    16 splits at a time), written back to x (the residual add of
//    src/engine.cpp:274-275);
// then wave 0 (lane l: elements 4l .. 4l+3, from LDS) applies
//  - RMSNorm (src/engine.cpp:23-41) when normw is given: the limbs of x * w
//    are formed with the block scale max|x * w| / 127 -- the limbs do not
//    depend on the row's 1 / rms factor, which the consuming GEMV applies
//    to the block scales from the per-block sums of x^2 stored in ssq[sb][m]
// and writes the limbs.
template <bool L16>
__global__ void __launch_bounds__(256) k_xq_prep(float* __restrict__ x, int64_t ldx,
                                                 const float* __restrict__ normw,
                                                 const float* __restrict__ part, int S,
                                                 int64_t ldpart, int64_t K, int M,
                                                 int8_t* __restrict__ frag,
                                                 int8_t* __restrict__ xs32,
                                                 int8_t* __restrict__ xs16,
                                                 float* __restrict__ scale,
                                                 float* __restrict__ ssq, int64_t cstride) {
#pragma clang fp contract(off)
    __shared__ float vs[256];
    const int64_t sb = blockIdx.x;
    // row m of 8-row chunk c: the chunk's operand lies cstride bytes after
    // the previous one's
    const int c = blockIdx.y >> 3, m = blockIdx.y & 7, t = threadIdx.x;
    const bool live = c * 8 + m < M;  // block-uniform
    float* row = x + (int64_t)(c * 8 + m) * ldx;
    frag += c * cstride;
    xs32 += c * cstride;
    xs16 += c * cstride;
    scale = (float*)((int8_t*)scale + c * cstride);
    ssq = (float*)((int8_t*)ssq + c * cstride);
    const int l = t & 63;
    const int64_t k0 = sb * 256 + 4 * l;
    // the norm weights of lane l's four elements are loaded first, so that
    // they arrive with x and the partials (one round trip, not two)
    float4 w4 = {1.f, 1.f, 1.f, 1.f};
    if (live && normw) w4 = *(const float4*)(normw + k0);
    const int64_t k = sb * 256 + t;
    float xv = 0.f;
    if (live) {
        xv = row[k];
        if (part) {
            float acc = 0.f;
            for (int s0 = 0; s0 < S; s0 += 16) {
                float p[16];
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    p[i] = s0 + i < S ? part[((int64_t)(s0 + i) * 8 + m) * ldpart + k] : 0.f;
#pragma unroll
                for (int i = 0; i < 16; ++i) acc += p[i];
            }
            xv += acc;
        }
        vs[t] = xv;
    }
    // every load has arrived on every path here (vmcnt 0, expcnt and lgkmcnt
    // untouched), which the compiler then knows at the join below
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    // every store after the barrier (which then waits for none) and after the
    // last use of a loaded value (so no wait for a load covers a store)
    if (t >= 64) {
        if (live && part) row[k] = xv;
        return;
    }
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
    if (live) {
        const float4 t4 = *(const float4*)&vs[4 * l];
        v[0] = t4.x;
        v[1] = t4.y;
        v[2] = t4.z;
        v[3] = t4.w;
        if (normw) {
            ss = v[0] * v[0];
            ss += v[1] * v[1];
            ss += v[2] * v[2];
            ss += v[3] * v[3];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            v[0] = v[0] * w4.x;
            v[1] = v[1] * w4.y;
            v[2] = v[2] * w4.z;
            v[3] = v[3] * w4.w;
        }
    }
    if (live && part) row[k] = xv;
    if (normw && l == 0) ssq[sb * 8 + m] = ss;
    if constexpr (L16)
        xq16_emit(v, sb, m, l, XqPtrs{frag, xs32, xs16, scale, ssq});
    else
        xq_emit(v, sb, m, l, XqPtrs{frag, xs32, xs16, scale, ssq});
}

// ---------------------------------------------------------------- row-dot

typedef unsigned v4u __attribute__((ext_vector_type(4)));

struct MvSeg {
    const uint8_t* W;
    int64_t row_bytes;
    int64_t N;
    int64_t tile0;  // first tile of the segment
    float* y;       // outputs [m][ldy]
    int64_t ldy;
    int rpt;        // weight rows per tile: 16 or 32
    int dt;
    int role;       // index of the caller's segment (EPI_QKV: 0 q, 1 k, 2 v)
};

struct MvArgs {
    MvSeg seg[3];
    int nseg;
    int64_t tiles;      // all tiles of the launch (SwiGLU: gate tiles then up tiles)
    int nsb;            // super-blocks per row (a multiple of 16)
    int M;
    int epi;            // EPI_STORE, EPI_ACCUM or EPI_SWIGLU (seg 0 gate, seg 1 up -> seg 0 y)
    const int8_t* frag;
    const int8_t* xs32;
    const int8_t* xs16;
    const float* scale;
    const float* ssq;   // per-block sums of x^2 [sb][8] when the input is RMS-normed, else null
    float eps;
    int64_t K;
    QkvEpi qkv;         // EPI_QKV: segments 0, 1, 2 are q, k, v
};

constexpr int MV_WAVES = 8;  // at most 8 waves per unit (512 threads)
// occupancy hint of the row-dot kernels: at least two waves per SIMD
constexpr int MV_WPE = 2;


__device__ __forceinline__ int mv_seg_of(const MvArgs& a, int64_t T) {
    int si = 0;
    while (si + 1 < a.nseg && T >= a.seg[si + 1].tile0) ++si;
    return si;
}

// one Q4_K super-block for weight row col of a tile: hdr = d, dmin, 12 scale bytes;
// qs[c] = bytes 32c + 16g .. +15 of the quants (sub-blocks 2c, 2c+1 in the
// low / high nibbles); af[j] = activation fragment of sub-block j; xv = the
// eight 32-element limb sums of activation row col (6-bit split rows).
__device__ __forceinline__ void q4k_block(const v4i hdr, const v4i* qs, const v4i* af, int2 xv,
                                          float4 s4, int g, float* acc) {
    const uint32_t S0 = (uint32_t)hdr.y, S1 = (uint32_t)hdr.z, S2 = (uint32_t)hdr.w;
    const uint32_t sc_lo = S0 & 0x3F3F3F3Fu;
    const uint32_t mn_lo = S1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
    const v16i zero16 = {};
    int ai[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) ai[r] = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const v4u w = __builtin_bit_cast(v4u, qs[j >> 1]);
        const v4u b = (j & 1) ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu;
        const v16i c =
            __builtin_amdgcn_mfma_i32_32x32x32_i8(af[j], __builtin_bit_cast(v4i, b), zero16, 0, 0, 0);
        const int sc = (int)(((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3))) & 0xFF);
#pragma unroll
        for (int r = 0; r < 8; ++r) ai[r] += __mul24(sc, c[r]);
        reg_fence8(ai);
    }
    const v4i ax = {xv.x, xv.y, 0, 0};
    const v4i bm = g == 0 ? v4i{(int)mn_lo, (int)mn_hi, 0, 0} : v4i{0, 0, 0, 0};
    const v16i dm = __builtin_amdgcn_mfma_i32_32x32x32_i8(ax, bm, zero16, 0, 0, 0);
    const float d = h2f((uint16_t)((uint32_t)hdr.x & 0xFFFF));
    const float dmin = h2f((uint16_t)((uint32_t)hdr.x >> 16));
    const float sm[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int mins = dm[r] + 64 * dm[r + 8];
        acc[r] += sm[r & 3] * (d * (float)ai[r] - dmin * (float)mins);
    }
}


// Q6_K quant word h (elements 8g + 4h .. +3) of sub-block s from the planar
// device layout: qlw = this lane's 64 low-nibble bytes [c][a][b][2 words],
// qhw = its 32 high-bit bytes [c][b][2 words]
__device__ __forceinline__ uint32_t q6k_word(const uint32_t* qlw, const uint32_t* qhw, int s,
                                             int h) {
    const int c = s >> 3, k = (s & 7) >> 1, b = s & 1;
    const uint32_t L = qlw[8 * c + 4 * (k & 1) + 2 * b + h];
    const uint32_t H = qhw[4 * c + 2 * b + h];
    const uint32_t lo = (k >> 1) ? (L >> 4) & 0x0F0F0F0Fu : L & 0x0F0F0F0Fu;
    const uint32_t hi = ((H >> (2 * k)) & 0x03030303u) << 4;
    return lo | hi;
}

// one Q6_K super-block: ql/qh as q6k_word, scv = the 16 int8 scales, x8[p] =
// 8 activation bytes of sub-block 2p + (col >= 16) (elements 8g .. 8g+7)
__device__ __forceinline__ void q6k_block(const v4i* ql, const v4i* qh, const v4i scv, float d,
                                          const long* x8, const v4i ax, float4 s4, int col, int g,
                                          float* acc) {
    const uint32_t* qlw = (const uint32_t*)ql;
    const uint32_t* qhw = (const uint32_t*)qh;
    const uint32_t* scw = (const uint32_t*)&scv;
    const v16i zero16 = {};
    const bool lower = col < 16;
    int ai[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) ai[r] = 0;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int s0 = 2 * p, s1 = 2 * p + 1;
        const v4i b = {(int)q6k_word(qlw, qhw, s0, 0), (int)q6k_word(qlw, qhw, s0, 1),
                       (int)q6k_word(qlw, qhw, s1, 0), (int)q6k_word(qlw, qhw, s1, 1)};
        const int xl = (int)(uint32_t)((uint64_t)x8[p]), xh = (int)(uint32_t)((uint64_t)x8[p] >> 32);
        const v4i af = lower ? v4i{xl, xh, 0, 0} : v4i{0, 0, xl, xh};
        const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, b, zero16, 0, 0, 0);
        const int sc0 = (int)(int8_t)((scw[s0 >> 2] >> (8 * (s0 & 3))) & 0xFF);
        const int sc1 = (int)(int8_t)((scw[s1 >> 2] >> (8 * (s1 & 3))) & 0xFF);
#pragma unroll
        for (int r = 0; r < 8; ++r) ai[r] += __mul24(sc0, c[r]) + __mul24(sc1, c[r + 8]);
        reg_fence8(ai);
    }
    const v4i bs = g == 0 ? scv : v4i{0, 0, 0, 0};
    const v16i dm = __builtin_amdgcn_mfma_i32_32x32x32_i8(ax, bs, zero16, 0, 0, 0);
    const float sm[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int corr = dm[r] + 64 * dm[r + 8];
        acc[r] += sm[r & 3] * (d * (float)(ai[r] - 32 * corr));
    }
}


// bytes per row and super-block
template <int DT>
constexpr int mv_bpr() { return DT == FTX_Q4_K ? 144 : 210; }

// weights of one (row, super-block): Q4_K hdr + 4 quant words, Q6_K 4 QL
// words, 2 QH words, scales and d
template <int DT>
struct MvW {
    v4i w[DT == FTX_Q4_K ? 5 : 7];
    uint16_t d;
};

// Byte offsets of a lane's chunks within one (tile, super-block).
// Row layout (GGUF Q4_K rows; the planar Q6_K device rows): `base` is the
// lane's weight row.  Tiled layout: `base` is the tile and the R-row block of
// a super-block is laid out so that every load is one contiguous run over the
// lanes (li = r + R*g, r = lane row within the tile):
//   Q4_K  QS [c 4][li 2R][16 B] | HDR [r R][16 B]                  (144 R B)
//   Q6_K  QL [i 4][li][16 B] | QH [i 2][li][16 B] | SC [r][16 B] | D [r][2 B]
//                                                                 (210 R B)
template <int DT, bool TILED>
__device__ __forceinline__ void mv_load(MvW<DT>& o, const uint8_t* base, int64_t nsb, int sb,
                                        int g, int r, int li, int R) {
    if constexpr (TILED) {
        const uint8_t* blk = base + (int64_t)sb * R * mv_bpr<DT>();
        if constexpr (DT == FTX_Q4_K) {
#pragma unroll
            for (int c = 0; c < 4; ++c) o.w[1 + c] = ld16g(blk + c * R * 32 + li * 16);
            o.w[0] = ld16g(blk + 4 * R * 32 + r * 16);
            o.d = 0;
        } else {
#pragma unroll
            for (int i = 0; i < 6; ++i) o.w[i] = ld16g(blk + i * R * 32 + li * 16);
            o.w[6] = ld16g(blk + 6 * R * 32 + r * 16);
            o.d = *(const uint16_t*)(blk + 6 * R * 32 + R * 16 + r * 2);
        }
    } else if constexpr (DT == FTX_Q4_K) {
        const uint8_t* blk = base + (int64_t)sb * 144;
        o.w[0] = ld16g(blk);
#pragma unroll
        for (int c = 0; c < 4; ++c) o.w[1 + c] = ld16g(blk + 16 + 32 * c + 16 * g);
        o.d = 0;
    } else {
        // planes: QL 128 B, QH 64 B, SC 16 B, D 2 B per super-block
#pragma unroll
        for (int i = 0; i < 4; ++i) o.w[i] = ld16g(base + (int64_t)sb * 128 + 64 * g + 16 * i);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            o.w[4 + i] = ld16g(base + nsb * 128 + (int64_t)sb * 64 + 32 * g + 16 * i);
        o.w[6] = ld16g(base + nsb * 192 + (int64_t)sb * 16);
        o.d = *(const uint16_t*)(base + nsb * 208 + (int64_t)sb * 2);
    }
}

// Re-tiling copy: thread (tile, super-block, li) moves its lane's chunks from
// the row layout to the tiled layout (rows past N repeat row N - 1).
template <int DT>
__global__ void __launch_bounds__(256) k_mv_tile(const uint8_t* __restrict__ src, int64_t rb,
                                                 int64_t N, int64_t nsb, int R, int64_t ntiles,
                                                 uint8_t* __restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per = nsb * 2 * R;
    if (t >= ntiles * per) return;
    const int64_t tl = t / per;
    const int sb = (int)((t % per) / (2 * R));
    const int li = (int)(t % (2 * R)), r = li % R, g = li / R;
    int64_t n = tl * R + r;
    if (n >= N) n = N - 1;
    MvW<DT> o;
    mv_load<DT, false>(o, src + n * rb, nsb, sb, g, r, li, R);
    uint8_t* blk = dst + (tl * nsb + sb) * R * mv_bpr<DT>();
    if constexpr (DT == FTX_Q4_K) {
#pragma unroll
        for (int c = 0; c < 4; ++c) *(v4i*)(blk + c * R * 32 + li * 16) = o.w[1 + c];
        if (g == 0) *(v4i*)(blk + 4 * R * 32 + r * 16) = o.w[0];
    } else {
#pragma unroll
        for (int i = 0; i < 6; ++i) *(v4i*)(blk + i * R * 32 + li * 16) = o.w[i];
        if (g == 0) {
            *(v4i*)(blk + 6 * R * 32 + r * 16) = o.w[6];
            *(uint16_t*)(blk + 6 * R * 32 + R * 16 + r * 2) = o.d;
        }
    }
}

// activation operand of one super-block for lane (col, g)
template <int DT>
struct MvX {
    v4i af[DT == FTX_Q4_K ? 8 : 1];
    long x8[DT == FTX_Q4_K ? 1 : 8];
    v4i ax;
    int2 xv;
    float4 s4;
};

template <int DT>
__device__ __forceinline__ void mv_load_x(MvX<DT>& x, const MvArgs& a, int sb, int col, int g) {
    if constexpr (DT == FTX_Q4_K) {
        const int8_t* fp = a.frag + (((int64_t)sb * 16 + g) * 16 + (col & 15)) * 16;
#pragma unroll
        for (int j = 0; j < 8; ++j) x.af[j] = ld16g(fp + 512 * j);
        x.xv = *(const int2*)(a.xs32 + ((int64_t)sb * 32 + col) * 8);
    } else {
        const int8_t* fp = a.frag + (int64_t)sb * 4096 + (col >> 4) * 256 + (col & 15) * 16 + 8 * g;
#pragma unroll
        for (int p = 0; p < 8; ++p) x.x8[p] = *(const long*)(fp + 512 * p);
        x.ax = ld16g(a.xs16 + ((int64_t)sb * 32 + col) * 16);
    }
    x.s4 = *(const float4*)(a.scale + (int64_t)sb * 8 + 4 * g);
}

// s4 = the block scales of rows 4g .. 4g+3 (times their RMSNorm factors)
template <int DT>
__device__ __forceinline__ void mv_block(const MvW<DT>& w, const MvX<DT>& x, float4 s4, int col,
                                         int g, float* acc) {
    if constexpr (DT == FTX_Q4_K)
        q4k_block(w.w[0], w.w + 1, x.af, x.xv, s4, g, acc);
    else
        q6k_block(w.w, w.w + 4, w.w[6], h2f(w.d), x.x8, x.ax, s4, col, g, acc);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// sum over the 16 lanes of each DPP row; every step adds a lane pair in
// both orders, so all 16 lanes end with the same bits
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_f<0x141>(v);  // row_half_mirror: lane i <-> 7 - i
    v += dpp_f<0x140>(v);  // row_mirror: lane i <-> 15 - i
    return v;
}

// items in flight ahead of the one being computed, within the register
// budget of each instantiation (Q6_K blocks are 1.5x Q4_K's); DEEP (single
// tiles, waves of a multiple of 4 super-blocks): three ahead, so that a
// 4-item wave has all its weights in flight at once
template <int DT, bool PAIR, bool DEEP>
constexpr int mv_depth() {
    if (DEEP) return 3;
    return DT == FTX_Q4_K ? 1 : (PAIR ? 0 : 1);
}

// grid = units; block = W waves (W divides the super-block count, W <= 8, so
// every wave takes an even number of super-blocks); at least 3 waves per
// SIMD fit (<= 168 VGPRs), 2 for the SwiGLU pairs, whose launches hold fewer
// waves per CU.
// Loads are issued so that no wait covers a later-needed, longer-latency
// load: the sums of squares first, then the first super-block's activation
// operand, then the first weights (vector-memory counters retire in issue
// order); the activation operand of super-block j + 1 is in flight while j
// computes, and the residual of the accumulate epilogue is read up front.
template <int DT, bool TILED, bool PAIR, bool DEEP>
__device__ __forceinline__ void mv_unit(const MvArgs& a, int64_t u) {
    __shared__ float part[PAIR ? 2 : 1][MV_WAVES][256];  // [tile of unit][wave][m * 32 + col]
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 31, g = lane >> 5;
    const int W = blockDim.x >> 6;
    constexpr bool pair = PAIR;
    constexpr int tpu = PAIR ? 2 : 1;
    const int64_t units = pair ? a.tiles / 2 : a.tiles;
    const int64_t nsb = a.nsb;
    const int spw = (int)(nsb / W), sb0 = w * spw;
    auto tile_of = [&](int ti) -> int64_t { return ti ? units + u : u; };
    auto load = [&](MvW<DT>& o, int ti, int sb) {
        const int64_t T = tile_of(ti);
        const MvSeg& sg = a.seg[mv_seg_of(a, T)];
        const int R = sg.rpt, r = col & (R - 1);
        const uint8_t* base;
        if constexpr (TILED) {
            base = sg.W + (T - sg.tile0) * nsb * R * mv_bpr<DT>();
        } else {
            int64_t n = (T - sg.tile0) * R + r;
            if (n >= sg.N) n = sg.N - 1;
            base = sg.W + n * sg.row_bytes;
        }
        mv_load<DT, TILED>(o, base, nsb, sb, g, r, r + R * g, R);
    };
    // items i = (super-block sb0 + i / tpu, tile i % tpu)
    const int nit = spw * tpu;
    float acc[tpu][8];
#pragma unroll
    for (int t = 0; t < tpu; ++t)
#pragma unroll
        for (int r = 0; r < 8; ++r) acc[t][r] = 0.f;
    // the weights of the next D items are in flight during an item's
    // arithmetic (a ring of D + 1 register buffers; loads past the last item
    // re-read it)
    constexpr int D = mv_depth<DT, PAIR, DEEP>();
    static_assert(D <= 1 || (D == 3 && !PAIR), "ring index: D + 1 must divide STEP * tpu");
    constexpr int STEP = D == 3 ? 4 : 2;  // super-blocks per unrolled step
    MvW<DT> buf[D + 1];
    auto item_load = [&](MvW<DT>& o, int j) {
        j = j < nit ? j : nit - 1;
        load(o, j % tpu, sb0 + j / tpu);
    };
    // lanes col and col ^ 16 each sum the super-blocks b = col % 16 + 16 k
    // of the per-block sums of squares (rows 4g .. 4g+3)
    float4 ss = {0.f, 0.f, 0.f, 0.f};
    if (a.ssq)
        for (int b = col & 15; b < a.nsb; b += 16) {
            const float4 t = *(const float4*)(a.ssq + (int64_t)b * 8 + 4 * g);
            ss.x += t.x;
            ss.y += t.y;
            ss.z += t.z;
            ss.w += t.w;
        }
    __builtin_amdgcn_sched_barrier(0);
    MvX<DT> x[DEEP ? 1 : 2];
    mv_load_x<DT>(x[0], a, sb0, col, g);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < D; ++d) item_load(buf[d], d);
    __builtin_amdgcn_sched_barrier(0);
    const int si = mv_seg_of(a, u);
    const MvSeg& sg = a.seg[si];
    const int rpt = sg.rpt;
    // the epilogue thread t < 8 * rpt owns output (m, c) = (t / rpt, t % rpt)
    // when W > 1: its residual (accumulate) or rotation (q / k) is read now
    const int t = threadIdx.x;
    const int em = t / rpt, ec = t % rpt;
    const int64_t en = (u - sg.tile0) * rpt + ec;
    const bool eown = W > 1 && t < 8 * rpt && em < a.M && en < sg.N;
    float eres = 0.f, ecs = 1.f, esn = 0.f;
    if (eown) {
        if (!pair && a.epi == EPI_ACCUM) eres = sg.y[(int64_t)em * sg.ldy + en];
        if (!pair && a.epi == EPI_QKV && sg.role < 2) {
            const int64_t d = en % a.qkv.hd;
            const float2 cs =
                *(const float2*)(a.qkv.cs + ((int64_t)em * (a.qkv.hd / 2) + d / 2) * 2);
            ecs = cs.x;
            esn = cs.y;
        }
    }
    // the RMSNorm factor 1 / rms of rows m = 4g .. 4g+3 (src/engine.cpp:23-41)
    float inv[4] = {1.f, 1.f, 1.f, 1.f};
    if (a.ssq) {
        const float kf = (float)a.K;
        inv[0] = 1.f / sqrtf(row16_sum(ss.x) / kf + a.eps);
        inv[1] = 1.f / sqrtf(row16_sum(ss.y) / kf + a.eps);
        inv[2] = 1.f / sqrtf(row16_sum(ss.z) / kf + a.eps);
        inv[3] = 1.f / sqrtf(row16_sum(ss.w) / kf + a.eps);
    }
    // STEP super-blocks per unrolled step: x[h % 2] holds super-block
    // sb0 + k + h; the item index i = (k + h) * tpu + ti keeps i % (D + 1) =
    // (h * tpu + ti) % (D + 1) because k is a multiple of STEP
    for (int k = 0; k < spw; k += STEP) {
#pragma unroll
        for (int h = 0; h < STEP; ++h) {
            // (DEEP: one activation buffer, loaded as its super-block starts --
            // the registers go to the weights, the longer-latency loads)
            constexpr int XB = DEEP ? 1 : 2;
            const int xc = h % XB;
            if (DEEP && k + h > 0) mv_load_x<DT>(x[0], a, sb0 + k + h, col, g);
            if (!DEEP && k + h + 1 < spw) mv_load_x<DT>(x[(h + 1) % XB], a, sb0 + k + h + 1, col, g);
            const float4 s4 = make_float4(x[xc].s4.x * inv[0], x[xc].s4.y * inv[1],
                                          x[xc].s4.z * inv[2], x[xc].s4.w * inv[3]);
#pragma unroll
            for (int ti = 0; ti < tpu; ++ti) {
                const int il = h * tpu + ti;
                const int i = k * tpu + il;
                __builtin_amdgcn_sched_barrier(0);
                item_load(buf[(il + D) % (D + 1)], i + D);
                __builtin_amdgcn_sched_barrier(0);
                mv_block<DT>(buf[il % (D + 1)], x[xc], s4, col, g, acc[ti]);
            }
        }
    }
    // lane (col, g) holds rows m = 4g + r of weight row col of each tile
    float v[tpu][4];
#pragma unroll
    for (int q = 0; q < tpu; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) v[q][r] = acc[q][r] + acc[q][r + 4] * (1.f / 256.f);
    if (W == 1) {
        // gv: this output; pv: the output of row n ^ 1 (the RoPE partner)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pv = __shfl_xor(v[0][r], 1, 64);
            const int m = 4 * g + r;
            const int64_t n = (u - sg.tile0) * rpt + col;
            if (col >= rpt || m >= a.M || n >= sg.N) continue;
            float* yp = sg.y + (int64_t)m * sg.ldy + n;
            const float gv = v[0][r];
            if (pair) {
                // src/engine.cpp:271-273: g / (1 + exp(-g)) * u
                *yp = gv / (1.f + expf(-gv)) * v[tpu - 1][r];
            } else if (a.epi == EPI_QKV) {
                float c = 1.f, sn = 0.f;
                if (sg.role < 2) {
                    const int64_t d = n % a.qkv.hd;
                    c = a.qkv.cs[((int64_t)m * (a.qkv.hd / 2) + d / 2) * 2];
                    sn = a.qkv.cs[((int64_t)m * (a.qkv.hd / 2) + d / 2) * 2 + 1];
                }
                qkv_store(a.qkv, sg.role, m, n, gv, pv, c, sn, yp);
            } else {
                *yp = a.epi == EPI_ACCUM ? *yp + gv : gv;
            }
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < tpu; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[q][w][(4 * g + r) * 32 + col] = v[q][r];
    __syncthreads();
    if (t < 8 * rpt) {
        float gv = 0.f, uv = 0.f;
        for (int ww = 0; ww < W; ++ww) gv += part[0][ww][em * 32 + ec];
        if constexpr (PAIR)
            for (int ww = 0; ww < W; ++ww) uv += part[tpu - 1][ww][em * 32 + ec];
        // threads t and t ^ 1 hold rows c and c ^ 1 (8 * rpt is whole waves)
        const float pv = __shfl_xor(gv, 1, 64);
        if (eown) {
            float* yp = sg.y + (int64_t)em * sg.ldy + en;
            if (pair)
                *yp = gv / (1.f + expf(-gv)) * uv;  // src/engine.cpp:271-273
            else if (a.epi == EPI_QKV)
                qkv_store(a.qkv, sg.role, em, en, gv, pv, ecs, esn, yp);
            else
                *yp = a.epi == EPI_ACCUM ? eres + gv : gv;
        }
    }
}

template <int DT, bool TILED, bool PAIR, bool DEEP>
__global__ void __launch_bounds__(64 * MV_WAVES) __attribute__((amdgpu_waves_per_eu(MV_WPE)))
k_mv(MvArgs a) {
    mv_unit<DT, TILED, PAIR, DEEP>(a, blockIdx.x);
}

// one launch over segments of both dtypes (q / k Q4_K with a Q6_K v): each
// workgroup takes the path of its unit's segment
template <bool TILED, bool DEEP>
__global__ void __launch_bounds__(64 * MV_WAVES) __attribute__((amdgpu_waves_per_eu(MV_WPE)))
k_mv_mix(MvArgs a) {
    const int64_t u = blockIdx.x;
    if (a.seg[mv_seg_of(a, u)].dt == FTX_Q4_K)
        mv_unit<FTX_Q4_K, TILED, false, DEEP>(a, u);
    else
        mv_unit<FTX_Q6_K, TILED, false, false>(a, u);  // deep Q6_K does not fit 256 VGPRs
}

// y[m*ldy + n] += sum_s part[s][m][n] in split order (ffn_down's splits)
__global__ void __launch_bounds__(256) k_part_reduce(const float* __restrict__ part, int S,
                                                     int64_t N, float* __restrict__ y,
                                                     int64_t ldy) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int m = blockIdx.y;
    if (t >= N) return;
    // rows past 8 read the partials of their own 8-row chunk, chunks S * 8 * N apart
    const float* pc = part + (int64_t)(m >> 3) * S * 8 * N;
    float v = 0.f;
#pragma unroll 8
    for (int s = 0; s < S; ++s) v += pc[((int64_t)s * 8 + (m & 7)) * N + t];
    y[(int64_t)m * ldy + t] += v;
}

}  // namespace

// fragments K*16 | xs32 K | xs16 2K | scales (K/256)*8 floats | ssq (K/256)*8 floats
size_t xq_bytes(int64_t K) { return (size_t)(K * 16 + K + K * 2 + K / 8 + K / 8 + 64); }
size_t xq_chunk_bytes(int64_t K) { return (xq_bytes(K) + 255) / 256 * 256; }

static float* xq_scale(int8_t* xq, int64_t K) { return xq_ptrs(xq, K).scale; }
static float* xq_ssq(int8_t* xq, int64_t K) { return xq_ptrs(xq, K).ssq; }

hipError_t launch_xq_prep(hipStream_t st, float* x, int64_t ldx, const float* normw,
                          const float* part, int S, int64_t ldpart, int64_t K, int64_t M,
                          int8_t* xq, int layout16) {
    if (K % 512 || K > 16384 || M < 1 || (part && M > 8)) return hipErrorInvalidValue;
    int8_t* frag = xq;
    int8_t* xs32 = xq + K * 16;
    int8_t* xs16 = xs32 + K;
    // one operand per 8-row chunk, xq_chunk_bytes(K) apart
    const int64_t chunks = (M + 7) / 8;
    hipLaunchKernelGGL(layout16 ? k_xq_prep<true> : k_xq_prep<false>,
                       dim3((unsigned)(K / 256), (unsigned)(8 * chunks)), dim3(256), 0, st, x, ldx,
                       normw, part, S, ldpart, K, (int)M, frag, xs32, xs16, xq_scale(xq, K),
                       xq_ssq(xq, K), (int64_t)xq_chunk_bytes(K));
    return hipGetLastError();
}

bool mv_swiglu_supported(int64_t K) { return K >= 256; }

bool mv_supported(int dt, int64_t K, int64_t M) {
    return (dt == FTX_Q4_K || dt == FTX_Q6_K) && M >= 1 && M <= 8 && K % 512 == 0 &&
           K <= 16384;
}

// y[m*ldy + n] += sum_s part[c][s][m % 8][n] for n < N, m < M, c = m / 8
// (the split partials of 8-row chunks, one after another)
hipError_t launch_part_reduce(hipStream_t st, const float* part, int S, int64_t N, int64_t M,
                              float* y, int64_t ldy) {
    hipLaunchKernelGGL(k_part_reduce, dim3((unsigned)((N + 255) / 256), (unsigned)M), dim3(256), 0,
                       st, part, S, N, y, ldy);
    return hipGetLastError();
}

int mv_tile_rows(int64_t N, int cu_count) {
    return (N + 31) / 32 < (cu_count > 0 ? cu_count : 256) ? 16 : 32;
}

size_t mv_tiled_bytes(int dt, int64_t N, int64_t K, int rpt) {
    const int64_t bpr = dt == FTX_Q4_K ? 144 : 210;
    return (size_t)((N + rpt - 1) / rpt * rpt) * (size_t)(K / 256) * (size_t)bpr;
}

hipError_t launch_mv_tile(hipStream_t st, const uint8_t* src, int64_t src_row_bytes, int dt,
                          int64_t N, int64_t K, int rpt, uint8_t* dst) {
    if ((dt != FTX_Q4_K && dt != FTX_Q6_K) || K % 256 || (rpt != 16 && rpt != 32) || N < 1)
        return hipErrorInvalidValue;
    const int64_t nsb = K / 256, ntiles = (N + rpt - 1) / rpt;
    const int64_t threads = ntiles * nsb * 2 * rpt;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (dt == FTX_Q4_K)
        hipLaunchKernelGGL(k_mv_tile<FTX_Q4_K>, grid, dim3(256), 0, st, src, src_row_bytes, N, nsb,
                           rpt, ntiles, dst);
    else
        hipLaunchKernelGGL(k_mv_tile<FTX_Q6_K>, grid, dim3(256), 0, st, src, src_row_bytes, N, nsb,
                           rpt, ntiles, dst);
    return hipGetLastError();
}

// segs: up to 3 same-K weight segments (Q4_K and / or Q6_K), all in the row
// layout or all tiled (GemvSeg::tiled, with the tile rows they were tiled
// with); one launch per dtype over that dtype's segments
hipError_t launch_mv(hipStream_t st, const GemvSeg* segs, int nseg, const int8_t* xq, int64_t K,
                     int64_t M, int epi, int cu_count, int normed, float eps,
                     const QkvEpi* qkv) {
    if (epi == EPI_QKV && (!qkv || nseg != 3 || qkv->hd % 2)) return hipErrorInvalidValue;
    if (nseg < 1 || nseg > 3 || M < 1 || M > 8 || K % 512 || K > 16384)
        return hipErrorInvalidValue;
    if (epi == EPI_SWIGLU && (nseg != 2 || segs[0].N != segs[1].N || segs[0].dt != segs[1].dt ||
                              segs[0].rpt != segs[1].rpt || !mv_swiglu_supported(K)))
        return hipErrorInvalidValue;
    const bool tiled = segs[0].tiled != 0;
    for (int i = 0; i < nseg; ++i)
        if ((segs[i].tiled != 0) != tiled || (tiled && segs[i].rpt != 16 && segs[i].rpt != 32))
            return hipErrorInvalidValue;
    const int cus = cu_count > 0 ? cu_count : 256;
    // mixed dtypes share one launch unless the units pair up for SwiGLU
    bool mixed = false;
    for (int i = 1; i < nseg; ++i) mixed |= segs[i].dt != segs[0].dt;
    const bool pair = epi == EPI_SWIGLU;
    for (int dt : {FTX_Q4_K, FTX_Q6_K}) {
        if (mixed && dt == FTX_Q6_K) break;  // the mixed launch took every segment
        MvArgs a{};
        int64_t tiles = 0;
        // a mixed launch puts the heavier Q6_K segments first, so that their
        // workgroups are dispatched first instead of finishing last
        int order[3];
        int no = 0;
        if (mixed) {
            for (int i = 0; i < nseg; ++i)
                if (segs[i].dt == FTX_Q6_K) order[no++] = i;
            for (int i = 0; i < nseg; ++i)
                if (segs[i].dt != FTX_Q6_K) order[no++] = i;
        } else {
            for (int i = 0; i < nseg; ++i) order[no++] = i;
        }
        for (int oi = 0; oi < no; ++oi) {
            const int i = order[oi];
            if (!mixed && segs[i].dt != dt) continue;
            MvSeg& sg = a.seg[a.nseg++];
            sg.role = i;
            sg.W = segs[i].W;
            sg.row_bytes = segs[i].row_bytes;
            sg.N = segs[i].N;
            sg.tile0 = tiles;
            sg.y = segs[i].y;
            sg.ldy = segs[i].ldy;
            sg.rpt = tiled ? segs[i].rpt : mv_tile_rows(segs[i].N, cus);
            sg.dt = segs[i].dt;
            tiles += (segs[i].N + sg.rpt - 1) / sg.rpt;
        }
        if (!a.nseg) continue;
        a.tiles = tiles;
        const int64_t units = pair ? tiles / 2 : tiles;
        a.nsb = (int)(K / 256);
        a.M = (int)M;
        a.epi = epi;
        a.frag = xq;
        a.xs32 = xq + K * 16;
        a.xs16 = xq + K * 16 + K;
        a.scale = xq_scale((int8_t*)xq, K);
        a.ssq = normed ? xq_ssq((int8_t*)xq, K) : nullptr;
        a.eps = eps;
        a.K = K;
        if (qkv) a.qkv = *qkv;
        // waves per unit: up to ~8 waves per CU over the launch (measured
        // best on the 8B shapes: gate/up W = 4, attention projections 8)
        // (every wave takes a multiple of two super-blocks: the unrolled
        // loop computes whole steps, so W doubles while 4 W divides nsb)
        int W = 1;
        while (W < MV_WAVES && a.nsb % (4 * W) == 0 && units * W * 2 <= (int64_t)cus * 8) W *= 2;
        // the W > 1 epilogue gives each of the 8 * rpt outputs of a tile its
        // own thread; where the block has fewer, one wave computes them all
        int maxr = 0;
        for (int i = 0; i < a.nseg; ++i) maxr = a.seg[i].rpt > maxr ? a.seg[i].rpt : maxr;
        if (W > 1 && 64 * W < 8 * maxr) W = 1;
        const dim3 gd((unsigned)units), bd(64 * W);
        // single Q4_K tiles whose waves take 4 super-blocks: every weight in
        // flight at once (Q6_K's larger blocks do not fit four deep)
        const bool deep = !pair && a.nsb / W == 4 && (mixed || dt == FTX_Q4_K);
        // instantiations: {Q4_K, Q6_K} x {row, tiled} x {single, SwiGLU pair, deep single}
        using K_t = void (*)(MvArgs);
        static const K_t kern[2][2][3] = {
            {{k_mv<FTX_Q4_K, false, false, false>, k_mv<FTX_Q4_K, false, true, false>,
              k_mv<FTX_Q4_K, false, false, true>},
             {k_mv<FTX_Q4_K, true, false, false>, k_mv<FTX_Q4_K, true, true, false>,
              k_mv<FTX_Q4_K, true, false, true>}},
            {{k_mv<FTX_Q6_K, false, false, false>, k_mv<FTX_Q6_K, false, true, false>,
              k_mv<FTX_Q6_K, false, false, false>},
             {k_mv<FTX_Q6_K, true, false, false>, k_mv<FTX_Q6_K, true, true, false>,
              k_mv<FTX_Q6_K, true, false, false>}}};
        static const K_t kmix[2][2] = {{k_mv_mix<false, false>, k_mv_mix<false, true>},
                                       {k_mv_mix<true, false>, k_mv_mix<true, true>}};
        const K_t kf = mixed ? kmix[tiled][deep]
                             : kern[dt == FTX_Q6_K][tiled][pair ? 1 : (deep ? 2 : 0)];
        ktimed_launch(kf, gd, bd, 0, st, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
