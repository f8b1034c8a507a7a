// k_gemm.hip -- the verify step's projections for more than 8 tokens (draft
// trees, several sequences in one step): quantised GEMMs that stream each
// weight once per 64-token tile, on v_mfma_f32_16x16x32_f16.
//
// Operands.  The activations enter as fp16 hi + lo parts (x = hi + lo to
// ~22 bits; two MFMAs per product); the weights as exact small integers,
// with their block scales applied to fp32 accumulators:
//   Q4_K  w = d*sc_j*q - dmin*m_j   B = sc_j*q (<= 945, exact in fp16),
//         a super-block's 8 sub-blocks accumulate into a temporary that is
//         added with the factor d; the min term dmin * sum_j m_j X_j (X_j the
//         sub-block sums of the activations) is one 16x16x16 MFMA per
//         super-block on the m_j
//   Q8_0  w = d*q                   B = q, one temporary per 32-block
//   Q4_0  w = d*(q - 8)             B = q - 8, the same
//   Q6_K  w = d*sc_s*(q - 32)       sc_s = 16 sh + sl (sh in -8..7, sl in
//         0..15): B = sl (q - 32) (<= 480) and 16 sh (q - 32) (<= 4096, a
//         power-of-two multiple of an exact <= 256), both exact in fp16; a
//         super-block accumulates into a temporary added with the factor d
// so every product and sum inside an MFMA is exact and the rounding is that
// of fp32 accumulation.
//
// Row-dot form (y = x W^T, blocks along the contraction; every projection
// but ffn_down): a workgroup of 8 waves owns 256 weight rows (32 per wave,
// two 16-column MFMA tiles) and a 64-token tile (four 16-row MFMA tiles);
// the activation tile is staged in LDS 256 contraction elements at a time
// (double-buffered, one barrier per stage) and shared by the eight waves,
// which read their weights straight from the tiled (Q4_K) or planar (Q8_0,
// Q4_0) copies the model keeps.  Split-K across workgroups where the tiles
// alone do not fill the device; partial sums then go to a buffer that the
// reduce launch adds in split order with the epilogue (store, accumulate,
// SwiGLU).
//
// Column-axpy form (ffn_down in the reference orientation, n_ff rows of
// n_embd columns, Q4_K blocks along the output): per 32-row slice the
// workgroup (one 256-column block) stages h*d and h*dmin of its rows as
// hi/lo activation operands and the 6-bit scales / mins as fp16 tables; the
// weights (the re-tiled copy of k_down.hip) enter as sc*q.
#include "ftx_internal.h"
#include "mm_dev.h"
#include "quant_dev.h"

namespace {

constexpr int MM_TOK = 64;              // tokens per workgroup tile
constexpr int MM_MS = MM_TOK / 16;      // 16-token MFMA tiles
// 8 waves of 32 weight rows (two waves per SIMD, so that one wave's
// unpacking and LDS reads overlap the other's MFMAs; measured 12% faster
// than 4 waves of 64 rows on the 52-token gate / up shape)
constexpr int MM_WAVES = 8;  // waves per workgroup (256 weight rows)
constexpr int MM_WROWS = 256 / MM_WAVES;  // weight rows (output columns) per wave
constexpr int MM_NT = MM_WROWS / 16;    // 16-column MFMA tiles per wave

// the activation operands of ffn_down are formed as (h d) * 2^10 so that
// their fp16 lo parts stay clear of the subnormal range (undone on the
// outputs)
constexpr float MMD_ASCALE = 1024.f;

// ---------------------------------------------------------------- prep
// The activation operand in MFMA fragment order, so that a workgroup copies
// it to LDS with one direct global->LDS load per 1 KB and every lane reads
// its fragment from 16 contiguous bytes: for 16-token tile mt and 32-element
// K-step ks, fragment (mt, ks) is 64 lanes x 8 halves with lane l holding
// elements 8 (l / 16) .. + 7 of the step for token 16 mt + l % 16 (Q4_0
// consumers: each octet stored as its even then its odd elements, the order
// of that format's nibbles).  Planes: hi [Mp / 16][K / 32][64][8], lo the
// same; the 32-element sums of the token rows, for the Q4_K min term, as
// fragments of the 16x16x16 operand: [Mp / 16][K / 256][32 lanes][4] with
// lane l holding sub-blocks 4 (l / 16) .. + 3 of the super-block for token
// 16 mt + l % 16 (hi and lo planes).  frag_at and frag_sum_at (mm_dev.h)
// give the slots.

// Workgroup (token row m < Mp, 1024-element slice): rows m >= M are zeros.
// v = (x * inv) * w with inv = 1 / sqrt(sum x^2 / K + eps) when normw is
// given (src/engine.cpp:23-41; every slice's workgroup forms the row's sum
// itself), else v = x; v is split into fp16 hi + lo.  gather (expert
// launches): operand row m is row gather[m] of x, a zero row where
// gather[m] < 0.
__global__ void __launch_bounds__(256) k_mm_prep(const float* __restrict__ x, int64_t ldx,
                                                 const float* __restrict__ normw, float eps,
                                                 int64_t K, int M, int inter,
                                                 const int32_t* __restrict__ gather,
                                                 _Float16* __restrict__ xh,
                                                 _Float16* __restrict__ xl,
                                                 _Float16* __restrict__ sh,
                                                 _Float16* __restrict__ sl) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    const int m = blockIdx.x, t = threadIdx.x;
    const int64_t nsb = K / 256;
    const int64_t k0 = (int64_t)blockIdx.y * 1024, k1 = min(k0 + 1024, K);
    const int src = m >= M ? -1 : (gather ? gather[m] : m);
    const bool live = src >= 0;  // block-uniform
    const float* row = x + (int64_t)(live ? src : 0) * ldx;
    float inv = 1.f;
    if (live && normw) {
        float ss = 0.f;
        for (int64_t k = 4 * t; k < K; k += 1024) {
            const float4 v = *(const float4*)(row + k);
            ss += v.x * v.x;
            ss += v.y * v.y;
            ss += v.z * v.z;
            ss += v.w * v.w;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if ((t & 63) == 0) red[t >> 6] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
        inv = 1.f / sqrtf(ss / (float)K + eps);
    }
    for (int64_t k = k0 + 4 * t; k < k1; k += 1024) {
        float o[4] = {0.f, 0.f, 0.f, 0.f};
        if (live) {
            const float4 v = *(const float4*)(row + k);
            o[0] = v.x;
            o[1] = v.y;
            o[2] = v.z;
            o[3] = v.w;
            if (normw) {
                const float4 w = *(const float4*)(normw + k);
                o[0] = (o[0] * inv) * w.x;
                o[1] = (o[1] * inv) * w.y;
                o[2] = (o[2] * inv) * w.z;
                o[3] = (o[3] * inv) * w.w;
            }
        }
        _Float16 hv[4], lv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) split_hl(o[i], hv[i], lv[i]);
        if (!inter) {
            const int64_t at = frag_at(m, k, K, false);  // 4 consecutive slots
            *(v4h*)(xh + at) = v4h{hv[0], hv[1], hv[2], hv[3]};
            *(v4h*)(xl + at) = v4h{lv[0], lv[1], lv[2], lv[3]};
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t at = frag_at(m, k + i, K, true);
                xh[at] = hv[i];
                xl[at] = lv[i];
            }
        }
        // the 8 threads of a 32-element sub-block
        float s = (o[0] + o[1]) + (o[2] + o[3]);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        s += __shfl_xor(s, 4, 64);
        if ((t & 7) == 0) {
            const int64_t j = k / 32, sb = j / 8;
            const int jj = (int)(j % 8);
            const int lane = (m & 15) + 16 * (jj >> 2);
            const int64_t at = (((int64_t)(m >> 4) * nsb + sb) * 32 + lane) * 4 + (jj & 3);
            _Float16 h, l;
            split_hl(s, h, l);
            sh[at] = h;
            sl[at] = l;
        }
    }
}

// The prep of a whole operand row per workgroup of 1024 threads (thread t:
// elements 4 t + 4096 c, c < CH = K / 4096 rounded up), for K <= 16384.
// The source row is x row gather[m] (expert launches; a zero operand row
// where gather[m] < 0) or row m (rows m >= M: zero operands, x untouched).
// With S > 0 the split partials of the previous GEMM are added into it
// first: x[m] <- x[m] + sum_ks part[ks][m] (the sum in split order first,
// then added, as k_mm_reduce does; the residual add of
// src/engine.cpp:274-275 / 516-517), the new row written back as the
// workgroup's last step.  Then RMSNorm of the row (every element already
// in registers) and the fp16 hi + lo fragments and 32-element sums as
// k_mm_prep writes them.  The norm weights and the row are loaded at entry,
// ahead of the partials, and the one barrier (the row's sum of squares)
// has no store in flight to wait for.
constexpr int MMF_CH = 4;  // 4096-element chunks per row: K <= 16384
template <int CH>
__global__ void __launch_bounds__(1024) k_mm_prep_row(float* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ normw, float eps,
                                                      int64_t K, int M, int inter,
                                                      const int32_t* __restrict__ gather,
                                                      const float* __restrict__ part,
                                                      int64_t split_stride, int64_t ldp, int S,
                                                      _Float16* __restrict__ xh,
                                                      _Float16* __restrict__ xl,
                                                      _Float16* __restrict__ sh,
                                                      _Float16* __restrict__ sl) {
#pragma clang fp contract(off)
    // splits loaded together per chunk (the registers of CH x SB float4s)
    constexpr int SB = CH <= 2 ? 8 : CH == 3 ? 4 : 2;
    __shared__ float red[16];
    const int m = blockIdx.x, t = threadIdx.x;
    const int64_t nsb = K / 256;
    const int src = m >= M ? -1 : (gather ? gather[m] : m);
    const bool live = src >= 0;  // block-uniform
    float* row = x + (int64_t)(live ? src : 0) * ldx;
    // (without norm weights the row is read in their place: every load is
    // unconditional, the indices clamped to the row)
    const float* nwp = normw ? normw : row;
    float4 w[CH], v[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int64_t k = min((int64_t)(4 * t + 4096 * c), K - 4);
        w[c] = *(const float4*)(nwp + k);
        v[c] = *(const float4*)(row + k);
    }
    if (S > 0) {
        float4 g[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) g[c] = float4{0.f, 0.f, 0.f, 0.f};
        const float* pp = part + (int64_t)(live ? src : 0) * ldp;
        for (int s0 = 0; s0 < S; s0 += SB) {
            float4 pv[CH][SB];
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int64_t k = min((int64_t)(4 * t + 4096 * c), K - 4);
#pragma unroll
                for (int i = 0; i < SB; ++i)
                    pv[c][i] = s0 + i < S
                                   ? *(const float4*)(pp + k + (int64_t)(s0 + i) * split_stride)
                                   : float4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
                for (int i = 0; i < SB; ++i) {
                    g[c].x += pv[c][i].x;
                    g[c].y += pv[c][i].y;
                    g[c].z += pv[c][i].z;
                    g[c].w += pv[c][i].w;
                }
        }
#pragma unroll
        for (int c = 0; c < CH; ++c)
            v[c] = float4{v[c].x + g[c].x, v[c].y + g[c].y, v[c].z + g[c].z, v[c].w + g[c].w};
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        if (!live || 4 * t + 4096 * c >= K) {
            v[c] = float4{0.f, 0.f, 0.f, 0.f};
            continue;
        }
        ss += v[c].x * v[c].x;
        ss += v[c].y * v[c].y;
        ss += v[c].z * v[c].z;
        ss += v[c].w * v[c].w;
    }
    float inv = 1.f;
    if (normw) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if ((t & 63) == 0) red[t >> 6] = ss;
        __syncthreads();
        if (live) {
            float tot = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) tot += red[i];
            inv = 1.f / sqrtf(tot / (float)K + eps);
        }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int64_t k = 4 * t + 4096 * c;
        if (k >= K) continue;  // whole 32-element groups of 8 threads alike (K % 256 == 0)
        float o[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
        if (live && normw) {
            o[0] = (o[0] * inv) * w[c].x;
            o[1] = (o[1] * inv) * w[c].y;
            o[2] = (o[2] * inv) * w[c].z;
            o[3] = (o[3] * inv) * w[c].w;
        }
        _Float16 hv[4], lv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) split_hl(o[i], hv[i], lv[i]);
        if (!inter) {
            const int64_t at = frag_at(m, k, K, false);
            *(v4h*)(xh + at) = v4h{hv[0], hv[1], hv[2], hv[3]};
            *(v4h*)(xl + at) = v4h{lv[0], lv[1], lv[2], lv[3]};
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t at = frag_at(m, k + i, K, true);
                xh[at] = hv[i];
                xl[at] = lv[i];
            }
        }
        float s = (o[0] + o[1]) + (o[2] + o[3]);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        s += __shfl_xor(s, 4, 64);
        if ((t & 7) == 0) {
            const int64_t j = k / 32, sb = j / 8;
            const int jj = (int)(j % 8);
            const int lane = (m & 15) + 16 * (jj >> 2);
            const int64_t at = (((int64_t)(m >> 4) * nsb + sb) * 32 + lane) * 4 + (jj & 3);
            _Float16 h, l;
            split_hl(s, h, l);
            sh[at] = h;
            sl[at] = l;
        }
    }
    if (S > 0 && live) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int64_t k = 4 * t + 4096 * c;
            if (k < K) *(float4*)(row + k) = v[c];
        }
    }
}

// ---------------------------------------------------------------- row-dot

struct MmSegDev {
    const uint8_t* W;   // tiled (Q4_K) or planar (Q8_0 / Q4_0) copy
    int64_t N;          // weight rows
    int64_t unit0;      // first 64-row unit of the segment in the launch
    int64_t col0;       // first output column of the segment
    int64_t row_bytes;  // planar rows
    int rpt;            // Q4_K tile rows (16 or 32)
};

struct MmOutDev {
    // row m of the outputs: base[s] + (m - row0[s]) * ld + col for the
    // sequence s with row0[s] <= m < row0[s + 1]; a split ks adds
    // ks * split_stride
    float* base[FTX_MAX_SEQ];
    int64_t row0[FTX_MAX_SEQ + 1];
    int nseq;
    int64_t ld;
    int64_t split_stride;
    int accum;          // += instead of =
};

struct MmArgs {
    MmSegDev seg[3];
    int64_t plane[3];   // expert launches: bytes from one expert's plane to the next
    // expert launches (null otherwise): the tile table of the routing,
    // [0] = tiles in use, then per tile (expert, rows in use); tile t covers
    // operand rows 64 t .. 64 t + 63
    const int32_t* xtab;
    int nseg;
    int64_t units;      // 32-row units over all segments
    int ntt;            // token tiles: workgroup b takes token tile b % ntt of unit group b / ntt
    int64_t K;
    int nsb;            // 256-element steps of the contraction
    int sb_per_split;
    const _Float16 *xh, *xl, *sh, *sl;  // fragment-order operands (k_mm_prep)
    int M;
    MmOutDev out;
};

__device__ __forceinline__ int mm_seg_of(const MmArgs& a, int64_t u) {
    int si = 0;
    while (si + 1 < a.nseg && u >= a.seg[si + 1].unit0) ++si;
    return si;
}

// weights of one 256-element step for the wave's column tiles
template <int DT>
struct MmW;
template <>
struct MmW<FTX_Q4_K> {
    v2i qs[MM_NT][4];  // the lane's 8 quant bytes of each 64-element chunk
    v4i hdr[MM_NT];    // d | dmin, 12 scale bytes of the lane's row
};
template <>
struct MmW<FTX_Q8_0_MMT> {
    v4i q[MM_NT][4];   // 8 quant bytes of each 32-block, two blocks per vector
    v4i d[MM_NT];      // the 8 fp16 block scales
};
template <>
struct MmW<FTX_Q4_0_MMT> {
    v4i q[MM_NT][2];   // 4 quant bytes (8 nibbles) of each 32-block, four blocks per vector
    v4i d[MM_NT];
};
template <>
struct MmW<FTX_Q6_K_MMT> {
    v4i q[MM_NT][3];   // the lane's 32 ql bytes (4 runs of 8) and 16 qh bytes (2 runs of 8)
    v4i sc[MM_NT];     // its row's 16 int8 sub-block scales
    uint32_t d[MM_NT]; // its row's fp16 super-block scale
};

// the re-tiled Q8_0 / Q4_0 copy (k_mm_tile): per 16-row tile and 256-element
// step, [lane 64][bytes of the lane's 8 blocks] then [row 16][8 fp16 scales].
// Q6_K: [lane 64][48 bytes] then [row 16][16 int8 scales] then [row 16][fp16
// d]; lane (col, kq) of row 16 T + col holds ql bytes 64 h + 32 a + 8 kq ..
// + 7 as run 2 h + a (h, a = 0, 1) and qh bytes 32 h + 8 kq .. + 7 as run 4
// + h (GGUF super-block byte indices), i.e. elements 8 kq .. 8 kq + 7 of
// every 32-element step
__host__ __device__ constexpr int64_t mmt_lane_bytes(int dt) {
    return dt == FTX_Q8_0_MMT ? 64 : (dt == FTX_Q6_K_MMT ? 48 : 32);
}
__host__ __device__ constexpr int64_t mmt_step_bytes(int dt) {
    return 64 * mmt_lane_bytes(dt) + 16 * 16 + (dt == FTX_Q6_K_MMT ? 32 : 0);
}

// raw buffer descriptor over `p` (no range limit): loads then take a lane's
// 32-bit offset and a uniform offset, with no per-load address arithmetic
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mm_rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, -1, 0x00020000);
}

// The lane's weight offsets, computed once per wave: per column tile the
// tile's byte offset in the segment (uniform; a step adds a uniform stride)
// and the lane's 32-bit offsets in the tile: lane (col = l % 16, kq = l / 16)
// of MFMA column tile t holds B[8 kq + e][col] of each 32-element K-step,
// i.e. elements 8 kq .. 8 kq + 7 of its row.
struct MmPtr {
    __amdgpu_buffer_rsrc_t rs;   // the segment's weights (expert launches: the expert's plane)
    uint32_t tile[MM_NT];        // column tile t's weight tile (uniform)
    uint32_t lq[MM_NT];          // Q4_K: the lane's bytes of chunk 0; others: of the step
    uint32_t lh[MM_NT];          // Q4_K: its row's header; Q8_0 / Q4_0 / Q6_K: its row's scales
    uint32_t ld[MM_NT];          // Q6_K: its row's d
    uint32_t qstep;              // bytes per 256-element step
    uint32_t cstride;            // Q4_K: bytes from one 64-element chunk to the next
};

// Rows past N read the last tile's padding rows (the tiled copies hold whole
// tiles) and a tile wholly past N reads the last tile; their results are
// discarded.  Segments are below 4 GB.
template <int DT>
__device__ __forceinline__ void mm_ptrs(MmPtr& p, const MmSegDev& sg, int64_t rbase, int nsb,
                                        int col, int kq) {
    p.rs = mm_rsrc(sg.W);
#pragma unroll
    for (int t = 0; t < MM_NT; ++t) {
        if constexpr (DT == FTX_Q4_K) {
            // rbase is a multiple of 32: row rbase + 16 t + col is row
            // (16 t + col) % R of tile (rbase + 16 t) / R
            const int R = sg.rpt;
            const int64_t T = min((rbase + 16 * t) / R, (sg.N - 1) / R);
            const int r = (16 * t + col) % R, li = r + R * (kq >> 1), half = kq & 1;
            p.tile[t] = (uint32_t)(T * nsb * R * 144);
            p.lq[t] = (uint32_t)(li * 16 + 8 * half);
            p.lh[t] = (uint32_t)(4 * R * 32 + r * 16);
            p.ld[t] = 0;
        } else {
            const int64_t T = min((rbase + 16 * t) / 16, (sg.N - 1) / 16);
            p.tile[t] = (uint32_t)(T * nsb * mmt_step_bytes(DT));
            p.lq[t] = (uint32_t)((col + 16 * kq) * mmt_lane_bytes(DT));
            p.lh[t] = (uint32_t)(64 * mmt_lane_bytes(DT) + col * 16);
            p.ld[t] = (uint32_t)(64 * mmt_lane_bytes(DT) + 256 + col * 2);
        }
    }
    if constexpr (DT == FTX_Q4_K) {
        p.qstep = (uint32_t)(sg.rpt * 144);
        p.cstride = (uint32_t)(sg.rpt * 32);
    } else {
        p.qstep = (uint32_t)mmt_step_bytes(DT);
        p.cstride = 0;
    }
}

__device__ __forceinline__ v2i mm_ld8(const __amdgpu_buffer_rsrc_t& rs, uint32_t v, uint32_t s) {
    return __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rs, v, s, 0));
}
__device__ __forceinline__ v4i mm_ld16(const __amdgpu_buffer_rsrc_t& rs, uint32_t v, uint32_t s) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, v, s, 0));
}

template <int DT>
__device__ __forceinline__ void mm_load(MmW<DT>& o, const MmPtr& p, int sb) {
#pragma unroll
    for (int t = 0; t < MM_NT; ++t) {
        const uint32_t so = p.tile[t] + (uint32_t)sb * p.qstep;  // uniform
        if constexpr (DT == FTX_Q4_K) {
#pragma unroll
            for (int c = 0; c < 4; ++c) o.qs[t][c] = mm_ld8(p.rs, p.lq[t], so + c * p.cstride);
            o.hdr[t] = mm_ld16(p.rs, p.lh[t], so);
        } else if constexpr (DT == FTX_Q8_0_MMT) {
#pragma unroll
            for (int v = 0; v < 4; ++v) o.q[t][v] = mm_ld16(p.rs, p.lq[t], so + 16 * v);
            o.d[t] = mm_ld16(p.rs, p.lh[t], so);
        } else if constexpr (DT == FTX_Q6_K_MMT) {
#pragma unroll
            for (int v = 0; v < 3; ++v) o.q[t][v] = mm_ld16(p.rs, p.lq[t], so + 16 * v);
            o.sc[t] = mm_ld16(p.rs, p.lh[t], so);
            o.d[t] = __builtin_amdgcn_raw_buffer_load_b16(p.rs, p.ld[t], so, 0);
        } else {
#pragma unroll
            for (int v = 0; v < 2; ++v) o.q[t][v] = mm_ld16(p.rs, p.lq[t], so + 16 * v);
            o.d[t] = mm_ld16(p.rs, p.lh[t], so);
        }
    }
}

__device__ __forceinline__ float scale8(const v4i& d, int b) {
    const uint32_t w = (uint32_t)d[b >> 1];
    return h2f((uint16_t)((b & 1) ? (w >> 16) : (w & 0xFFFF)));
}

// four bytes (values < 2048) -> two fp16 pairs, exact
__device__ __forceinline__ void bytes4_h(uint32_t w, v2h& lo, v2h& hi) {
    const v2h o = {(_Float16)(-1024.f), (_Float16)(-1024.f)};
    lo = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(w, 0x64646464u, 0x00050004u)) + o;
    hi = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(w, 0x64646464u, 0x00070006u)) + o;
}

typedef __attribute__((address_space(3))) void lds_void;

// waves per SIMD the register allocation targets: two workgroups per CU for
// Q4_0 16-row tiles (they fit 128 registers), one otherwise (the larger
// weight register sets of Q8_0 and Q4_K would spill at 128)
template <int DT, int MS>
constexpr int MM_WPE = (MS == 1 && DT == FTX_Q4_0_MMT) ? 4 : 2;

// grid = (ceil(units / 8) x token tiles, 1, splits), workgroup b taking
// token tile b % ntt of unit group b / ntt; block = 512.  Per 256-element
// step the workgroup's activation fragments (MS 16-token tiles x 8 K-steps,
// hi and lo: 16 MS KB) are copied to one of two LDS buffers by direct loads,
// issued a whole step ahead together with the next step's weights (two
// register sets used in turn); one wait and one barrier per step.  Every
// wave takes part in the copies and barriers, and none branches around its
// MFMAs: a wave past the last unit computes on its clamped rows and stores
// nothing.
// XT (expert launches): the token tile index walks the routing's tile
// table; a tile past the tiles in use ends at once (the whole workgroup),
// the weights are the tile's expert's planes, and 16-token tiles past the
// tile's rows in use are neither copied nor multiplied (a block-uniform
// choice).  MS: 16-token MFMA tiles per workgroup tile (4 for 64-token
// tiles; 2 / 1 for dense launches of at most 32 / 16 tokens; 1 for the
// 16-row expert tiles of routings with few tokens per expert, whose 32 KB
// of LDS and smaller register set let several workgroups share a CU).
template <int DT, bool XT, int MS>
__global__ void __launch_bounds__(64 * MM_WAVES)
    __attribute__((amdgpu_waves_per_eu(MM_WPE<DT, MS>, MM_WPE<DT, MS>))) k_mm(MmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t mm_lds[];  // [2][MS * 16 KB]
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kq = lane >> 4;
    // the token tiles of one weight unit are logical neighbours on one XCD,
    // so they run together and a unit's weights come from memory about once
    const uint32_t lb = xcd_order(blockIdx.x + gridDim.x * blockIdx.z, gridDim.x * gridDim.z);
    const uint32_t bx = lb % gridDim.x;
    const int by = (int)(bx % (unsigned)a.ntt);
    const int64_t u = (int64_t)(bx / (unsigned)a.ntt) * MM_WAVES + w;
    const bool live = u < a.units;  // wave-uniform
    const int si = mm_seg_of(a, live ? u : a.units - 1);
    MmSegDev sg = a.seg[si];
    const int64_t rbase = ((live ? u : a.units - 1) - sg.unit0) * MM_WROWS;
    const int64_t mt0 = (int64_t)by * MS;  // first 16-token tile
    int nsub = MS, mend = a.M;  // 16-token tiles in use, rows in use end
    if constexpr (XT) {
        if (by >= a.xtab[0]) return;
        const int ex = a.xtab[1 + 2 * by], nv = a.xtab[2 + 2 * by];
        sg.W += (int64_t)ex * a.plane[si];
        nsub = (nv + 15) >> 4;
        mend = by * 16 * MS + nv;
    }
    const int ks = (int)(lb / gridDim.x);
    const int sb0 = ks * a.sb_per_split;
    const int sb1 = min(sb0 + a.sb_per_split, a.nsb);
    const int64_t nks = a.K / 32;
    MmPtr wp;
    mm_ptrs<DT>(wp, sg, rbase, a.nsb, col, kq);

    // the step's 16 MS fragments: block b = (hl, ms, j) = 8 (MS hl + ms) + j
    // -> LDS offset b KB; wave w copies blocks BPW w .. BPW w + BPW - 1 (one
    // (hl, ms) per wave: BPW divides 8)
    constexpr int BPW = 16 * MS / MM_WAVES;
    constexpr int BUF = MS * 16384;
    const int b0 = BPW * w, hl0 = b0 / (8 * MS), ms0 = (b0 / 8) % MS, j0 = b0 % 8;
    const __amdgpu_buffer_rsrc_t xrs = mm_rsrc(hl0 ? a.xl : a.xh);
    const uint32_t xoff = (uint32_t)((mt0 + ms0) * nks * 64 * 8 * 2);  // bytes, uniform
    const uint32_t glane = (uint32_t)lane * 16;
    auto stage = [&](int sb, int buf) {
        if (XT && ms0 >= nsub) return;  // this wave's blocks belong to an unused token tile
        const uint32_t so = xoff + (uint32_t)(sb * 8 + j0) * 1024;
#pragma unroll
        for (int i = 0; i < BPW; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xrs, (lds_void*)(mm_lds + buf * BUF + (b0 + i) * 1024), 16, glane, so + i * 1024, 0, 0);
    };
    auto frag = [&](int buf, int hl, int ms, int j) -> v8h {
        return *(const v8h*)(mm_lds + buf * BUF + ((hl * MS + ms) * 8 + j) * 1024 + lane * 16);
    };
    // Q4_K min term: this lane's sub-block sums (K slots of the 16x16x16
    // operand); lanes kq >= 2 read lane - 32's sums, which meet zero mins
    const __amdgpu_buffer_rsrc_t srs = mm_rsrc(a.sh), lrs = mm_rsrc(a.sl);
    const uint32_t soff = (uint32_t)(mt0 * a.nsb * 32 * 4 * 2);  // bytes, uniform
    const uint32_t xlane = (uint32_t)(lane & 31) * 8;

    v4f acc[MM_NT][MS];
#pragma unroll
    for (int t = 0; t < MM_NT; ++t)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) acc[t][ms] = v4f{0.f, 0.f, 0.f, 0.f};
    const v4f zero4 = {0.f, 0.f, 0.f, 0.f};

    // one 256-element step from LDS buffer `buf` with weights `wc`; the
    // next step's copies and weights (into `wn`) are issued first
    auto step = [&](int sb, int buf, const MmW<DT>& wc, MmW<DT>& wn) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // this step's fragments and weights
        __syncthreads();                     // every wave is done with the other buffer
        // Q4_K: the step's sub-block sums, loaded before the next step's
        // copies and weights so that their wait at the min term does not
        // wait for those
        v4h xsh[MS], xsl[MS];
        if constexpr (DT == FTX_Q4_K) {
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                if (XT && ms >= nsub) break;
                const uint32_t o = soff + (uint32_t)((ms * a.nsb + sb) * 32 * 4 * 2);
                xsh[ms] = __builtin_bit_cast(v4h, mm_ld8(srs, xlane, o));
                xsl[ms] = __builtin_bit_cast(v4h, mm_ld8(lrs, xlane, o));
            }
        }
        // the next step's copies and weights; the last step loads itself
        // again (unused), so that no branch leaves the waits for the sums
        // above counting as if these loads were not in flight
        {
            const int sbn = min(sb + 1, sb1 - 1);
            stage(sbn, buf ^ 1);
            mm_load<DT>(wn, wp, sbn);
        }
        // keep every load above ahead of the step's arithmetic (the
        // scheduler would otherwise sink the weight loads below the MFMAs
        // to save registers, and their latency would no longer be hidden)
        __builtin_amdgcn_sched_barrier(0);
        v2h scp[MM_NT][4], scn[MM_NT][4];  // Q4_K: sc and -1024 sc per sub-block, fp16 pairs
        v4h mnh[MM_NT];                    // Q4_K: the 4 mins of the lane's K slots
        if constexpr (DT == FTX_Q4_K) {
#pragma unroll
            for (int t = 0; t < MM_NT; ++t) {
                const uint32_t S0 = wc.hdr[t].y, S1 = wc.hdr[t].z, S2 = wc.hdr[t].w;
                const uint32_t sc0 = S0 & 0x3F3F3F3Fu;
                const uint32_t sc1 = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
                // the mins of the lane's K slots: sub-blocks 4 kq .. 4 kq + 3
                // (none for kq >= 2, whose slots are past the 8 sub-blocks)
                // (blended by masks: a branch here would wait for every load
                // in flight)
                const uint32_t odd = 0u - (uint32_t)(kq & 1), low = 0u - (uint32_t)(kq < 2);
                const uint32_t mhi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
                const uint32_t mn = ((mhi & odd) | (S1 & 0x3F3F3F3Fu & ~odd)) & low;
                v2h a0, a1;
                bytes4_h(sc0, scp[t][0], scp[t][1]);
                bytes4_h(sc1, scp[t][2], scp[t][3]);
                bytes4_h(mn, a0, a1);
                mnh[t] = v4h{a0[0], a0[1], a1[0], a1[1]};
#pragma unroll
                for (int i = 0; i < 4; ++i) scn[t][i] = scp[t][i] * v2h{(_Float16)(-1024.f), (_Float16)(-1024.f)};
            }
        }
        v4f tmp[MM_NT][MS];
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // 32-element K-step (sub-block / block) of the step
            // every fragment read of the K-step first, then the weight
            // operands, then the MFMAs
            v8h ah[MS], al[MS];
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                if (XT && ms >= nsub) break;
                ah[ms] = frag(buf, 0, ms, j);
                al[ms] = frag(buf, 1, ms, j);
            }
            v8h bw[MM_NT], bw2[MM_NT];
            float bs[MM_NT];
#pragma unroll
            for (int t = 0; t < MM_NT; ++t) {
                if constexpr (DT == FTX_Q4_K) {
                    // (1024 + q) * sc - 1024 sc = sc q, one rounding of an exact
                    // integer <= 945
                    const v2i wv = wc.qs[t][j >> 1];
                    const uint32_t x0 = (j & 1) ? ((uint32_t)wv.x >> 4) & 0x0F0F0F0Fu
                                                : (uint32_t)wv.x & 0x0F0F0F0Fu;
                    const uint32_t x1 = (j & 1) ? ((uint32_t)wv.y >> 4) & 0x0F0F0F0Fu
                                                : (uint32_t)wv.y & 0x0F0F0F0Fu;
                    const v2h sc = (j & 1) ? v2h{scp[t][j >> 1][1], scp[t][j >> 1][1]}
                                           : v2h{scp[t][j >> 1][0], scp[t][j >> 1][0]};
                    const v2h sn = (j & 1) ? v2h{scn[t][j >> 1][1], scn[t][j >> 1][1]}
                                           : v2h{scn[t][j >> 1][0], scn[t][j >> 1][0]};
                    v2h q[4];
                    q[0] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(x0, 0x64646464u, 0x00050004u));
                    q[1] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(x0, 0x64646464u, 0x00070006u));
                    q[2] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(x1, 0x64646464u, 0x00050004u));
                    q[3] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(x1, 0x64646464u, 0x00070006u));
#pragma unroll
                    for (int i = 0; i < 4; ++i) q[i] = __builtin_elementwise_fma(q[i], sc, sn);
                    bw[t] = v8h{q[0][0], q[0][1], q[1][0], q[1][1], q[2][0], q[2][1], q[3][0], q[3][1]};
                    bs[t] = 0.f;
                } else if constexpr (DT == FTX_Q8_0_MMT) {
                    const v4i qv = wc.q[t][j >> 1];
                    bw[t] = i8x8((j & 1) ? v2i{qv[2], qv[3]} : v2i{qv[0], qv[1]});
                    bs[t] = scale8(wc.d[t], j);
                } else if constexpr (DT == FTX_Q6_K_MMT) {
                    // elements 32 j + 8 kq .. + 7: half h, 32-group g of it;
                    // low nibbles from ql run 2 h + (g & 1) (high half of
                    // the byte for g >= 2), two high bits from qh run h
                    const int h = j >> 2, g = j & 3, run = 2 * h + (g & 1);
                    const v4i qv = wc.q[t][run >> 1], hv = wc.q[t][2];
                    const uint32_t w0 = (uint32_t)qv[2 * (run & 1)], w1 = (uint32_t)qv[2 * (run & 1) + 1];
                    const uint32_t h0 = (uint32_t)hv[2 * h], h1 = (uint32_t)hv[2 * h + 1];
                    const uint32_t b0 = ((w0 >> (4 * (g >> 1))) & 0x0F0F0F0Fu) |
                                        (((h0 >> (2 * g)) & 0x03030303u) << 4);
                    const uint32_t b1 = ((w1 >> (4 * (g >> 1))) & 0x0F0F0F0Fu) |
                                        (((h1 >> (2 * g)) & 0x03030303u) << 4);
                    // the scale of sub-block 2 j + kq / 2, split 16 sh + sl
                    const int sc = (int)(int8_t)(((uint32_t)wc.sc[t][j >> 1]) >>
                                                 (8 * (2 * (j & 1) + (kq >> 1))));
                    const int sl = sc & 15, sh = sc >> 4;
                    const _Float16 fl = (_Float16)(float)sl, fh = (_Float16)(float)sh;
                    const _Float16 ol = (_Float16)(float)(-1056 * sl), oh = (_Float16)(float)(-1056 * sh);
                    const v2h l1 = {fl, fl}, l0 = {ol, ol}, m1 = {fh, fh}, m0 = {oh, oh};
                    const v2h s16 = {(_Float16)16.f, (_Float16)16.f};
                    v2h q[4];
                    q[0] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(b0, 0x64646464u, 0x00050004u));
                    q[1] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(b0, 0x64646464u, 0x00070006u));
                    q[2] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(b1, 0x64646464u, 0x00050004u));
                    q[3] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(b1, 0x64646464u, 0x00070006u));
                    v2h r1[4], r2[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // (1024 + q) x - 1056 x = x (q - 32), exact
                        r1[i] = __builtin_elementwise_fma(q[i], l1, l0);
                        r2[i] = __builtin_elementwise_fma(q[i], m1, m0) * s16;
                    }
                    bw[t] = v8h{r1[0][0], r1[0][1], r1[1][0], r1[1][1], r1[2][0], r1[2][1], r1[3][0], r1[3][1]};
                    bw2[t] = v8h{r2[0][0], r2[0][1], r2[1][0], r2[1][1], r2[2][0], r2[2][1], r2[3][0], r2[3][1]};
                    bs[t] = 0.f;
                } else {
                    bw[t] = nib8((uint32_t)wc.q[t][j >> 2][j & 3], 8.f);
                    bs[t] = scale8(wc.d[t], j);
                }
            }
            if constexpr (DT == FTX_Q4_K || DT == FTX_Q6_K_MMT) {
                // hi parts of every tile first, then lo: no MFMA waits on the
                // one before it
#pragma unroll
                for (int t = 0; t < MM_NT; ++t)
#pragma unroll
                    for (int ms = 0; ms < MS; ++ms) {
                        if (XT && ms >= nsub) break;
                        tmp[t][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            ah[ms], bw[t], j == 0 ? zero4 : tmp[t][ms], 0, 0, 0);
                    }
#pragma unroll
                for (int t = 0; t < MM_NT; ++t)
#pragma unroll
                    for (int ms = 0; ms < MS; ++ms) {
                        if (XT && ms >= nsub) break;
                        tmp[t][ms] =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(al[ms], bw[t], tmp[t][ms], 0, 0, 0);
                    }
                if constexpr (DT == FTX_Q6_K_MMT) {
#pragma unroll
                    for (int t = 0; t < MM_NT; ++t)
#pragma unroll
                        for (int ms = 0; ms < MS; ++ms)
                            tmp[t][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ms], bw2[t],
                                                                                tmp[t][ms], 0, 0, 0);
#pragma unroll
                    for (int t = 0; t < MM_NT; ++t)
#pragma unroll
                        for (int ms = 0; ms < MS; ++ms)
                            tmp[t][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[ms], bw2[t],
                                                                                tmp[t][ms], 0, 0, 0);
                }
            } else {
                v4f p[MM_NT][MS];
#pragma unroll
                for (int t = 0; t < MM_NT; ++t)
#pragma unroll
                    for (int ms = 0; ms < MS; ++ms) {
                        if (XT && ms >= nsub) break;
                        p[t][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ms], bw[t], zero4, 0, 0, 0);
                    }
#pragma unroll
                for (int t = 0; t < MM_NT; ++t)
#pragma unroll
                    for (int ms = 0; ms < MS; ++ms) {
                        if (XT && ms >= nsub) break;
                        p[t][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[ms], bw[t], p[t][ms], 0, 0, 0);
                    }
#pragma unroll
                for (int t = 0; t < MM_NT; ++t)
#pragma unroll
                    for (int ms = 0; ms < MS; ++ms) {
                        if (XT && ms >= nsub) break;
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[t][ms][r] += bs[t] * p[t][ms][r];
                    }
            }
        }
        if constexpr (DT == FTX_Q6_K_MMT) {
#pragma unroll
            for (int t = 0; t < MM_NT; ++t) {
                const float d = h2f((uint16_t)wc.d[t]);
#pragma unroll
                for (int ms = 0; ms < MS; ++ms)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[t][ms][r] += d * tmp[t][ms][r];
            }
        }
        if constexpr (DT == FTX_Q4_K) {
            // acc += d * tmp - dmin * sum_j m_j X_j (the min term one 16x16x16
            // MFMA on the sub-block sums and the mins)
#pragma unroll
            for (int t = 0; t < MM_NT; ++t) {
                const float d = h2f((uint16_t)((uint32_t)wc.hdr[t].x & 0xFFFF));
                const float dmin = h2f((uint16_t)((uint32_t)wc.hdr[t].x >> 16));
#pragma unroll
                for (int ms = 0; ms < MS; ++ms) {
                    if (XT && ms >= nsub) break;
                    v4f mt = __builtin_amdgcn_mfma_f32_16x16x16f16(xsh[ms], mnh[t], zero4, 0, 0, 0);
                    mt = __builtin_amdgcn_mfma_f32_16x16x16f16(xsl[ms], mnh[t], mt, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[t][ms][r] = fmaf(-dmin, mt[r], fmaf(d, tmp[t][ms][r], acc[t][ms][r]));
                }
            }
        }
    };
    MmW<DT> wa, wb;
    if (sb0 < sb1) {
        stage(sb0, 0);
        mm_load<DT>(wa, wp, sb0);
    }
    // two weight register sets used in turn (no copy between steps)
    for (int sb = sb0; sb < sb1; sb += 2) {
        step(sb, 0, wa, wb);
        if (sb + 1 >= sb1) break;
        step(sb + 1, 1, wb, wa);
    }
    if (!live) return;
    // lane (col, kq) holds C[4 kq + r][col] of each tile: token 16 (mt0 + ms)
    // + 4 kq + r, output column col0 + rbase + 16 t + col
    const MmOutDev& o = a.out;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = 16 * (mt0 + ms) + 4 * kq + r;
            if (m >= mend) continue;
            int s = 0;
            while (s + 1 < o.nseq && m >= o.row0[s + 1]) ++s;
            float* yrow = o.base[s] + (m - o.row0[s]) * o.ld + (int64_t)ks * o.split_stride;
#pragma unroll
            for (int t = 0; t < MM_NT; ++t) {
                const int64_t n = rbase + 16 * t + col;
                if (n >= sg.N) continue;
                float* yp = yrow + sg.col0 + n;
                *yp = o.accum ? *yp + acc[t][ms][r] : acc[t][ms][r];
            }
        }
}

// ---------------------------------------------------------------- ffn_down

struct MmDownArgs {
    const uint8_t* qs;   // QS plane of the re-tiled copy
    const uint8_t* hdr;  // headers [N / 256][n_in] x 16 B
    const float* h;      // [M][ldh]
    int64_t ldh;
    int M;
    int64_t n_in, N;
    int slices_per_split;
    int ntt;             // token tiles (grid x = column blocks x token tiles)
    MmOutDev out;
};

// grid = (N / 256 x token tiles, 1, splits); block = 512: wave w owns
// columns 256 bx + 32 w .. + 31 (two 16-column tiles ct, all in sub-block w
// of the block) for all of the workgroup's 16 MS tokens (64, or 32 for
// launches of at most 32 tokens), so that each weight operand is built once
// and feeds 4 MS MFMAs; per 32-row slice the workgroup stages, for its
// tokens, A_d = h d 2^10 and A_m = h dmin 2^10 (hi / lo) and the fp16 tables
// of the block's 8 sub-block scales (also as -1024 sc) and 8 mins, one table
// entry per thread; y = (sum_i A_d sc q - sum_i A_m mn) / 2^10 with the min
// term (one 16-column MFMA tile whose columns are the sub-blocks) done by
// wave w < MS for tokens 16 w .. 16 w + 15 and handed to the other waves
// through LDS.
constexpr int MMD_PITCH = 32 + 8;
constexpr int MMD_WAVES = 8;  // two per SIMD
constexpr int MMD_RING = 4;  // slices whose global operands are in flight (even: LDS buffer = slice parity)

// 8 nibbles (slot t: byte t % 4, nibble t / 4) -> fp16 sc_t q_t, exact:
// (1024 + q) sc + (-1024 sc) in one fused multiply-add per pair
__device__ __forceinline__ v8h nib8_sc(uint32_t w, const v8h& sc, const v8h& sn) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    v2h p[4];
    p[0] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(lo, 0x64646464u, 0x00050004u));
    p[1] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(lo, 0x64646464u, 0x00070006u));
    p[2] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(hi, 0x64646464u, 0x00050004u));
    p[3] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(hi, 0x64646464u, 0x00070006u));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        p[i] = __builtin_elementwise_fma(p[i], v2h{sc[2 * i], sc[2 * i + 1]},
                                         v2h{sn[2 * i], sn[2 * i + 1]});
    return v8h{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

// MS: 16-token tiles of a workgroup (4: 64 tokens; 2: launches of at most
// 32 tokens); a thread stages RPT = MS rows of one token
template <int MS>
__global__ void __launch_bounds__(64 * MMD_WAVES) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_mm_down(MmDownArgs a) {
    constexpr int TOK = 16 * MS, RPT = MS, TPR = 32 / RPT;  // tokens, rows per thread, threads per token
    __shared__ _Float16 ad[2][2][TOK][MMD_PITCH];  // [buf][hi / lo][token][row i]
    __shared__ _Float16 am[2][2][TOK][MMD_PITCH];
    __shared__ _Float16 tsm[2][16][MMD_PITCH];         // [buf][sc of sub-block 0-7, mn 0-7][row i]
    __shared__ _Float16 tsn[2][16][MMD_PITCH];         // [buf][-1024 sc (rows 8-15 unused)][row i]
    __shared__ float mins[TOK][9];                     // [token][sub-block]
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kq = lane >> 4;
    // token tiles of one column block are logical neighbours on one XCD
    // (they share the block's weights)
    const uint32_t lb = xcd_order(blockIdx.x + gridDim.x * blockIdx.z, gridDim.x * gridDim.z);
    const uint32_t bx = lb % gridDim.x;
    const int64_t jb = bx / (unsigned)a.ntt;
    const int64_t m0 = (int64_t)(bx % (unsigned)a.ntt) * TOK;
    const int ks = (int)(lb / gridDim.x);
    const int64_t nsl = a.n_in / 32, nc64 = a.N / 64;
    const int64_t I0 = (int64_t)ks * a.slices_per_split;
    const int64_t I1 = min(I0 + (int64_t)a.slices_per_split, nsl);

    // staging: thread t takes token sm = t / TPR and rows RPT sp .. RPT sp +
    // RPT - 1 of the slice (h of tokens past M is zero), and table entry (row t / 16,
    // value t % 16: sub-block scale 0-7, then min 0-7).  A slice's global
    // operands (h, the rows' d / dmin, the header words, each wave's
    // nibbles) go to one of MMD_RING register slots MMD_RING slices ahead of
    // its use, so that the loads of several slices are in flight while one
    // is computed.  Per slice the bases move by uniform strides; the lanes'
    // offsets are fixed 32-bit values.
    const int sm = tid / TPR, sp = tid % TPR;
    const int trow = tid >> 4, tv = tid & 15, ts = tv & 7, tmn = tv >> 3;
    const bool tok_ok = m0 + sm < a.M;
    const float hscale = tok_ok ? MMD_ASCALE : 0.f;
    const uint32_t h_off = (uint32_t)(((tok_ok ? m0 + sm : 0) * a.ldh + RPT * sp) * 4);
    const uint32_t d_off = (uint32_t)(RPT * sp * 16);
    const uint32_t t_off = (uint32_t)(trow * 16);
    const uint32_t q_off = (uint32_t)(((((w >> 1) * 4 + kq) * 16 + col) * 16) + 8 * (w & 1));
    const uint8_t* hb = (const uint8_t*)a.h;
    const uint8_t* db = a.hdr + jb * a.n_in * 16;
    const uint8_t* qb = a.qs + jb * 4 * 4 * 16 * 16;
    const int64_t q_stride = nc64 * 4 * 16 * 16;
    struct Slot {
        float hv[RPT];
        uint32_t dw[RPT];  // d | dmin << 16 of rows RPT sp + e
        uint32_t ta, tb; // table entry: scale (S0) or min (S1) word, and S2 word
        v2i wq;          // this wave's nibbles of the slice (two column tiles)
    };
    auto issue = [&](Slot& o, int64_t I) {
        if constexpr (RPT == 4) {
            const float4 v = *(const float4*)(hb + I * 128 + h_off);
            o.hv[0] = v.x; o.hv[1] = v.y; o.hv[2] = v.z; o.hv[3] = v.w;
        } else {
            const float2 v = *(const float2*)(hb + I * 128 + h_off);
            o.hv[0] = v.x; o.hv[1] = v.y;
        }
        const uint8_t* dI = db + I * 512;
#pragma unroll
        for (int e = 0; e < RPT; ++e) o.dw[e] = *(const uint32_t*)(dI + d_off + e * 16);
        o.ta = *(const uint32_t*)(dI + t_off + 4 + 4 * tmn);
        o.tb = *(const uint32_t*)(dI + t_off + 12);
        o.wq = *(const v2i*)(qb + I * q_stride + q_off);
    };
    auto stage_store = [&](const Slot& o, int buf) {
        float hv[RPT];
#pragma unroll
        for (int e = 0; e < RPT; ++e) hv[e] = o.hv[e] * hscale;
        typedef _Float16 vRh __attribute__((ext_vector_type(RPT)));
        vRh dh, dl, mh, ml;
#pragma unroll
        for (int e = 0; e < RPT; e += 2) {
            float pd[2], pm[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                pd[i] = hv[e + i] * h2f((uint16_t)(o.dw[e + i] & 0xFFFF));
                pm[i] = hv[e + i] * h2f((uint16_t)(o.dw[e + i] >> 16));
            }
            v2h h, l;
            split_hl2(pd[0], pd[1], h, l);
            dh[e] = h[0];
            dh[e + 1] = h[1];
            dl[e] = l[0];
            dl[e + 1] = l[1];
            split_hl2(pm[0], pm[1], h, l);
            mh[e] = h[0];
            mh[e + 1] = h[1];
            ml[e] = l[0];
            ml[e + 1] = l[1];
        }
        *(vRh*)&ad[buf][0][sm][RPT * sp] = dh;
        *(vRh*)&ad[buf][1][sm][RPT * sp] = dl;
        *(vRh*)&am[buf][0][sm][RPT * sp] = mh;
        *(vRh*)&am[buf][1][sm][RPT * sp] = ml;
        // 6-bit scale (ta = S0) or min (ta = S1) of sub-block ts: byte ts of
        // the low words for ts < 4, else the low / high nibble of S2's byte
        // ts - 4 with the top two bits of ta's
        const int sh = 8 * (ts & 3);
        const uint32_t a8 = (o.ta >> sh) & 0xFFu, b8 = (o.tb >> sh) & 0xFFu;
        const uint32_t v = ts < 4 ? (a8 & 63u) : ((tmn ? (b8 >> 4) : (b8 & 15u)) | ((a8 >> 6) << 4));
        const _Float16 fv = (_Float16)(float)v;
        tsm[buf][tv][trow] = fv;
        tsn[buf][tv][trow] = fv * (_Float16)(-1024.f);
    };

    v4f acc[2][MS];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) acc[ct][ms] = v4f{0.f, 0.f, 0.f, 0.f};
    v4f accm = {0.f, 0.f, 0.f, 0.f};

    // one slice from LDS buffer buf with the wave's nibbles wq
    auto compute = [&](const v2i& wq, int buf) {
        v8h ah[MS], al[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            ah[ms] = ld8h(&ad[buf][0][16 * ms + col][8 * kq]);
            al[ms] = ld8h(&ad[buf][1][16 * ms + col][8 * kq]);
        }
        const v8h scv = ld8h(&tsm[buf][w][8 * kq]);
        const v8h snv = ld8h(&tsn[buf][w][8 * kq]);
        v8h b[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) b[ct] = nib8_sc((uint32_t)wq[ct], scv, snv);
        // every hi product first, then the lo ones: no MFMA waits on the
        // one before it
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms)
                acc[ct][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ms], b[ct], acc[ct][ms], 0, 0, 0);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms)
                acc[ct][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[ms], b[ct], acc[ct][ms], 0, 0, 0);
        // min term of tokens 16 w .. + 15 (waves 0 .. MS - 1): B columns = the 8 sub-blocks
        if (w < MS) {
            const v8h bm = col < 8 ? ld8h(&tsm[buf][8 + (col & 7)][8 * kq]) : v8h{};
            const v8h mh = ld8h(&am[buf][0][16 * w + col][8 * kq]);
            const v8h ml = ld8h(&am[buf][1][16 * w + col][8 * kq]);
            accm = __builtin_amdgcn_mfma_f32_16x16x32_f16(mh, bm, accm, 0, 0, 0);
            accm = __builtin_amdgcn_mfma_f32_16x16x32_f16(ml, bm, accm, 0, 0, 0);
        }
    };

    // slices I0 + k (k < MMD_RING) in flight; slice I0 staged
    Slot ring[MMD_RING];
#pragma unroll
    for (int k = 0; k < MMD_RING; ++k)
        if (I0 + k < I1) issue(ring[k], I0 + k);
    if (I0 < I1) stage_store(ring[0], 0);
    __syncthreads();
    // slice I = I0 + k uses slot k % MMD_RING; after its compute that slot
    // takes slice I + MMD_RING, and slice I + 1 (slot (k + 1) % MMD_RING) is
    // staged into the other LDS buffer
    for (int64_t Ib = I0; Ib < I1; Ib += MMD_RING) {
#pragma unroll
        for (int k = 0; k < MMD_RING; ++k) {
            const int64_t I = Ib + k;
            if (I >= I1) break;  // block-uniform
            const int buf = k & 1;
            if (I + 1 < I1) stage_store(ring[(k + 1) % MMD_RING], buf ^ 1);
            compute(ring[k].wq, buf);
            if (I + MMD_RING < I1) issue(ring[k], I + MMD_RING);
            __syncthreads();
        }
    }
    // the min terms of every token and sub-block, through LDS
    if (w < MS && col < 8) {
#pragma unroll
        for (int r = 0; r < 4; ++r) mins[16 * w + 4 * kq + r][col] = accm[r];
    }
    __syncthreads();
    const MmOutDev& o = a.out;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tk = 16 * ms + 4 * kq + r;
            const int64_t m = m0 + tk;
            if (m >= a.M) continue;
            int sq = 0;
            while (sq + 1 < o.nseq && m >= o.row0[sq + 1]) ++sq;
            float* yrow = o.base[sq] + (m - o.row0[sq]) * o.ld + (int64_t)ks * o.split_stride;
            const float mn = mins[tk][w];
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const float v = (acc[ct][ms][r] - mn) * (1.f / MMD_ASCALE);
                float* yp = yrow + jb * 256 + 32 * w + 16 * ct + col;
                *yp = o.accum ? *yp + v : v;
            }
        }
}

// ---------------------------------------------------------------- re-tile
// Q8_0 / Q4_0 rows (planes of `rows` rows, nplanes of them) into the
// one-pass GEMM's tiles: thread (plane, tile T, step s, lane l) copies the
// lane's bytes of the step's 8 blocks (row 16 T + l % 16, bytes 8 (l / 16) ..
// (Q8_0) or 4 (l / 16) .. (Q4_0) of each block's quants), threads past the
// lanes copy the tile's 16 x 8 scales; rows past `rows` are zeros.  Q6_K
// (from the planar device rows): the lane's ql / qh runs, then the rows'
// scales and d.
__global__ void __launch_bounds__(256) k_mm_tile(const uint8_t* __restrict__ src, int dt,
                                                 int64_t rows, int64_t nplanes, int64_t K,
                                                 uint8_t* __restrict__ dst) {
    const int64_t nsb = K / 256, tiles = (rows + 15) / 16;
    const int bb = dt == FTX_Q8_0_MMT ? 34 : 18;
    const int lb = (int)mmt_lane_bytes(dt);
    const int64_t rb = K / 32 * bb;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= nplanes * tiles * nsb * 80) return;
    const int64_t u = id / 80;  // (plane, tile, step)
    const int w = (int)(id % 80);
    const int64_t s = u % nsb, T = (u / nsb) % tiles, pl = u / (nsb * tiles);
    uint8_t* out = dst + u * mmt_step_bytes(dt);
    if (dt == FTX_Q6_K_MMT) {
        // from the planar Q6_K rows (quant_dev.h): QL, QH, SC and D planes
        const int64_t prb = q6k_dev_row_bytes(K);
        const uint8_t* pp = src + pl * rows * prb;
        if (w < 64) {
            const int col = w & 15, kq = w >> 4;
            const int64_t n = 16 * T + col;
            const uint8_t* row = pp + n * prb;
            for (int r = 0; r < 4; ++r)
                for (int i = 0; i < 8; ++i)
                    out[w * 48 + 8 * r + i] =
                        n < rows ? row[s * 128 + q6k_ql_dev(32 * r + 8 * kq + i)] : 0;
            for (int h = 0; h < 2; ++h)
                for (int i = 0; i < 8; ++i)
                    out[w * 48 + 32 + 8 * h + i] =
                        n < rows ? row[nsb * 128 + s * 64 + q6k_qh_dev(32 * h + 8 * kq + i)] : 0;
        } else {
            const int r = w - 64;
            const int64_t n = 16 * T + r;
            const uint8_t* row = pp + n * prb;
            for (int i = 0; i < 16; ++i) out[64 * 48 + r * 16 + i] = n < rows ? row[nsb * 192 + s * 16 + i] : 0;
            for (int i = 0; i < 2; ++i) out[64 * 48 + 256 + r * 2 + i] = n < rows ? row[nsb * 208 + s * 2 + i] : 0;
        }
        return;
    }
    const uint8_t* plane = src + pl * rows * rb;
    if (w < 64) {
        const int col = w & 15, kq = w >> 4;
        const int64_t n = 16 * T + col;
        for (int j = 0; j < 8; ++j)
            for (int i = 0; i < lb / 8; ++i)
                out[w * lb + j * (lb / 8) + i] =
                    n < rows ? plane[n * rb + (8 * s + j) * bb + 2 + kq * (lb / 8) + i] : 0;
    } else {
        const int r = w - 64;
        const int64_t n = 16 * T + r;
        for (int j = 0; j < 8; ++j)
            for (int i = 0; i < 2; ++i)
                out[64 * lb + r * 16 + 2 * j + i] = n < rows ? plane[n * rb + (8 * s + j) * bb + i] : 0;
    }
}

// ---------------------------------------------------------------- reduce
// out[m][n] (= or +=) sum_ks part[ks][m][n] in split order; SwiGLU:
// out[m][n] = silu(g) * u with g, u the sums of columns n and n + N
// (src/engine.cpp:271-273).  grid = (ceil(N / 256), M).
// Expert launches (xtab set): rows outside the tiles in use, and past a
// tile's rows in use, are zeros.  Fragment output (fh set): the result
// times fscale goes to the fp16 hi + lo operand planes (k_mm_prep's
// fragment order, contraction fK) instead of out.
struct MmReduceArgs {
    const float* part;
    int64_t split_stride, ldp;
    int S;
    int64_t N;
    int swiglu;
    MmOutDev out;
    const int32_t* xtab;
    int64_t trows;  // rows per tile of xtab
    _Float16 *fh, *fl;
    float fscale;
    int64_t fK;
};

__global__ void __launch_bounds__(256) k_mm_reduce(MmReduceArgs a) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t m = blockIdx.y;
    if (n >= a.N) return;
    bool valid = true;
    if (a.xtab) {
        const int64_t t = m / a.trows;
        valid = t < a.xtab[0] && m - t * a.trows < a.xtab[2 + 2 * t];
    }
    float v = 0.f;
    if (valid) {
        const float* p = a.part + m * a.ldp + n;
        float g = 0.f, u = 0.f;
        for (int s = 0; s < a.S; ++s) g += p[(int64_t)s * a.split_stride];
        if (a.swiglu)
            for (int s = 0; s < a.S; ++s) u += p[(int64_t)s * a.split_stride + a.N];
        v = a.swiglu ? g / (1.f + expf(-g)) * u : g;
    }
    if (a.fh) {
#pragma clang fp contract(off)
        const int64_t at = frag_at(m, n, a.fK, false);
        _Float16 h, l;
        split_hl(v * a.fscale, h, l);
        a.fh[at] = h;
        a.fl[at] = l;
        return;
    }
    const MmOutDev& o = a.out;
    int sq = 0;
    while (sq + 1 < o.nseq && m >= o.row0[sq + 1]) ++sq;
    float* yp = o.base[sq] + (m - o.row0[sq]) * o.ld + n;
    *yp = o.accum ? *yp + v : v;
}

// The same for dense launches (no tile table, no fragment output) with every
// row, split and output 16-byte aligned: four columns per thread, the same
// sums in the same order.  grid = (ceil(N / 1024), M).
__global__ void __launch_bounds__(256) k_mm_reduce4(MmReduceArgs a) {
    const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const int64_t m = blockIdx.y;
    if (n >= a.N) return;
    const float* p = a.part + m * a.ldp + n;
    float4 g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < a.S; ++s) {
        const float4 t = *(const float4*)(p + (int64_t)s * a.split_stride);
        g.x += t.x;
        g.y += t.y;
        g.z += t.z;
        g.w += t.w;
    }
    if (a.swiglu) {
        for (int s = 0; s < a.S; ++s) {
            const float4 t = *(const float4*)(p + (int64_t)s * a.split_stride + a.N);
            u.x += t.x;
            u.y += t.y;
            u.z += t.z;
            u.w += t.w;
        }
        g.x = g.x / (1.f + expf(-g.x)) * u.x;
        g.y = g.y / (1.f + expf(-g.y)) * u.y;
        g.z = g.z / (1.f + expf(-g.z)) * u.z;
        g.w = g.w / (1.f + expf(-g.w)) * u.w;
    }
    const MmOutDev& o = a.out;
    int sq = 0;
    while (sq + 1 < o.nseq && m >= o.row0[sq + 1]) ++sq;
    float4* yp = (float4*)(o.base[sq] + (m - o.row0[sq]) * o.ld + n);
    if (o.accum) {
        const float4 y = *yp;
        g.x += y.x;
        g.y += y.y;
        g.z += y.z;
        g.w += y.w;
    }
    *yp = g;
}

}  // namespace

// ---------------------------------------------------------------- host

int64_t mm_pad_tokens(int64_t M) { return (M + MM_TOK - 1) / MM_TOK * MM_TOK; }

size_t mm_act_halves(int64_t Mp, int64_t K) { return (size_t)(Mp * K * 2 + Mp * (K / 32) * 2); }

MmAct mm_act(void* buf, int64_t Mp, int64_t K) {
    MmAct a;
    a.xh = (_Float16*)buf;
    a.xl = a.xh + Mp * K;
    a.sh = a.xl + Mp * K;
    a.sl = a.sh + Mp * (K / 32);
    a.Mp = Mp;
    a.K = K;
    return a;
}

// k_mm_prep_row for K <= 16384 (S = 0: no partials to add)
static hipError_t launch_prep_row(hipStream_t st, float* x, int64_t ldx, const float* normw,
                                  float eps, int64_t M, const MmAct& act, int weight_dt,
                                  const int32_t* gather, const float* part, int64_t split_stride,
                                  int64_t ldp, int S) {
    const int ch = (int)((act.K + 4095) / 4096);
    auto kern = ch == 1 ? k_mm_prep_row<1>
              : ch == 2 ? k_mm_prep_row<2>
              : ch == 3 ? k_mm_prep_row<3>
                        : k_mm_prep_row<4>;
    hipLaunchKernelGGL(kern, dim3((unsigned)act.Mp), dim3(1024), 0, st, x, ldx, normw, eps, act.K,
                       (int)M, weight_dt == FTX_Q4_0_MMT ? 1 : 0, gather, part, split_stride, ldp,
                       S, act.xh, act.xl, act.sh, act.sl);
    return hipGetLastError();
}

hipError_t launch_mm_prep(hipStream_t st, const float* x, int64_t ldx, const float* normw,
                          float eps, int64_t M, const MmAct& act, int weight_dt,
                          const int32_t* gather) {
    if (act.K % 256 || M < 1 || M > act.Mp || act.Mp % MM_TOK || ldx % 4 || ((uintptr_t)x & 15) ||
        ((uintptr_t)normw & 15))
        return hipErrorInvalidValue;
    // (the row kernel does not write x when it adds no partials)
    if (act.K <= 4096 * MMF_CH)
        return launch_prep_row(st, const_cast<float*>(x), ldx, normw, eps, M, act, weight_dt,
                               gather, nullptr, 0, 0, 0);
    hipLaunchKernelGGL(k_mm_prep, dim3((unsigned)act.Mp, (unsigned)((act.K + 1023) / 1024)),
                       dim3(256), 0, st, x, ldx, normw, eps,
                       act.K, (int)M, weight_dt == FTX_Q4_0_MMT ? 1 : 0, gather, act.xh,
                       act.xl, act.sh, act.sl);
    return hipGetLastError();
}

hipError_t launch_mm_prep_fold(hipStream_t st, float* x, int64_t ldx, const float* normw,
                               float eps, int64_t M, const MmAct& act, int weight_dt,
                               const MmPend& fold) {
    if (fold.S < 1) return launch_mm_prep(st, x, ldx, normw, eps, M, act, weight_dt);
    if (!fold.accum || act.K % 256 || act.K > 4096 * MMF_CH || M < 1 || M > act.Mp || act.Mp % MM_TOK ||
        ldx % 4 || ((uintptr_t)x & 15) || ((uintptr_t)normw & 15) || fold.N != act.K ||
        fold.ldp % 4 || fold.split_stride % 4 || ((uintptr_t)fold.part & 15))
        return hipErrorInvalidValue;
    return launch_prep_row(st, x, ldx, normw, eps, M, act, weight_dt, nullptr, fold.part,
                           fold.split_stride, fold.ldp, fold.S);
}

// k_mm_reduce over `rows` rows, four columns per thread where the operands
// allow (no tile table or fragment output, 16-byte aligned rows and splits)
static hipError_t launch_reduce(hipStream_t st, const MmReduceArgs& r, int64_t rows) {
    bool vec = !r.xtab && !r.fh && r.N % 4 == 0 && r.ldp % 4 == 0 && r.split_stride % 4 == 0 &&
               ((uintptr_t)r.part & 15) == 0 && r.out.ld % 4 == 0;
    for (int s = 0; s < r.out.nseq; ++s) vec = vec && ((uintptr_t)r.out.base[s] & 15) == 0;
    if (vec)
        hipLaunchKernelGGL(k_mm_reduce4, dim3((unsigned)((r.N + 1023) / 1024), (unsigned)rows),
                           dim3(256), 0, st, r);
    else
        hipLaunchKernelGGL(k_mm_reduce, dim3((unsigned)((r.N + 255) / 256), (unsigned)rows),
                           dim3(256), 0, st, r);
    return hipGetLastError();
}

hipError_t launch_mm_fold(hipStream_t st, const MmPend& fold, int64_t M, float* y, int64_t ldy) {
    if (fold.S < 1) return hipSuccess;
    MmReduceArgs r{};
    r.part = fold.part;
    r.split_stride = fold.split_stride;
    r.ldp = fold.ldp;
    r.S = fold.S;
    r.swiglu = 0;
    r.N = fold.N;
    r.out.nseq = 1;
    r.out.base[0] = y;
    r.out.row0[0] = 0;
    r.out.row0[1] = M;
    r.out.ld = ldy;
    r.out.accum = fold.accum;
    return launch_reduce(st, r, M);
}

bool mm_supported(int dt, int64_t K) {
    return (dt == FTX_Q4_K || dt == FTX_Q8_0_MMT || dt == FTX_Q4_0_MMT || dt == FTX_Q6_K_MMT) &&
           K % 256 == 0 && K >= 256;
}

int mm_tiled_dtype(int dt, int64_t K) {
    if (K % 256) return -1;
    return dt == FTX_Q8_0   ? FTX_Q8_0_MMT
           : dt == FTX_Q4_0 ? FTX_Q4_0_MMT
           : dt == FTX_Q6_K ? FTX_Q6_K_MMT
                            : -1;
}

size_t mm_tiled_bytes(int mdt, int64_t rows, int64_t K) {
    return (size_t)((rows + 15) / 16) * (size_t)(K / 256) * (size_t)mmt_step_bytes(mdt);
}

hipError_t launch_mm_tile(hipStream_t st, const uint8_t* src, int dt, int64_t rows,
                          int64_t nplanes, int64_t K, uint8_t* dst) {
    const int mdt = mm_tiled_dtype(dt, K);
    if (mdt < 0 || rows < 1 || nplanes < 1) return hipErrorInvalidValue;
    const int64_t n = nplanes * ((rows + 15) / 16) * (K / 256) * 80;
    hipLaunchKernelGGL(k_mm_tile, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src, mdt,
                       rows, nplanes, K, dst);
    return hipGetLastError();
}

bool mm_down_supported(int dt, int64_t n_in, int64_t N) {
    return dt == FTX_Q4_K && n_in % 32 == 0 && N % 256 == 0;
}

static MmOutDev out_dev(const MmOut& o) {
    MmOutDev d{};
    d.nseq = o.nseq;
    for (int s = 0; s < o.nseq; ++s) {
        d.base[s] = o.base[s];
        d.row0[s] = o.row0[s];
    }
    d.row0[o.nseq] = o.row0[o.nseq];
    d.ld = o.ld;
    d.split_stride = 0;
    d.accum = o.accum;
    return d;
}

// split count for `tiles` workgroups over `steps` contraction steps: the
// kernels hold one workgroup per CU, so the tiles x S workgroups run in
// rounds of cu_count, each as long as its ceil(steps / S) steps plus, when
// split, writing its partials (about pcost steps); the S <= 32 (and at
// least two steps per split) of the fewest step times, the smallest on ties
// (a 70B-shaped batch: gate / up 896 tiles -> 2 splits, 7 full rounds
// instead of 3.5; qkv 160 tiles -> 3 splits)
constexpr int64_t MM_SPLIT_COST = 2;    // k_mm: 256-element steps
constexpr int64_t MMD_SPLIT_COST = 14;  // k_mm_down: 32-row slices
static int mm_splits(int64_t tiles, int64_t steps, int cu_count, int64_t pcost) {
    const int64_t cus = cu_count > 0 ? cu_count : 256;
    if (tiles < 1) return 1;
    int best = 1;
    int64_t best_cost = -1;
    for (int64_t S = 1; S <= 32 && (S == 1 || S <= steps / 2); ++S) {
        const int64_t cost = (tiles * S + cus - 1) / cus * ((steps + S - 1) / S + (S > 1 ? pcost : 0));
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = (int)S;
        }
    }
    return best;
}

size_t mm_part_floats(int64_t Mp, int64_t N, int64_t steps, int64_t ntiles, int cu_count) {
    const int S = mm_splits(ntiles * (Mp / MM_TOK), steps, cu_count, MM_SPLIT_COST);
    return S > 1 ? (size_t)S * (size_t)Mp * (size_t)N : 0;
}

// both forms: dense (xtab null: rows 0 .. M - 1 of the operand, tiles of
// 64) and expert (grid.y = ntile_max entries of the tile table; plane:
// bytes per expert plane of each segment; the outputs are operand rows)
static hipError_t mm_launch(hipStream_t st, const MmSeg* segs, int nseg, const MmAct& act,
                            int64_t M, int epi, const MmOut& out, float* part,
                            size_t part_floats, int cu_count, const int32_t* xtab,
                            const int64_t* plane, int64_t ntile_max, int64_t trows,
                            const MmFragOut* fo, MmPend* pend) {
    if (pend) *pend = MmPend{};
    if (nseg < 1 || nseg > 3 || M < 1 || M > act.Mp || out.nseq < 1 || out.nseq > FTX_MAX_SEQ)
        return hipErrorInvalidValue;
    if (xtab && (ntile_max < 1 || (trows != 16 && trows != 64) || ntile_max * trows > act.Mp ||
                 !plane))
        return hipErrorInvalidValue;
    // dense launches of at most 32 tokens take 16- or 32-token tiles: the
    // MFMAs, fragment reads and accumulator updates of the padding rows of a
    // 64-token tile are then not spent
    const int ms = xtab ? (int)(trows / 16) : (M <= 16 ? 1 : (M <= 32 ? 2 : MM_MS));
    if (fo && (!xtab || epi != EPI_SWIGLU)) return hipErrorInvalidValue;
    const int dt = segs[0].dt;
    MmArgs a{};
    a.nseg = nseg;
    int64_t units = 0, cols = 0;
    for (int i = 0; i < nseg; ++i) {
        if (segs[i].dt != dt || !mm_supported(dt, act.K)) return hipErrorInvalidValue;
        if (dt == FTX_Q4_K && segs[i].rpt != 16 && segs[i].rpt != 32) return hipErrorInvalidValue;
        MmSegDev& d = a.seg[i];
        d.W = segs[i].W;
        d.N = segs[i].N;
        d.unit0 = units;
        d.col0 = cols;
        d.row_bytes = segs[i].row_bytes;
        d.rpt = segs[i].rpt;
        units += (segs[i].N + MM_WROWS - 1) / MM_WROWS;
        cols += segs[i].N;
        a.plane[i] = plane ? plane[i] : 0;
    }
    a.xtab = xtab;
    a.units = units;
    a.K = act.K;
    a.nsb = (int)(act.K / 256);
    a.xh = act.xh;
    a.xl = act.xl;
    a.sh = act.sh;
    a.sl = act.sl;
    a.M = (int)M;
    const int64_t wg = (units + MM_WAVES - 1) / MM_WAVES,
                  mt = xtab ? ntile_max : (ms == MM_MS ? act.Mp / MM_TOK : 1);
    int S = mm_splits(wg * mt, a.nsb, cu_count, MM_SPLIT_COST);
    // SwiGLU needs the gate and up sums together: always through the reduce
    const bool via_part = S > 1 || epi == EPI_SWIGLU || xtab;
    if (via_part) {
        if (!part || (size_t)S * (size_t)act.Mp * (size_t)cols > part_floats) {
            S = 1;
            if (!part || (size_t)act.Mp * (size_t)cols > part_floats) return hipErrorInvalidValue;
        }
        MmOutDev& o = a.out;
        o.nseq = 1;
        o.base[0] = part;
        o.row0[0] = 0;
        o.row0[1] = act.Mp;
        o.ld = cols;
        o.split_stride = act.Mp * cols;
        o.accum = 0;
    } else {
        a.out = out_dev(out);
    }
    a.sb_per_split = (a.nsb + S - 1) / S;
    S = (a.nsb + a.sb_per_split - 1) / a.sb_per_split;
    a.ntt = (int)mt;
    const dim3 grid((unsigned)(wg * mt), 1, (unsigned)S);
    const size_t lds = 2 * (size_t)ms * 16384;
    using K_t = void (*)(MmArgs);
    // [dtype][dense 64 | expert 64-row tiles | expert 16-row tiles | dense
    // 32 | dense 16] (Q6_K: dense only)
    static const K_t kerns[4][5] = {
        {k_mm<FTX_Q4_K, false, 4>, k_mm<FTX_Q4_K, true, 4>, k_mm<FTX_Q4_K, true, 1>,
         k_mm<FTX_Q4_K, false, 2>, k_mm<FTX_Q4_K, false, 1>},
        {k_mm<FTX_Q8_0_MMT, false, 4>, k_mm<FTX_Q8_0_MMT, true, 4>, k_mm<FTX_Q8_0_MMT, true, 1>,
         k_mm<FTX_Q8_0_MMT, false, 2>, k_mm<FTX_Q8_0_MMT, false, 1>},
        {k_mm<FTX_Q4_0_MMT, false, 4>, k_mm<FTX_Q4_0_MMT, true, 4>, k_mm<FTX_Q4_0_MMT, true, 1>,
         k_mm<FTX_Q4_0_MMT, false, 2>, k_mm<FTX_Q4_0_MMT, false, 1>},
        {k_mm<FTX_Q6_K_MMT, false, 4>, nullptr, nullptr, k_mm<FTX_Q6_K_MMT, false, 2>,
         k_mm<FTX_Q6_K_MMT, false, 1>}};
    const int di = dt == FTX_Q4_K ? 0 : (dt == FTX_Q8_0_MMT ? 1 : (dt == FTX_Q4_0_MMT ? 2 : 3));
    const int vi = xtab ? (ms == 4 ? 1 : 2) : (ms == 4 ? 0 : (ms == 2 ? 3 : 4));
    const K_t kern = kerns[di][vi];
    if (!kern) return hipErrorInvalidValue;
    static bool lds_set[20] = {};
    const int ki = di * 5 + vi;
    if (!lds_set[ki]) {
        hipError_t e = hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        lds_set[ki] = true;
    }
    ktimed_launch(kern, grid, dim3(64 * MM_WAVES), (uint32_t)lds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !via_part) return e;
    if (pend && epi != EPI_SWIGLU && !xtab && out.nseq == 1 && !fo) {
        // left for the consumer to add into (or store as) out
        pend->part = part;
        pend->split_stride = act.Mp * cols;
        pend->ldp = cols;
        pend->S = S;
        pend->N = cols;
        pend->accum = out.accum;
        return hipSuccess;
    }
    MmReduceArgs r{};
    r.part = part;
    r.split_stride = act.Mp * cols;
    r.ldp = cols;
    r.S = S;
    r.swiglu = epi == EPI_SWIGLU;
    r.N = r.swiglu ? cols / 2 : cols;
    r.out = out_dev(out);
    r.xtab = xtab;
    r.trows = trows;
    if (fo) {
        r.fh = fo->h;
        r.fl = fo->l;
        r.fscale = fo->scale;
        r.fK = fo->K;
    }
    return launch_reduce(st, r, xtab ? ntile_max * trows : M);
}

hipError_t launch_mm(hipStream_t st, const MmSeg* segs, int nseg, const MmAct& act, int64_t M,
                     int epi, const MmOut& out, float* part, size_t part_floats, int cu_count,
                     MmPend* pend) {
    return mm_launch(st, segs, nseg, act, M, epi, out, part, part_floats, cu_count, nullptr,
                     nullptr, 0, 0, nullptr, pend);
}

hipError_t launch_mm_experts(hipStream_t st, const MmSeg* segs, int nseg, const int64_t* plane,
                             const MmAct& act, const int32_t* xtab, int64_t ntile_max,
                             int64_t trows, const MmFragOut& fo, float* part, size_t part_floats,
                             int cu_count) {
    if (fo.K != segs[0].N || fo.K % 32) return hipErrorInvalidValue;
    MmOut o{};
    o.nseq = 1;
    o.row0[1] = ntile_max * trows;
    return mm_launch(st, segs, nseg, act, ntile_max * trows, EPI_SWIGLU, o, part, part_floats,
                     cu_count, xtab, plane, ntile_max, trows, &fo, nullptr);
}

hipError_t launch_mm_down(hipStream_t st, const uint8_t* tiled, int64_t n_in, int64_t N,
                          const float* h, int64_t ldh, int64_t M, const MmOut& out, float* part,
                          size_t part_floats, int cu_count, MmPend* pend) {
    if (pend) *pend = MmPend{};
    const int64_t Mp = mm_pad_tokens(M);
    if (!mm_down_supported(FTX_Q4_K, n_in, N) || M < 1 || out.nseq < 1 || out.nseq > FTX_MAX_SEQ ||
        ldh % 4 || ((uintptr_t)h & 15))
        return hipErrorInvalidValue;
    MmDownArgs a{};
    a.qs = tiled;
    a.hdr = tiled + n_in * N / 2;
    a.h = h;
    a.ldh = ldh;
    a.M = (int)M;
    a.n_in = n_in;
    a.N = N;
    // launches of at most 32 tokens take 32-token tiles
    const int ms = M <= 32 ? 2 : MM_MS;
    const int64_t nsl = n_in / 32, nb = N / 256, mt = ms == MM_MS ? Mp / MM_TOK : 1;
    int S = mm_splits(nb * mt, nsl, cu_count, MMD_SPLIT_COST);
    if (S > 1 && (!part || (size_t)S * (size_t)Mp * (size_t)N > part_floats)) S = 1;
    a.slices_per_split = (int)((nsl + S - 1) / S);
    S = (int)((nsl + a.slices_per_split - 1) / a.slices_per_split);
    if (S > 1) {
        MmOutDev& o = a.out;
        o.nseq = 1;
        o.base[0] = part;
        o.row0[0] = 0;
        o.row0[1] = Mp;
        o.ld = N;
        o.split_stride = Mp * N;
        o.accum = 0;
    } else {
        a.out = out_dev(out);
    }
    a.ntt = (int)mt;
    if (ms == 2)
        ktimed_launch(k_mm_down<2>, dim3((unsigned)(nb * mt), 1, (unsigned)S), dim3(64 * MMD_WAVES), 0,
                      st, a);
    else
        ktimed_launch(k_mm_down<MM_MS>, dim3((unsigned)(nb * mt), 1, (unsigned)S),
                      dim3(64 * MMD_WAVES), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    if (pend && out.accum && out.nseq == 1) {
        // left for the next activation prep to add into out
        pend->part = part;
        pend->split_stride = Mp * N;
        pend->ldp = N;
        pend->S = S;
        pend->N = N;
        pend->accum = 1;
        return hipSuccess;
    }
    MmReduceArgs r{};
    r.part = part;
    r.split_stride = Mp * N;
    r.ldp = N;
    r.S = S;
    r.swiglu = 0;
    r.N = N;
    r.out = out_dev(out);
    return launch_reduce(st, r, M);
}

size_t mm_down_part_floats(int64_t Mp, int64_t n_in, int64_t N, int cu_count) {
    const int S = mm_splits((N / 256) * (Mp / MM_TOK), n_in / 32, cu_count, MMD_SPLIT_COST);
    return S > 1 ? (size_t)S * (size_t)Mp * (size_t)N : 0;
}
