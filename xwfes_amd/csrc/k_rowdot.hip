// k_rowdot.hip -- the verify step's quantised GEMV for up to 8 activation
// rows (y = x W^T, quantisation blocks along the contraction) on
// v_mfma_i32_16x16x32_i8 with the weights as the B operand.
//
// Math (as k_mfma.hip).  Activations are split per row m and 256-element
// block into two int8 limbs with a block scale s = max|x_block| / 127:
// x ~= s*(a + b/256).  Weights enter the MFMA as their raw quantised
// integers, so every product and sum inside it is exact; scales are applied
// to the MFMA outputs:
//   Q4_K  w = d*sc_j*q - dmin*m_j  (q in 0..15, sub-block j of 32)
//     y = sum_sb s_sb * [ d * sum_j sc_j * (A_j . q_j) - dmin * sum_j m_j * X_j ]
//   Q6_K  w = d*sc_s*(q - 32)      (q in 0..63, sub-block s of 16)
//     y = sum_sb s_sb * d * [ sum_s sc_s * (A_s . q_s) - 32 * sum_s sc_s * X_s ]
// with X the limb sums of a sub-block (formed by two more MFMAs whose B
// operand holds the eight m_j, or the sixteen sc_s, and whose A operand the
// 6-bit-split sums of the activation operand).
// Shapes.  v_mfma_i32_16x16x32_i8: lane l holds A[l%16][8(l/16) + e],
// B[8(l/16) + e][l%16] (e < 8) and C[4(l/16) + i][l%16] (i < 4).  A rows
// 0..7 = limb a of rows m = 0..7, rows 8..15 = limb b, so each activation
// byte is held once; B columns = 16 weight rows (lane l's own row l%16), so
// a lane needs the scales of its own row only.  C lane (col, g) holds limb
// g / 2 of rows 4 (g % 2) .. +3 for weight row col.
//   Q4_K: one MFMA per 32-element sub-block (its nibbles are the B bytes).
//   Q6_K: K = 32 holds two 16-element sub-blocks (lanes g < 2 and g >= 2);
//   two MFMAs, each with the other sub-block's B lanes zero.
// Weights come from the tiled copies of k_mfma.hip (tiles of R = 16 or 32
// rows per super-block); a unit is 16 rows (a gate sub-tile and its up
// sub-tile for SwiGLU), and lane (col, g) reads its bytes as 8-byte runs,
// each wave-wide load one contiguous 512-byte run (R = 16).
// Work split.  A workgroup owns one unit over the whole contraction; its W
// waves take SPW consecutive super-blocks each, and every load a wave makes
// (the sums of squares, activation operands, limb sums, block scales and
// weights of all its super-blocks) is issued at entry, so no use waits for a
// load issued after an earlier use.  The wave partials are added in wave
// order in LDS (deterministic), then the epilogue (store, accumulate, SwiGLU
// or the qkv RoPE / KV write) runs on one thread per output.
#include "ftx_internal.h"
#include "quant_dev.h"
#include "xq_dev.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int RD_MAXW = 8;  // waves per unit (K <= 8192 at 4 super-blocks a wave)

struct RdSeg {
    const uint8_t* W;  // tiled copy, R rows per tile
    int64_t N;
    int64_t u0;        // first unit of the segment
    float* y;          // outputs [m][ldy]
    int64_t ldy;
    int R;             // 16 or 32
    int dt;
    int role;          // the caller's segment index (EPI_QKV: 0 q, 1 k, 2 v)
};

struct RdArgs {
    RdSeg seg[3];
    int nseg;
    int64_t units;   // 16-row units (SwiGLU: gate sub-tiles; sub-tile u of seg 1 is its up)
    int nsb;         // super-blocks per row
    int W;           // waves with super-blocks (the block may hold one more)
    int M;
    int epi;
    const int8_t* frag;
    const int8_t* xs32;
    const int8_t* xs16;
    const float* scale;
    const float* ssq;  // per-block sums of x^2 [sb][8] for an RMS-normed input, else null
    float eps;
    int64_t K;
    QkvEpi qkv;
};

__device__ __forceinline__ long as_long(v2i v) { return __builtin_bit_cast(long, v); }

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
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
}

// Keeps the compiler from re-associating the integer multiply-add chain
// into a tree that holds every MFMA result live at once.  Emits nothing.
__device__ __forceinline__ void reg_fence4(int* v) {
#pragma unroll
    for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(v[r]));
}

// one (16-row sub-tile, super-block) of weights for lane (col, g)
template <int DT>
struct RdW {
    v2i q[DT == FTX_Q4_K ? 4 : 6];  // Q4_K: pairs c; Q6_K: QL runs 0..3, QH runs 4..5
    v4i h;                          // Q4_K header / Q6_K int8 scales
    uint32_t d;                     // Q6_K fp16 d
};

// the activation operand of one super-block for lane (r, g)
struct RdX {
    v4i a[4];   // 64 bytes: sub-block j at bytes 8 j ..
    v4i xs;     // Q4_K: 32-element sums (lo 8 B, hi 8 B) of row r; Q6_K: 16-element lo / hi runs
    float4 s4;  // block scales of rows 4 (g % 2) .. +3
};

__device__ __forceinline__ long af_of(const RdX& x, int j) {
    const v4i v = x.a[j >> 1];
    return (j & 1) ? as_long(v2i{v.z, v.w}) : as_long(v2i{v.x, v.y});
}

template <int DT>
__device__ __forceinline__ void rd_load_w(RdW<DT>& o, const RdSeg& sg, int64_t st, int nsb, int sb,
                                          int col, int g) {
    const int R = sg.R, per = R >> 4;
    const int64_t T = st / per;
    const int r = 16 * (int)(st % per) + col;
    if constexpr (DT == FTX_Q4_K) {
        const uint8_t* blk = sg.W + (T * nsb + sb) * (int64_t)R * 144;
        const int li = r + R * (g >> 1), off = 8 * (g & 1);
#pragma unroll
        for (int c = 0; c < 4; ++c) o.q[c] = *(const v2i*)(blk + (c * 2 * R + li) * 16 + off);
        o.h = *(const v4i*)(blk + 8 * R * 16 + r * 16);
        o.d = 0;
    } else {
        const uint8_t* blk = sg.W + (T * nsb + sb) * (int64_t)R * 210;
        const int li = r + R * (g & 1), off = 8 * (g >> 1);
#pragma unroll
        for (int i = 0; i < 6; ++i) o.q[i] = *(const v2i*)(blk + (i * 2 * R + li) * 16 + off);
        o.h = *(const v4i*)(blk + 12 * R * 16 + r * 16);
        o.d = *(const uint16_t*)(blk + 12 * R * 16 + R * 16 + r * 2);
    }
}

template <int DT>
__device__ __forceinline__ void rd_load_x(RdX& x, const RdArgs& a, int sb, int lane, int g) {
    const v4i* fp = (const v4i*)(a.frag + (int64_t)sb * 4096 + lane * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) x.a[i] = fp[i];
    const int r = lane & 15;
    if constexpr (DT == FTX_Q4_K) {
        x.xs = *(const v4i*)(a.xs32 + (int64_t)sb * 256 + r * 16);
    } else {
        const int8_t* p = a.xs16 + (int64_t)sb * 512 + r * 32 + 8 * (g & 1);
        const v2i lo = *(const v2i*)p, hi = *(const v2i*)(p + 16);
        x.xs = v4i{lo.x, lo.y, hi.x, hi.y};
    }
    x.s4 = *(const float4*)(a.scale + (int64_t)sb * 8 + 4 * (g & 1));
}

// acc[i] += the super-block's contribution to C row 4 g + i (see the header)
__device__ __forceinline__ void rd_q4k(const RdW<FTX_Q4_K>& w, const RdX& x, float4 s4, int g,
                                       float* acc) {
    const uint32_t S0 = (uint32_t)w.h.y, S1 = (uint32_t)w.h.z, S2 = (uint32_t)w.h.w;
    const uint32_t sc_lo = S0 & 0x3F3F3F3Fu;
    const uint32_t mn_lo = S1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
    const v4i zero = {0, 0, 0, 0};
    int ai[4] = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t w0 = (uint32_t)w.q[c].x, w1 = (uint32_t)w.q[c].y;
#pragma unroll
        for (int hn = 0; hn < 2; ++hn) {
            const int j = 2 * c + hn;
            const v2i b = hn ? v2i{(int)((w0 >> 4) & 0x0F0F0F0Fu), (int)((w1 >> 4) & 0x0F0F0F0Fu)}
                             : v2i{(int)(w0 & 0x0F0F0F0Fu), (int)(w1 & 0x0F0F0F0Fu)};
            const v4i cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(af_of(x, j), as_long(b), zero, 0, 0, 0);
            const int sc = (int)(((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3))) & 0xFF);
#pragma unroll
            for (int i = 0; i < 4; ++i) ai[i] += __mul24(sc, cc[i]);
        }
        reg_fence4(ai);
    }
    // min term: A = the row's 6-bit-split 32-element sums (k = j < 8, lanes
    // g = 0), B = the eight m_j of the lane's row
    const bool g0 = g == 0;
    const long bm = g0 ? as_long(v2i{(int)mn_lo, (int)mn_hi}) : 0;
    const long alo = g0 ? as_long(v2i{x.xs.x, x.xs.y}) : 0;
    const long ahi = g0 ? as_long(v2i{x.xs.z, x.xs.w}) : 0;
    const v4i dlo = __builtin_amdgcn_mfma_i32_16x16x32_i8(alo, bm, zero, 0, 0, 0);
    const v4i dhi = __builtin_amdgcn_mfma_i32_16x16x32_i8(ahi, bm, zero, 0, 0, 0);
    const float d = h2f((uint16_t)((uint32_t)w.h.x & 0xFFFF));
    const float dmin = h2f((uint16_t)((uint32_t)w.h.x >> 16));
    const float sm[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int mins = dlo[i] + 64 * dhi[i];
        acc[i] += sm[i] * (d * (float)ai[i] - dmin * (float)mins);
    }
}

__device__ __forceinline__ void rd_q6k(const RdW<FTX_Q6_K>& w, const RdX& x, float4 s4, int g,
                                       float* acc) {
    const v4i zero = {0, 0, 0, 0};
    const bool lo_half = g < 2;  // lanes of the step's first 16-element sub-block
    int ai[4] = {0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int hf = p >> 2, k4 = p & 3;
        const v2i L = w.q[2 * hf + (k4 & 1)], H = w.q[4 + hf];
        const int nsh = 4 * (k4 >> 1), hsh = 2 * k4;
        const uint32_t q0 = (((uint32_t)L.x >> nsh) & 0x0F0F0F0Fu) | ((((uint32_t)H.x >> hsh) & 0x03030303u) << 4);
        const uint32_t q1 = (((uint32_t)L.y >> nsh) & 0x0F0F0F0Fu) | ((((uint32_t)H.y >> hsh) & 0x03030303u) << 4);
        const long b = as_long(v2i{(int)q0, (int)q1});
        const long b0 = lo_half ? b : 0, b1 = lo_half ? 0 : b;
        const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(af_of(x, p), b0, zero, 0, 0, 0);
        const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(af_of(x, p), b1, zero, 0, 0, 0);
        const int s0 = 2 * p, s1 = 2 * p + 1;
        const int sc0 = (int)(int8_t)(((uint32_t)w.h[s0 >> 2] >> (8 * (s0 & 3))) & 0xFF);
        const int sc1 = (int)(int8_t)(((uint32_t)w.h[s1 >> 2] >> (8 * (s1 & 3))) & 0xFF);
#pragma unroll
        for (int i = 0; i < 4; ++i) ai[i] += __mul24(sc0, c0[i]) + __mul24(sc1, c1[i]);
        reg_fence4(ai);
    }
    // -32 term: A = the row's 6-bit-split 16-element sums (k = s < 16, lanes
    // g < 2), B = the sixteen sc_s of the lane's row
    const v2i scp = (g & 1) ? v2i{w.h.z, w.h.w} : v2i{w.h.x, w.h.y};
    const long bs = lo_half ? as_long(scp) : 0;
    const long alo = lo_half ? as_long(v2i{x.xs.x, x.xs.y}) : 0;
    const long ahi = lo_half ? as_long(v2i{x.xs.z, x.xs.w}) : 0;
    const v4i clo = __builtin_amdgcn_mfma_i32_16x16x32_i8(alo, bs, zero, 0, 0, 0);
    const v4i chi = __builtin_amdgcn_mfma_i32_16x16x32_i8(ahi, bs, zero, 0, 0, 0);
    const float d = h2f((uint16_t)w.d);
    const float sm[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int corr = clo[i] + 64 * chi[i];
        acc[i] += sm[i] * (d * (float)(ai[i] - 32 * corr));
    }
}

__device__ __forceinline__ int rd_seg_of(const RdArgs& a, int64_t u) {
    return (a.nseg > 1 && u >= a.seg[1].u0) ? ((a.nseg > 2 && u >= a.seg[2].u0) ? 2 : 1) : 0;
}

// segment si of the launch, selected without indexing the argument array
__device__ __forceinline__ RdSeg rd_seg(const RdArgs& a, int si) {
    return si == 0 ? a.seg[0] : (si == 1 ? a.seg[1] : a.seg[2]);
}

// the epilogue's reads of output (m, n): (residual for EPI_ACCUM, cos, sin
// of a q / k row's rotation for EPI_QKV)
template <bool PAIR>
__device__ __forceinline__ float3 rd_epi_reads(const RdArgs& a, const RdSeg& sg, bool own, int m,
                                               int64_t n) {
    float3 r = make_float3(0.f, 1.f, 0.f);
    if (!PAIR && own) {
        if (a.epi == EPI_ACCUM) r.x = sg.y[(int64_t)m * sg.ldy + n];
        if (a.epi == EPI_QKV && sg.role < 2) {
            const int64_t d = n % a.qkv.hd;
            const float2 cs = *(const float2*)(a.qkv.cs + ((int64_t)m * (a.qkv.hd / 2) + d / 2) * 2);
            r.y = cs.x;
            r.z = cs.y;
        }
    }
    return r;
}

// the unit u of dtype DT: NT = 2 sub-tiles (SwiGLU gate, up) or 1
template <int DT, bool PAIR, int SPW>
__device__ __forceinline__ void rd_unit(const RdArgs& a, int64_t u, int si) {
    constexpr int NT = PAIR ? 2 : 1;
    __shared__ float part[RD_MAXW][NT][8][16];
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), W = a.W;
    const int sb0 = w * SPW;
    const RdSeg sg = rd_seg(a, si);
    const RdSeg sg1 = PAIR ? a.seg[1] : sg;  // the up segment of a SwiGLU pair
    const int64_t st = u - sg.u0;  // the unit's sub-tile in its segment(s)
    const int em = tid >> 4, ec = tid & 15;
    const int64_t en = st * 16 + ec;
    const bool eown = tid < 128 && em < a.M && en < sg.N;
    // the epilogue thread t < 128 owns output (m, c) = (t / 16, t % 16); its
    // residual (accumulate) or rotation (q / k) is read with the operands
    // (a wave past the super-blocks only joins the epilogue)
    float3 er = make_float3(0.f, 1.f, 0.f);
    if (w >= W) er = rd_epi_reads<PAIR>(a, sg, eown, em, en);
    if (w < W) {  // wave-uniform
    // ---- loads: sums of squares, activation operands, weights
    float4 ss = {0.f, 0.f, 0.f, 0.f};
    if (a.ssq)
        for (int b = col; b < a.nsb; b += 16) {
            const float4 t = *(const float4*)(a.ssq + (int64_t)b * 8 + 4 * (g & 1));
            ss.x += t.x;
            ss.y += t.y;
            ss.z += t.z;
            ss.w += t.w;
        }
    __builtin_amdgcn_sched_barrier(0);
    RdX x[SPW];
#pragma unroll
    for (int k = 0; k < SPW; ++k) rd_load_x<DT>(x[k], a, sb0 + k, lane, g);
    __builtin_amdgcn_sched_barrier(0);
    RdW<DT> wt[SPW][NT];
#pragma unroll
    for (int k = 0; k < SPW; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) rd_load_w<DT>(wt[k][t], t ? sg1 : sg, st, a.nsb, sb0 + k, col, g);
    __builtin_amdgcn_sched_barrier(0);
    er = rd_epi_reads<PAIR>(a, sg, eown, em, en);
    // the RMSNorm factor 1 / rms of rows 4 (g % 2) .. +3 (src/engine.cpp:23-41)
    float inv[4] = {1.f, 1.f, 1.f, 1.f};
    if (a.ssq) {
        const float kf = (float)a.K;
        inv[0] = 1.f / sqrtf(row16_sum(ss.x) / kf + a.eps);
        inv[1] = 1.f / sqrtf(row16_sum(ss.y) / kf + a.eps);
        inv[2] = 1.f / sqrtf(row16_sum(ss.z) / kf + a.eps);
        inv[3] = 1.f / sqrtf(row16_sum(ss.w) / kf + a.eps);
    }
    float acc[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = 0.f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        const float4 s4 = make_float4(x[k].s4.x * inv[0], x[k].s4.y * inv[1], x[k].s4.z * inv[2],
                                      x[k].s4.w * inv[3]);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if constexpr (DT == FTX_Q4_K)
                rd_q4k(wt[k][t], x[k], s4, g, acc[t]);
            else
                rd_q6k(wt[k][t], x[k], s4, g, acc[t]);
        }
    }
    // limb b (lanes g >= 2) onto limb a: lane (col, g < 2) then holds rows
    // 4 g .. 4 g + 3 of weight row col
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = acc[t][i] + __shfl_xor(acc[t][i], 32, 64) * (1.f / 256.f);
            if (g < 2) part[w][t][4 * g + i][col] = v;
        }
    }
    __syncthreads();
    if (tid < 128) {
        float gv = 0.f, uv = 0.f;
        for (int ww = 0; ww < W; ++ww) gv += part[ww][0][em][ec];
        if constexpr (PAIR)
            for (int ww = 0; ww < W; ++ww) uv += part[ww][NT - 1][em][ec];
        // threads t and t ^ 1 hold rows c and c ^ 1 (the RoPE pair)
        const float pv = __shfl_xor(gv, 1, 64);
        if (eown) {
            float* yp = sg.y + (int64_t)em * sg.ldy + en;
            if (PAIR)
                *yp = gv / (1.f + expf(-gv)) * uv;  // src/engine.cpp:271-273
            else if (a.epi == EPI_QKV)
                qkv_store(a.qkv, sg.role, em, en, gv, pv, er.y, er.z, yp);
            else
                *yp = a.epi == EPI_ACCUM ? er.x + gv : gv;
        }
    }
}

template <bool PAIR, int SPW, int MAXT>
__global__ void __launch_bounds__(MAXT) k_rd(RdArgs a) {
    const int64_t u = blockIdx.x;
    const int si = PAIR ? 0 : rd_seg_of(a, u);
    if (rd_seg(a, si).dt == FTX_Q4_K)
        rd_unit<FTX_Q4_K, PAIR, SPW>(a, u, si);
    else
        rd_unit<FTX_Q6_K, PAIR, SPW>(a, u, si);
}

}  // namespace

bool rd_supported(int dt, int64_t K, int64_t M) {
    return (dt == FTX_Q4_K || dt == FTX_Q6_K) && M >= 1 && M <= 8 && K % 512 == 0 &&
           K <= 8192;
}

// super-blocks per wave: 2 (measured faster than 4 on the 8B projections:
// the q / k / v launch 9.0 against 10.0 us, o 5.5 against 5.9 us), 4 where
// 2 would need more than RD_MAXW waves
static int rd_spw(int64_t K) { return K / 256 / 2 <= RD_MAXW ? 2 : 4; }

bool rd_take(const int* dts, const int64_t* Ns, const int* rpts, int nseg, int64_t K, int64_t M,
             int epi, int cu_count) {
    if (epi == EPI_SWIGLU || nseg < 1 || nseg > 3) return false;
    int64_t units = 0;
    for (int i = 0; i < nseg; ++i) {
        if (!rd_supported(dts[i], K, M) || (rpts[i] != 16 && rpts[i] != 32)) return false;
        units += (Ns[i] + rpts[i] - 1) / rpts[i] * (rpts[i] / 16);
    }
    // one round of resident waves: every wave loads all its operands at
    // entry and holds them, so a launch of several rounds exposes each
    // round's latency (the SwiGLU pairs and the LM head keep k_mv's
    // streaming ring: 14.8 against 18.6 us and 86 against 116 us measured)
    const int64_t W = K / 256 / rd_spw(K);
    const int64_t cus = cu_count > 0 ? cu_count : 256;
    return units * W <= cus * 16;
}

hipError_t launch_rd(hipStream_t st, const GemvSeg* segs, int nseg, const int8_t* xq, int64_t K,
                     int64_t M, int epi, int normed, float eps, const QkvEpi* qkv) {
    if (epi == EPI_QKV && (!qkv || nseg != 3 || qkv->hd % 2)) return hipErrorInvalidValue;
    if (nseg < 1 || nseg > 3 || M < 1 || M > 8 || K % 512 || K > 8192)
        return hipErrorInvalidValue;
    const bool pair = epi == EPI_SWIGLU;
    if (pair && (nseg != 2 || segs[0].N != segs[1].N || segs[0].dt != segs[1].dt ||
                 segs[0].rpt != segs[1].rpt))
        return hipErrorInvalidValue;
    RdArgs a{};
    int64_t units = 0;
    for (int i = 0; i < nseg; ++i) {
        if (!segs[i].tiled || (segs[i].rpt != 16 && segs[i].rpt != 32) ||
            (segs[i].dt != FTX_Q4_K && segs[i].dt != FTX_Q6_K))
            return hipErrorInvalidValue;
        RdSeg& sg = a.seg[a.nseg++];
        sg.W = segs[i].W;
        sg.N = segs[i].N;
        sg.u0 = pair ? 0 : units;
        sg.y = segs[i].y;
        sg.ldy = segs[i].ldy;
        sg.R = segs[i].rpt;
        sg.dt = segs[i].dt;
        sg.role = i;
        // 16-row units, whole tiles (the tiled copy pads the last tile)
        const int64_t su = (segs[i].N + segs[i].rpt - 1) / segs[i].rpt * (segs[i].rpt / 16);
        if (!pair || i == 0) units += su;
    }
    a.units = units;
    a.nsb = (int)(K / 256);
    a.M = (int)M;
    a.epi = epi;
    const XqPtrs p = xq_ptrs(const_cast<int8_t*>(xq), K);
    a.frag = p.frag;
    a.xs32 = p.xs32;
    a.xs16 = p.xs16;
    a.scale = p.scale;
    a.ssq = normed ? p.ssq : nullptr;
    a.eps = eps;
    a.K = K;
    if (qkv) a.qkv = *qkv;
    const int spw = rd_spw(K);
    const int W = a.nsb / spw;
    if (W > RD_MAXW) return hipErrorInvalidValue;
    a.W = W;
    using K_t = void (*)(RdArgs);
    const K_t kf = spw == 4 ? (pair ? k_rd<true, 4, 512> : k_rd<false, 4, 512>)
                            : (pair ? k_rd<true, 2, 512> : k_rd<false, 2, 512>);
    // at least two waves a unit for the epilogue's 128 threads (a row of
    // two super-blocks: one wave computes, both store)
    ktimed_launch(kf, dim3((unsigned)units), dim3(64 * (W < 2 ? 2 : W)), 0, st, a);
    return hipGetLastError();
}
