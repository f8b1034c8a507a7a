// k_moe.hip -- the mixture-of-experts FFN of the verify step
// (Impl::moe_ffn, src/engine.cpp:179-258) on the device, all experts
// resident:
//   route    the router rows -> softmax, top-U, renormalised weights, the
//            experts' first-use order and, per expert, its tokens in token
//            order, laid out as 64-row tiles of one expert each (a tile
//            table that the expert GEMMs walk without a host round trip);
//   gate/up  k_gemm.hip's one-pass GEMM over the gathered rows, tile by tile,
//            with SwiGLU into the down operand (launch_mm_experts);
//   down     the experts' ffn_down (reference orientation, n_ff rows of
//            n_embd columns, Q4_0 blocks along the columns) on
//            v_mfma_f32_16x16x32_f16 over a re-tiled copy (below);
//   combine  tmpo[m] = sum over token m's experts, in first-use order, of
//            weight * row (src/engine.cpp:232-239), added into x or stored.
//
// The down GEMM.  y[s][j] = sum_i h[s][i] d[i][b(j)] (q[i][j] - 8): the
// block scale runs along the contraction, so it cannot be applied to the
// MFMA outputs; it is folded into the weight operand instead, exactly: d =
// d_hi + d_lo with d_hi the top 8 significant bits of d (the low 3 mantissa
// bits cleared) and d_lo the rest, so that d_hi (q - 8) (<= 11 bits) and
// d_lo (q - 8) (<= 6 bits) are both exact in fp16.  With h = h_hi + h_lo
// (fp16 hi / lo) a product takes three MFMAs: h_hi B_hi + h_lo B_hi + h_hi
// B_lo (h_lo B_lo is below 2^-19 of the product and dropped).  Small
// values reach these operands as fp16 subnormals (h_lo, d_lo (q - 8)),
// which this MFMA multiplies exactly on gfx950 (checked on the device:
// subnormal B times ones sums to the exact multiple), so no operand is
// rescaled.
// Re-tiled copy, per expert plane, per 64-column pair of Q4_0 blocks P and
// 32-row group g, 1152 bytes (the same bytes as the 32 rows' two blocks):
//   [lane 0..63][column tile c 0..3] 4 bytes: the 8 nibbles of rows 32 g +
//     8 (lane / 16) + t, t = 0..7, column 64 P + 16 c + lane % 16, slot t at
//     byte t % 4, nibble t / 4 (the operand order of nib8);
//   [block 0..1][row 0..31] fp16 d of the block's rows.
// Tiles of one P are consecutive in g, so a wave streams 1152 contiguous
// bytes per 32 rows.
#include "ftx_internal.h"
#include "mm_dev.h"
#include "quant_dev.h"

#include <climits>

namespace {

constexpr int MOE_TILE = 64;   // operand rows per tile (the k_mm token tile)
constexpr int MOE_MAXM = 256;  // tokens of one step
constexpr int MOE_MAXE = 256;  // experts
constexpr int MOE_MAXU = 8;    // experts per token
constexpr int MOE_TB = 1152;   // bytes of one re-tiled (pair-block, row-group) tile

// ---------------------------------------------------------------- route
// One workgroup.  Thread m (strided) takes token m: router row plus bias,
// softmax_inplace (float max, float exp, double sum, float scale;
// src/engine.cpp:62-72), the U largest in descending order with ties to the
// lower index (std::partial_sort's order for distinct values), the weights
// renormalised by their float sum (src/engine.cpp:201-215).  Then thread e
// (strided) takes expert e: first use and token count; thread 0 lays out
// the tiles (experts in index order, ceil(count / 64) tiles each); thread e
// assigns its tokens' operand rows in token order; thread m orders its
// experts by first use for the combine.
__global__ void __launch_bounds__(256) k_moe_route(float* __restrict__ router,
                                                   const float* __restrict__ rbias, int M, int E,
                                                   int U, int ntile_max, MoeRoute r) {
#pragma clang fp contract(off)
    __shared__ int te[MOE_MAXM * MOE_MAXU];
    __shared__ float tw[MOE_MAXM * MOE_MAXU];
    __shared__ int slot_of[MOE_MAXM * MOE_MAXU];
    __shared__ int firstpos[MOE_MAXE], cnt[MOE_MAXE], tile0[MOE_MAXE], rank[MOE_MAXE];
    const int t = threadIdx.x;
    const int MU = M * U;
    for (int m = t; m < M; m += blockDim.x) {
        float* p = router + (int64_t)m * E;
        if (rbias)
            for (int j = 0; j < E; ++j) p[j] = p[j] + rbias[j];
        float mx = p[0];
        for (int j = 1; j < E; ++j) mx = fmaxf(mx, p[j]);
        double sum = 0.0;
        for (int j = 0; j < E; ++j) {
            const float e = expf(p[j] - mx);
            p[j] = e;
            sum += (double)e;
        }
        const float inv = (float)(1.0 / sum);
        for (int j = 0; j < E; ++j) p[j] = p[j] * inv;
        int* top = te + m * U;
        for (int u = 0; u < U; ++u) {
            int best = -1;
            float bv = 0.f;
            for (int j = 0; j < E; ++j) {
                bool taken = false;
                for (int v = 0; v < u; ++v) taken |= top[v] == j;
                if (taken) continue;
                const float pj = p[j];
                if (best < 0 || pj > bv) {
                    best = j;
                    bv = pj;
                }
            }
            top[u] = best;
        }
        float wsum = 0.f;
        for (int u = 0; u < U; ++u) wsum = wsum + p[top[u]];
        const float winv = wsum > 0.f ? 1.f / wsum : 0.f;
        for (int u = 0; u < U; ++u) tw[m * U + u] = p[top[u]] * winv;
    }
    __syncthreads();
    for (int e = t; e < E; e += blockDim.x) {
        int fp = INT_MAX, c = 0;
        for (int i = 0; i < MU; ++i)
            if (te[i] == e) {
                if (fp == INT_MAX) fp = i;
                ++c;
            }
        firstpos[e] = fp;
        cnt[e] = c;
    }
    for (int i = t; i < ntile_max * MOE_TILE; i += blockDim.x) r.slot_tok[i] = -1;
    __syncthreads();
    for (int e = t; e < E; e += blockDim.x) {
        int k = 0;
        for (int e2 = 0; e2 < E; ++e2) k += firstpos[e2] < firstpos[e];
        rank[e] = k;
    }
    if (t == 0) {
        int nt = 0;
        for (int e = 0; e < E; ++e) {
            tile0[e] = nt;
            for (int k = 0; k < cnt[e] && nt < ntile_max; k += MOE_TILE, ++nt) {
                r.tab[1 + 2 * nt] = e;
                r.tab[2 + 2 * nt] = min(MOE_TILE, cnt[e] - k);
            }
        }
        r.tab[0] = nt;
    }
    __syncthreads();
    for (int e = t; e < E; e += blockDim.x) {
        if (!cnt[e]) continue;
        const int base = MOE_TILE * tile0[e];
        int k = 0;
        for (int i = 0; i < MU; ++i)
            if (te[i] == e) {
                const int s = base + k < ntile_max * MOE_TILE ? base + k : 0;
                slot_of[i] = s;
                r.slot_tok[s] = i / U;
                ++k;
            }
    }
    __syncthreads();
    for (int m = t; m < M; m += blockDim.x) {
        int idx[MOE_MAXU];
        for (int u = 0; u < U; ++u) idx[u] = m * U + u;
        for (int u = 1; u < U; ++u)  // insertion sort by first-use rank
            for (int v = u; v > 0 && rank[te[idx[v]]] < rank[te[idx[v - 1]]]; --v) {
                const int x = idx[v];
                idx[v] = idx[v - 1];
                idx[v - 1] = x;
            }
        for (int k = 0; k < U; ++k) {
            r.comb_slot[m * U + k] = slot_of[idx[k]];
            r.comb_w[m * U + k] = tw[idx[k]];
        }
    }
}

// ---------------------------------------------------------------- down
// One thread per 4-byte nibble word or per fp16 scale of the re-tiled copy.
__global__ void __launch_bounds__(256) k_moe_down_tile(const uint8_t* __restrict__ src,
                                                       int64_t F, int64_t K, int64_t E,
                                                       uint8_t* __restrict__ dst) {
    const int64_t G = F / 32, NP = K / 64, rb = K / 32 * 18;
    const int64_t per_tile = 256 + 64;  // nibble words, then scales
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= E * NP * G * per_tile) return;
    const int64_t tile = id / per_tile, w = id % per_tile;
    const int64_t e = tile / (NP * G), P = (tile / G) % NP, g = tile % G;
    const uint8_t* plane = src + e * F * rb;
    uint8_t* out = dst + tile * MOE_TB;
    if (w < 256) {
        const int lane = (int)(w / 4), c = (int)(w % 4);
        const int64_t j = 64 * P + 16 * c + (lane & 15);
        const int64_t b = j / 32, k = j % 32;
        uint32_t word = 0;
        for (int s = 0; s < 8; ++s) {
            const int64_t i = 32 * g + 8 * (lane >> 4) + s;
            const uint8_t byte = plane[i * rb + b * 18 + 2 + k / 2];
            const uint32_t q = (k & 1) ? (byte >> 4) : (byte & 15);
            word |= q << (8 * (s % 4) + 4 * (s / 4));
        }
        *(uint32_t*)(out + lane * 16 + c * 4) = word;
    } else {
        const int hw = (int)(w - 256), blk = hw / 32, rr = hw % 32;
        const int64_t i = 32 * g + rr, b = 2 * P + blk;
        const uint8_t* s = plane + i * rb + b * 18;
        out[1024 + hw * 2] = s[0];
        out[1024 + hw * 2 + 1] = s[1];
    }
}

struct MoeDownArgs {
    const uint8_t* W;     // re-tiled copy of all planes
    int64_t plane;        // bytes per expert
    const _Float16 *ah, *al;
    const int32_t* xtab;
    int64_t F, K, rows;   // rows: operand rows (ntile_max * 64)
    int g_per_split;
    float* part;          // [S][rows][K]
};

struct MoeDownOps {
    v4i nib;      // this lane's nibble words of the four column tiles
    v4i s0, s1;   // d of its 8 rows in block 0 and block 1
    v8h ah[4], al[4];
};

// grid = (K / 256, ntile_max, S); block = 256: wave w owns the pair-block
// P = 4 bx + w (64 columns, four 16-column MFMA tiles) for the tile's rows
// in use (16-row MFMA tiles, a block-uniform count) over its split's row
// groups; the next row group's operands are loaded while the current one's
// are multiplied.
__global__ void __launch_bounds__(256) k_moe_down(MoeDownArgs a) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int by = blockIdx.y;
    if (by >= a.xtab[0]) return;
    const int ex = a.xtab[1 + 2 * by], nv = a.xtab[2 + 2 * by];
    const int nsub = (nv + 15) >> 4;
    const int64_t G = a.F / 32;
    const int64_t g0 = (int64_t)blockIdx.z * a.g_per_split;
    const int64_t g1 = min(g0 + (int64_t)a.g_per_split, G);
    const int64_t P = 4 * (int64_t)blockIdx.x + w;
    const uint8_t* tb = a.W + ex * a.plane + P * G * MOE_TB;
    // fragment (mt, g) of the operand at ((mt * G + g) * 64 + lane) * 8
    const int64_t mt0 = (int64_t)by * 4;
    auto load = [&](MoeDownOps& o, int64_t g) {
        const uint8_t* t = tb + g * MOE_TB;
        o.nib = *(const v4i*)(t + lane * 16);
        o.s0 = *(const v4i*)(t + 1024 + 16 * kq);
        o.s1 = *(const v4i*)(t + 1088 + 16 * kq);
#pragma unroll
        for (int ms = 0; ms < 4; ++ms) {
            if (ms >= nsub) break;
            const int64_t f = (((mt0 + ms) * G + g) * 64 + lane) * 8;
            o.ah[ms] = ld8h(a.ah + f);
            o.al[ms] = ld8h(a.al + f);
        }
    };
    v4f acc[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int ms = 0; ms < 4; ++ms) acc[c][ms] = v4f{0.f, 0.f, 0.f, 0.f};
    MoeDownOps cur, nxt;
    if (g0 < g1) load(cur, g0);
    for (int64_t g = g0; g < g1; ++g) {
        if (g + 1 < g1) load(nxt, g + 1);
        const v4i hmask = {(int)0xFFF8FFF8u, (int)0xFFF8FFF8u, (int)0xFFF8FFF8u, (int)0xFFF8FFF8u};
        const v8h d0 = __builtin_bit_cast(v8h, cur.s0), d1 = __builtin_bit_cast(v8h, cur.s1);
        const v8h d0h = __builtin_bit_cast(v8h, cur.s0 & hmask), d1h = __builtin_bit_cast(v8h, cur.s1 & hmask);
        const v8h d0l = d0 - d0h, d1l = d1 - d1h;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const v8h q = nib8((uint32_t)cur.nib[c], 8.f);
            const v8h bh = q * (c < 2 ? d0h : d1h);
            const v8h bl = q * (c < 2 ? d0l : d1l);
#pragma unroll
            for (int ms = 0; ms < 4; ++ms) {
                if (ms >= nsub) break;
                acc[c][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.ah[ms], bh, acc[c][ms], 0, 0, 0);
                acc[c][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.al[ms], bh, acc[c][ms], 0, 0, 0);
                acc[c][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.ah[ms], bl, acc[c][ms], 0, 0, 0);
            }
        }
        if (g + 1 < g1) cur = nxt;
    }
    // lane (col, kq) holds C[4 kq + r][col]: operand row 64 by + 16 ms + 4 kq
    // + r, column 64 P + 16 c + col
    float* base = a.part + (int64_t)blockIdx.z * a.rows * a.K;
#pragma unroll
    for (int ms = 0; ms < 4; ++ms) {
        if (ms >= nsub) break;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rr = 16 * ms + 4 * kq + r;
            if (rr >= nv) continue;
            float* y = base + ((int64_t)by * MOE_TILE + rr) * a.K + 64 * P + col;
#pragma unroll
            for (int c = 0; c < 4; ++c) y[16 * c] = acc[c][ms][r];
        }
    }
}

// ---------------------------------------------------------------- combine
// grid = (ceil(K / 256), M); token m, column j: t = sum_k w_k a_k in the
// token's first-use order with a_k = sum_s part[s][slot_k][j] (fp32, the
// products rounded before each add as trow[j] += wgt * arow[j]).
__global__ void __launch_bounds__(256) k_moe_combine(const float* __restrict__ part, int S,
                                                     int64_t rows, int64_t K, MoeRoute r, int U,
                                                     float* __restrict__ y, int accum) {
#pragma clang fp contract(off)
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t m = blockIdx.y;
    if (j >= K) return;
    float t = 0.f;
    for (int k = 0; k < U; ++k) {
        const int64_t s = r.comb_slot[m * U + k];
        float acb = 0.f;
        for (int q = 0; q < S; ++q) acb += part[((int64_t)q * rows + s) * K + j];
        t = t + r.comb_w[m * U + k] * acb;
    }
    float* yp = y + m * K + j;
    *yp = accum ? *yp + t : t;
}

__global__ void __launch_bounds__(256) k_add(const float* __restrict__ x, float* __restrict__ y,
                                             int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = y[i] + x[i];
}

}  // namespace

int64_t moe_tiles_max(int64_t M, int64_t E, int64_t U) {
    // sum_e ceil(c_e / 64) <= (M U) / 64 + (experts in use)
    const int64_t MU = M * U;
    return (MU + MOE_TILE - 1) / MOE_TILE + std::min(E, MU);
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t moe_route_bytes(int64_t Mmax, int64_t E, int64_t U) {
    const int64_t T = moe_tiles_max(Mmax, E, U);
    return align256((size_t)(1 + 2 * T) * 4) + align256((size_t)(T * MOE_TILE) * 4) +
           align256((size_t)(Mmax * U) * 4) * 2;
}

MoeRoute moe_route_view(void* buf, int64_t Mmax, int64_t E, int64_t U) {
    const int64_t T = moe_tiles_max(Mmax, E, U);
    uint8_t* p = (uint8_t*)buf;
    MoeRoute r;
    r.tab = (int32_t*)p;
    p += align256((size_t)(1 + 2 * T) * 4);
    r.slot_tok = (int32_t*)p;
    p += align256((size_t)(T * MOE_TILE) * 4);
    r.comb_slot = (int32_t*)p;
    p += align256((size_t)(Mmax * U) * 4);
    r.comb_w = (float*)p;
    return r;
}

hipError_t launch_moe_route(hipStream_t st, float* router, const float* rbias, int64_t M,
                            int64_t E, int64_t U, const MoeRoute& r) {
    if (M < 1 || M > MOE_MAXM || E < 2 || E > MOE_MAXE || U < 1 || U > MOE_MAXU || U > E)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(256), 0, st, router, rbias, (int)M, (int)E,
                       (int)U, (int)moe_tiles_max(M, E, U), r);
    return hipGetLastError();
}

bool moe_down_supported(int dt, int64_t F, int64_t K) {
    return dt == FTX_Q4_0 && F % 32 == 0 && K % 256 == 0 && F >= 32;
}

size_t moe_down_tiled_bytes(int dt, int64_t F, int64_t K, int64_t E) {
    (void)dt;
    return (size_t)(E * (K / 64) * (F / 32)) * MOE_TB;
}

hipError_t launch_moe_down_tile(hipStream_t st, const uint8_t* src, int dt, int64_t F, int64_t K,
                                int64_t E, uint8_t* dst) {
    if (!moe_down_supported(dt, F, K) || E < 1) return hipErrorInvalidValue;
    const int64_t n = E * (K / 64) * (F / 32) * (256 + 64);
    hipLaunchKernelGGL(k_moe_down_tile, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src,
                       F, K, E, dst);
    return hipGetLastError();
}

// splits of the n_ff rows so that the launch holds about four workgroups
// per CU, at least 8 row groups per split
int moe_down_splits(int64_t F, int64_t K, int64_t ntile_max, int cu_count) {
    const int64_t cus = cu_count > 0 ? cu_count : 256;
    const int64_t wgs = (K / 256) * ntile_max;
    int64_t S = (4 * cus + wgs - 1) / wgs;
    const int64_t G = F / 32;
    if (S > G / 8) S = G / 8;
    if (S > 32) S = 32;
    return S < 1 ? 1 : (int)S;
}

hipError_t launch_moe_down(hipStream_t st, const uint8_t* tiled, int dt, int64_t F, int64_t K,
                           const _Float16* ah, const _Float16* al, const int32_t* xtab,
                           int64_t ntile_max, int S, float* part, size_t part_floats) {
    if (!moe_down_supported(dt, F, K) || ntile_max < 1 || S < 1 ||
        (size_t)S * (size_t)(ntile_max * MOE_TILE) * (size_t)K > part_floats)
        return hipErrorInvalidValue;
    MoeDownArgs a{};
    a.W = tiled;
    a.ah = ah;
    a.al = al;
    a.xtab = xtab;
    a.F = F;
    a.K = K;
    a.rows = ntile_max * MOE_TILE;
    a.part = part;
    const int64_t G = F / 32;
    a.g_per_split = (int)((G + S - 1) / S);
    // the real split count: splits past the last row group would leave
    // their partial rows unwritten
    if ((int64_t)a.g_per_split * (S - 1) >= G) return hipErrorInvalidValue;
    a.plane = (K / 64) * G * MOE_TB;
    hipLaunchKernelGGL(k_moe_down, dim3((unsigned)(K / 256), (unsigned)ntile_max, (unsigned)S),
                       dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_moe_combine(hipStream_t st, const float* part, int S, int64_t rows, int64_t K,
                              const MoeRoute& r, int64_t M, int64_t U, float* y, int accum) {
    if (M < 1 || K < 1 || S < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((K + 255) / 256), (unsigned)M), dim3(256), 0,
                       st, part, S, rows, K, r, (int)U, y, accum);
    return hipGetLastError();
}

hipError_t launch_add(hipStream_t st, const float* x, float* y, int64_t n) {
    if (n < 1) return hipSuccess;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
    return hipGetLastError();
}
