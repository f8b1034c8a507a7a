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

constexpr int MOE_MAXM = 256;  // tokens of one step
constexpr int MOE_MAXE = 256;  // experts
constexpr int MOE_MAXU = 8;    // experts per token
constexpr int MOE_TB = 1152;   // bytes of one re-tiled (pair-block, row-group) tile
constexpr int MOE_GB = 4;      // 4096-element batches of a router row (n_embd <= 16384)

// ---------------------------------------------------------------- route
// ffn_norm, router and per-token choice, one workgroup per token m: the
// RMSNorm of the residual row (src/engine.cpp:23-41; the row's sum of
// squares as wave sums), written out as the experts' operand row xn[m]; the
// router row (router weights dot xn[m], any stored dtype, wave sums) plus
// the bias; then softmax_inplace (float max, float exp, double sum in
// expert order, float scale; src/engine.cpp:62-72), the U largest in
// descending order with ties to the lower index (std::partial_sort's order
// for distinct values), the weights renormalised by their float sum
// (src/engine.cpp:197-215).  Writes te[m][u] (expert), tw[m][u] (weight).
// Every load of the launch's first phase goes out at entry (the bias, the
// row and its norm weights, then the first eight router rows, which arrive
// while the row is normalised), and the barriers order LDS only, so no
// phase waits for the xn stores to complete.
__device__ void moe_route_wg(const int32_t* __restrict__ te_g, const float* __restrict__ tw_g,
                             int M, int E, int U, int ntile_max, int TR, const MoeRoute& r);

// Workgroup barrier that orders LDS accesses only: each wave waits for its
// own LDS operations, not (as __syncthreads' release fence does) for every
// global store it has in flight, which costs a memory round trip.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// NB = the row's 4096-element batches, ceil(K / 4096) <= MOE_GB
template <int NB>
__global__ void __launch_bounds__(256) k_moe_gate(const float* __restrict__ x, int64_t K,
                                                  const float* __restrict__ normw, float eps,
                                                  float* __restrict__ xn,
                                                  const uint8_t* __restrict__ W, int dt,
                                                  int64_t row_bytes, const float* __restrict__ rbias,
                                                  int E, int U, int ntile_max, int TR, MoeRoute r) {
#pragma clang fp contract(off)
    int32_t* __restrict__ te = r.te;
    float* __restrict__ tw = r.tw;
    extern __shared__ float xs[];  // [K] then the E logits
    __shared__ float red[4];
    float* lg = xs + K;
    const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const float* xr = x + (int64_t)m * K;
    // the bias of expert `lane` (read by the softmax of E <= 64 experts;
    // without a bias the load reads the row, in bounds, and is replaced by
    // zero)
    const float* rbp = rbias ? rbias : xr;
    float rbv = rbp[min(lane, (rbias ? E : (int)min((int64_t)E, K)) - 1)];
    if (!rbias) rbv = 0.f;
    // 16 elements per thread with their loads in flight together (element
    // order per thread as a plain strided loop)
    // (the norm weights' loads go out with the row's and wait in registers:
    // K <= 256 * 16 * NB)
    float xv[NB][16], nv[NB][16];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int64_t k0 = t + (int64_t)b * 256 * 16;
        if (k0 >= K) break;  // block-uniform for all but the last batch's tail
#pragma unroll
        for (int i = 0; i < 16; ++i) xv[b][i] = xr[min(k0 + 256 * i, K - 1)];
#pragma unroll
        for (int i = 0; i < 16; ++i) nv[b][i] = normw[min(k0 + 256 * i, K - 1)];
    }
    // the first eight router rows' first 1024 float4 columns (the F32
    // router's first group), behind the row, with the indices clamped to
    // rows < E and columns < K; another router dtype reads the norm weights
    // instead (16-byte aligned, K floats) and discards them
    const bool f32 = dt == FTX_F32;
    const uint8_t* Wp = f32 ? W : (const uint8_t*)normw;
    const int64_t rstep = f32 ? row_bytes : 0, n4 = K / 4;
    float4 rv[8][4];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const float4* r4 = (const float4*)(Wp + (int64_t)min(r, E - 1) * rstep);
#pragma unroll
        for (int i = 0; i < 4; ++i) rv[r][i] = r4[min((int64_t)t + 256 * i, n4 - 1)];
    }
    float ss = 0.f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int64_t k0 = t + (int64_t)b * 256 * 16;
        if (k0 >= K) break;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (k0 + 256 * i < K) {
                xs[k0 + 256 * i] = xv[b][i];
                ss += xv[b][i] * xv[b][i];
            }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) red[w] = ss;
    lds_barrier();
    const float rinv = 1.f / sqrtf((((red[0] + red[1]) + red[2]) + red[3]) / (float)K + eps);
    // the normed row stays in xv until the workgroup's last step, where it
    // is stored as xn[m]: a store in flight would hold up every later wait
    // for a load (vector-memory counters cover stores too) and the fences
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t k = t + (int64_t)b * 256 * 16 + 256 * i;
            if (k < K) {
                xv[b][i] = xv[b][i] * rinv * nv[b][i];
                xs[k] = xv[b][i];
            }
        }
    auto store_xn = [&]() {
        float* xo = xn + (int64_t)m * K;
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t k = t + (int64_t)b * 256 * 16 + 256 * i;
                if (k < K) xo[k] = xv[b][i];
            }
    };
    lds_barrier();
    if (f32) {
        // groups of 8 router rows: every thread's float4s of the group's
        // rows (4 per row per 4096 columns) in flight together (the first
        // group's since entry); per row, the threads' partial dots summed by
        // wave (shuffles) and then in wave order
        __shared__ float rsum[4][8];
        const float4* x4 = (const float4*)xs;
        for (int e0 = 0; e0 < E; e0 += 8) {
            float acc[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) acc[r] = 0.f;
            for (int64_t p0 = 0; p0 < n4; p0 += 1024) {
                float4 (&v)[8][4] = rv;
                if (e0 > 0 || p0 > 0) {
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const float4* r4 = (const float4*)(W + (int64_t)min(e0 + r, E - 1) * row_bytes);
#pragma unroll
                        for (int i = 0; i < 4; ++i) v[r][i] = r4[min(p0 + t + 256 * i, n4 - 1)];
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t c = p0 + t + 256 * i;
                    if (c < n4) {
                        const float4 xc = x4[c];
#pragma unroll
                        for (int r = 0; r < 8; ++r)
                            acc[r] += v[r][i].x * xc.x + v[r][i].y * xc.y + v[r][i].z * xc.z +
                                      v[r][i].w * xc.w;
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) {
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) acc[r] += __shfl_xor(acc[r], o, 64);
            }
            if (lane == 0)
#pragma unroll
                for (int r = 0; r < 8; ++r) rsum[w][r] = acc[r];
            lds_barrier();
            if (t < 8 && e0 + t < E) lg[e0 + t] = ((rsum[0][t] + rsum[1][t]) + rsum[2][t]) + rsum[3][t];
            lds_barrier();
        }
    } else {
        for (int e = w; e < E; e += 4) {
            const uint8_t* row = W + (int64_t)e * row_bytes;
            float acc = 0.f;
            for (int64_t c = lane; c < K / 8; c += 64) {
                float v[8];
                dq8(row, dt, 8 * c, K, v);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc += v[i] * xs[8 * c + i];
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
            if (lane == 0) lg[e] = acc;
        }
        lds_barrier();
    }
    if (w == 0) {
    int top[MOE_MAXU];
    float topw[MOE_MAXU];
    if (E <= 64) {
    // softmax and top-U on wave 0 for up to 64 experts: lane j holds expert
    // j, and every lane runs one thread's loops over the lanes in expert
    // order (float max, float exp, double sum, float scale); then each lane
    // counts the experts ahead of its own in (probability descending, index
    // ascending) order, and the u-th choice is the lane with u ahead -- the
    // U passes for the largest not yet taken, ties to the lower index
    const float pj = lane < E ? (rbias ? lg[lane] + rbv : lg[lane]) : -INFINITY;
    float mx = -INFINITY;
    for (int j = 0; j < E; ++j) mx = fmaxf(mx, lane_f(pj, j));
    const float ej = lane < E ? expf(pj - mx) : 0.f;
    double sum = 0.0;
    for (int j = 0; j < E; ++j) sum += (double)lane_f(ej, j);
    const float pr = ej * (float)(1.0 / sum);
    int ahead = 0;
    for (int j = 0; j < E; ++j) {
        const float v = lane_f(pr, j);
        ahead += (v > pr) | ((v == pr) & (j < lane));
    }
    for (int u = 0; u < U; ++u) {
        const uint64_t b = __ballot(lane < E && ahead == u);
        const int j = b ? __builtin_ctzll(b) : 0;
        top[u] = j;
        topw[u] = lane_f(pr, j);
    }
    } else {
    // softmax and top-U on wave 0: lane l holds experts l, l + 64, l + 128,
    // l + 192 (E <= 256); the arithmetic and its order as one thread's
    // loops: float max, float exp, double sum in expert order, float scale
    float pv[4];
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int j = lane + 64 * q;
        pv[q] = j < E ? (rbias ? lg[j] + rbias[j] : lg[j]) : -INFINITY;
        mx = fmaxf(mx, pv[q]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
#pragma unroll
    for (int q = 0; q < 4; ++q) pv[q] = lane + 64 * q < E ? expf(pv[q] - mx) : 0.f;
    double sum = 0.0;
    for (int j = 0; j < E; ++j) {
        const float src = j < 64 ? pv[0] : j < 128 ? pv[1] : j < 192 ? pv[2] : pv[3];
        sum += (double)lane_f(src, j & 63);
    }
    const float inv = (float)(1.0 / sum);
#pragma unroll
    for (int q = 0; q < 4; ++q) pv[q] = pv[q] * inv;
    // the U largest, ties to the lower index: U wave reductions of (p, j)
    // over the experts not yet taken (a taken expert's key is -1 < p)
    float key[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) key[q] = lane + 64 * q < E ? pv[q] : -2.f;
    for (int u = 0; u < U; ++u) {
        float bv = key[0];
        int bj = lane;
#pragma unroll
        for (int q = 1; q < 4; ++q)
            if (key[q] > bv) {
                bv = key[q];
                bj = lane + 64 * q;
            }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oj = __shfl_xor(bj, o, 64);
            if (ov > bv || (ov == bv && oj < bj)) {
                bv = ov;
                bj = oj;
            }
        }
        top[u] = bj;
        topw[u] = bv;
        if ((bj & 63) == lane) key[bj >> 6] = -1.f;
    }
    }
    float wsum = 0.f;
    for (int u = 0; u < U; ++u) wsum = wsum + topw[u];
    const float winv = wsum > 0.f ? 1.f / wsum : 0.f;
    if (lane == 0)
        for (int u = 0; u < U; ++u) {
            te[m * U + u] = top[u];
            tw[m * U + u] = topw[u] * winv;
        }
    }
    // The last of the M router workgroups to finish groups the tokens (one
    // launch fewer per MoE layer than a grouping kernel of its own).  Thread
    // 0, which stored this token's choice, publishes it with a device-scope
    // fence before counting the workgroup done; the last one's threads fence
    // again before reading every token's choice.  The counter is back at 0
    // when the launch ends.  (xn[m], which only the next launches read, is
    // stored after all of this.)
    __shared__ int last;
    if (t == 0) {
        __threadfence();
        last = atomicAdd(r.done, 1u) == (unsigned)(gridDim.x - 1);
    }
    lds_barrier();
    if (!last) {  // block-uniform
        store_xn();
        return;
    }
    __threadfence();
    moe_route_wg(te, tw, (int)gridDim.x, E, U, ntile_max, TR, r);
    store_xn();
    if (t == 0) atomicExch(r.done, 0u);
}

// Grouping, by the last router workgroup (src/engine.cpp:210-239).  The
// entries i = (token, rank) are walked in order by wave 0, 64 at a time:
// per distinct expert of a 64-entry chunk one ballot gives its entries'
// places k among the expert's entries so far, its count and its first use.
// Then wave 0 lays out the tiles (experts in index order, ceil(count / TR)
// tiles each, at most ntile_max in all), each expert's first entry slot
// (the prefix sums of counts) and the experts' first-use ranks, and turns
// every entry's k into its operand row.  After one LDS barrier every thread
// writes its share of the row table (each row once: the token of the entry
// that takes it, or -1) and thread m orders token m's experts by first use
// for the combine.
__device__ void moe_route_wg(const int32_t* __restrict__ te_g, const float* __restrict__ tw_g,
                             int M, int E, int U, int ntile_max, int TR, const MoeRoute& r) {
    __shared__ int te[MOE_MAXM * MOE_MAXU];
    __shared__ float tw[MOE_MAXM * MOE_MAXU];
    __shared__ int slot_of[MOE_MAXM * MOE_MAXU];  // k, then the operand row
    __shared__ int ent[MOE_MAXM * MOE_MAXU];      // entries by expert: ent[off[e] + k]
    __shared__ int firstpos[MOE_MAXE], cnt[MOE_MAXE], tile0[MOE_MAXE], off[MOE_MAXE],
        rank[MOE_MAXE];
    __shared__ int tile_e[MOE_MAXM * MOE_MAXU / 16 + 1 + MOE_MAXE];  // expert of each tile
    __shared__ int nt_s;
    const int t = threadIdx.x, lane = t & 63;
    const int MU = M * U;
    for (int i = t; i < MU; i += blockDim.x) {
        te[i] = te_g[i];
        tw[i] = tw_g[i];
    }
    for (int e = t; e < E; e += blockDim.x) {
        cnt[e] = 0;
        firstpos[e] = INT_MAX;
    }
    __syncthreads();
    if (t < 64) {
        // (one wave: its LDS accesses are ordered, so no barrier inside)
        const uint64_t below = (1ull << lane) - 1;
        for (int c0 = 0; c0 < MU; c0 += 64) {
            const int i = c0 + lane;
            const int e = i < MU ? te[i] : -1;
            uint64_t todo = __ballot(i < MU);
            int k = 0;
            while (todo) {
                const int ld = __builtin_ctzll(todo);
                const int el = lane_i(e, ld);
                const uint64_t mk = __ballot(e == el);
                const int base = cnt[el];
                if (e == el) k = base + __popcll(mk & below);
                if (lane == 0) {
                    if (base == 0) firstpos[el] = c0 + ld;
                    cnt[el] = base + __popcll(mk);
                }
                todo &= ~mk;
            }
            if (i < MU) slot_of[i] = k;
        }
        // tiles and entry offsets: exclusive prefix sums over the experts
        // in index order, 64 experts a round
        int ct = 0, cc = 0;
        for (int q = 0; q < E; q += 64) {
            const int e = q + lane;
            const int c = e < E ? cnt[e] : 0;
            const int n = (c + TR - 1) / TR;
            int sn = n, sc = c;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int an = __shfl_up(sn, o, 64), ac = __shfl_up(sc, o, 64);
                if (lane >= o) {
                    sn += an;
                    sc += ac;
                }
            }
            if (e < E) {
                const int t0 = min(ct + sn - n, ntile_max);
                const int nte = min(n, ntile_max - t0);
                tile0[e] = t0;
                off[e] = cc + sc - c;
                for (int j = 0; j < nte; ++j) {
                    r.tab[1 + 2 * (t0 + j)] = e;
                    r.tab[2 + 2 * (t0 + j)] = min(TR, c - j * TR);
                    tile_e[t0 + j] = e;
                }
            }
            ct += lane_i(sn, 63);
            cc += lane_i(sc, 63);
        }
        if (lane == 0) {
            nt_s = min(ct, ntile_max);
            r.tab[0] = min(ct, ntile_max);
        }
        for (int e = lane; e < E; e += 64) {
            const int fp = firstpos[e];
            int k = 0;
            for (int e2 = 0; e2 < E; ++e2) k += firstpos[e2] < fp;
            rank[e] = k;
        }
        for (int i = lane; i < MU; i += 64) {
            const int e = te[i], k = slot_of[i];
            const int s = TR * tile0[e] + k;
            slot_of[i] = s < ntile_max * TR ? s : 0;
            ent[off[e] + k] = i;
        }
    }
    lds_barrier();
    const int nt = nt_s;
    for (int row = t; row < ntile_max * TR; row += blockDim.x) {
        const int tl = row / TR;
        int tok = -1;
        if (tl < nt) {
            const int e = tile_e[tl];
            const int k = (tl - tile0[e]) * TR + row % TR;
            if (k < cnt[e]) tok = ent[off[e] + k] / U;
        }
        r.slot_tok[row] = tok;
    }
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
    int64_t F, K, rows;   // rows: operand rows (ntile_max * trows)
    int trows;            // rows per tile (16 or 64)
    int g_per_split;      // 32-row groups per split, a multiple of the chunk (MOE_CGS)
    float* part;          // [S][rows][K]
};

constexpr int MOE_CG = 8;  // the most row groups a chunk stages (split sizes are multiples)
// row groups per staged chunk: 8 for 16-row routing tiles (more bytes in
// flight per wave; their smaller operand stage leaves the room), 4 for
// 64-row tiles
template <int MS>
constexpr int MOE_CGS = MS == 1 ? 8 : 4;
// LDS per chunk buffer: the operand fragments [ms MS][g][hi / lo][1 KB], then
// the scales of the workgroup's four pair-blocks [P 4][g][2 blocks x 32 rows]
template <int MS>
constexpr int MOE_A_BYTES = MS * MOE_CGS<MS> * 2 * 1024;
template <int MS>
constexpr int MOE_BUF = MOE_A_BYTES<MS> + 4 * MOE_CGS<MS> * 128;

typedef __attribute__((address_space(3))) void moe_lds_void;

// grid = (K / 256, ntile_max, S); block = 256: wave w owns the pair-block
// P = 4 bx + w (64 columns, four 16-column MFMA tiles) for the tile's rows
// in use (16-row MFMA tiles, a block-uniform count) over its split's row
// groups, CG groups at a time.  Per chunk the operand fragments (of the
// rows in use) and the workgroup's scales go to one of two LDS buffers by
// direct loads, and each wave's nibbles to one of two register sets, all
// issued a chunk ahead; one wait and one barrier per chunk.  MS: 16-row
// MFMA tiles per routing tile (4 for 64-row tiles, 1 for 16-row tiles, whose
// smaller LDS and register set let more workgroups share a CU).
template <int MS>
__global__ void __launch_bounds__(256) k_moe_down(MoeDownArgs a) {
    constexpr int CG = MOE_CGS<MS>, BUF = MOE_BUF<MS>, ABYTES = MOE_A_BYTES<MS>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // [2][BUF]
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
    const uint8_t* wb = a.W + ex * a.plane;  // the expert's tiles
    const int64_t P = 4 * (int64_t)blockIdx.x + w;
    const uint8_t* tb = wb + P * G * MOE_TB;  // this wave's pair-block
    const int64_t mt0 = (int64_t)by * (a.trows / 16);
    // a group index for addresses: groups past the split's end (never
    // multiplied) read the last group of the plane
    auto gc = [&](int64_t g) { return g < G ? g : G - 1; };
    auto stage = [&](int64_t c0, int buf, v4i* nib) {
        uint8_t* L = lds + buf * BUF;
        // fragment copies q = w + 4 i over (ms, g, hl), one direct load each
#pragma unroll
        for (int i = 0; i < 2 * CG * MS / 4; ++i) {
            const int q = w + 4 * i;
            const int ms = q / (2 * CG), g = (q / 2) % CG, hl = q & 1;
            if (ms >= nsub || c0 + g >= g1) continue;
            const _Float16* src =
                (hl ? a.al : a.ah) + (((mt0 + ms) * G + c0 + g) * 64 + lane) * 8;
            __builtin_amdgcn_global_load_lds(
                (const void*)src, (moe_lds_void*)(L + ((ms * CG + g) * 2 + hl) * 1024), 16, 0,
                0);
        }
        // scales: waves w < CG / 2, piece p = 64 w + lane -> pair-block
        // p / (8 CG), group (p / 8) % CG, 16 bytes at 16 (p % 8) of the
        // tile's scales
        if (w < CG / 2) {
            const int p = 64 * w + lane;
            const int pw = p / (8 * CG), g = (p / 8) % CG, piece = p % 8;
            const uint8_t* src =
                wb + ((4 * (int64_t)blockIdx.x + pw) * G + gc(c0 + g)) * MOE_TB + 1024 + 16 * piece;
            __builtin_amdgcn_global_load_lds((const void*)src,
                                             (moe_lds_void*)(L + ABYTES + 1024 * w), 16, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < CG; ++g) nib[g] = *(const v4i*)(tb + gc(c0 + g) * MOE_TB + lane * 16);
    };
    v4f acc[4][MS];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) acc[c][ms] = v4f{0.f, 0.f, 0.f, 0.f};
    const v4i hmask = {(int)0xFFF8FFF8u, (int)0xFFF8FFF8u, (int)0xFFF8FFF8u, (int)0xFFF8FFF8u};
    auto compute = [&](int64_t c0, int buf, const v4i* nib) {
        const uint8_t* L = lds + buf * BUF;
#pragma unroll
        for (int g = 0; g < CG; ++g) {
            if (c0 + g >= g1) break;
            const uint8_t* sc = L + ABYTES + (w * CG + g) * 128 + 16 * kq;
            const v4i s0 = *(const v4i*)sc, s1 = *(const v4i*)(sc + 64);
            const v8h d0 = __builtin_bit_cast(v8h, s0), d1 = __builtin_bit_cast(v8h, s1);
            const v8h d0h = __builtin_bit_cast(v8h, s0 & hmask);
            const v8h d1h = __builtin_bit_cast(v8h, s1 & hmask);
            const v8h d0l = d0 - d0h, d1l = d1 - d1h;
            v8h ah[MS], al[MS];
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                if (ms >= nsub) break;
                ah[ms] = *(const v8h*)(L + ((ms * CG + g) * 2 + 0) * 1024 + lane * 16);
                al[ms] = *(const v8h*)(L + ((ms * CG + g) * 2 + 1) * 1024 + lane * 16);
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const v8h q = nib8((uint32_t)nib[g][c], 8.f);
                const v8h bh = q * (c < 2 ? d0h : d1h);
                const v8h bl = q * (c < 2 ? d0l : d1l);
#pragma unroll
                for (int ms = 0; ms < MS; ++ms) {
                    if (ms >= nsub) break;
                    acc[c][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ms], bh, acc[c][ms], 0, 0, 0);
                    acc[c][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[ms], bh, acc[c][ms], 0, 0, 0);
                    acc[c][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ms], bl, acc[c][ms], 0, 0, 0);
                }
            }
        }
    };
    v4i na[CG], nb[CG];
    if (g0 < g1) stage(g0, 0, na);
    for (int64_t c0 = g0; c0 < g1; c0 += 2 * CG) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // this chunk's copies and nibbles
        __syncthreads();                     // every wave is done with the other buffer
        if (c0 + CG < g1) stage(c0 + CG, 1, nb);
        compute(c0, 0, na);
        if (c0 + CG >= g1) break;
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        if (c0 + 2 * CG < g1) stage(c0 + 2 * CG, 0, na);
        compute(c0 + CG, 1, nb);
    }
    // lane (col, kq) holds C[4 kq + r][col]: operand row 64 by + 16 ms + 4 kq
    // + r, column 64 P + 16 c + col
    float* base = a.part + (int64_t)blockIdx.z * a.rows * a.K;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        if (ms >= nsub) break;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rr = 16 * ms + 4 * kq + r;
            if (rr >= nv) continue;
            float* y = base + ((int64_t)by * a.trows + rr) * a.K + 64 * P + col;
#pragma unroll
            for (int c = 0; c < 4; ++c) y[16 * c] = acc[c][ms][r];
        }
    }
}

// ---------------------------------------------------------------- combine
// grid = (ceil(K / 256), M); token m, column j: t = sum_k w_k a_k in the
// token's first-use order with a_k = sum_s part[s][slot_k][j] (fp32, the
// products rounded before each add as trow[j] += wgt * arow[j]).  The
// output (when accumulating) and the token's slots and weights are loaded
// first, then the partials of every expert, eight splits at a time, all in
// flight together (indices clamped, the surplus masked); UM >= U.
template <int UM>
__global__ void __launch_bounds__(256) k_moe_combine(const float* __restrict__ part, int S,
                                                     int64_t rows, int64_t K, MoeRoute r, int U,
                                                     float* __restrict__ y, int accum) {
#pragma clang fp contract(off)
    constexpr int QB = 8;  // splits per batch
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t m = blockIdx.y;
    if (j >= K) return;
    float* yp = y + m * K + j;
    const float y0 = *yp;  // (read whether or not it is used: in bounds)
    int64_t slot[UM];
    float wk[UM];
#pragma unroll
    for (int k = 0; k < UM; ++k) {
        const int64_t e = m * U + min(k, U - 1);
        slot[k] = r.comb_slot[e];
        wk[k] = r.comb_w[e];
    }
    float acb[UM];
#pragma unroll
    for (int k = 0; k < UM; ++k) acb[k] = 0.f;
    for (int q0 = 0; q0 < S; q0 += QB) {
        float pv[UM][QB];
#pragma unroll
        for (int k = 0; k < UM; ++k)
#pragma unroll
            for (int i = 0; i < QB; ++i)
                pv[k][i] = part[((int64_t)min(q0 + i, S - 1) * rows + slot[k]) * K + j];
#pragma unroll
        for (int k = 0; k < UM; ++k)
#pragma unroll
            for (int i = 0; i < QB; ++i)
                if (q0 + i < S) acb[k] += pv[k][i];
    }
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < UM; ++k)
        if (k < U) t = t + wk[k] * acb[k];
    *yp = accum ? y0 + t : t;
}

__global__ void __launch_bounds__(256) k_add(const float* __restrict__ x, float* __restrict__ y,
                                             int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = y[i] + x[i];
}

}  // namespace

int64_t moe_tile_rows(int64_t M, int64_t E, int64_t U) {
    // 16-row tiles while the average expert takes at most 16 rows (each
    // plane is then read about once either way, and the small tiles waste
    // no MFMA work), 64-row tiles beyond that (fewer re-reads of a plane)
    return M * U <= 16 * E ? 16 : 64;
}

int64_t moe_tiles_max(int64_t M, int64_t E, int64_t U) {
    // sum_e ceil(c_e / TR) <= (M U) / TR + (experts in use)
    const int64_t MU = M * U, TR = moe_tile_rows(M, E, U);
    return (MU + TR - 1) / TR + std::min(E, MU);
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// the largest tile table and operand row count of any step up to Mmax tokens
static void moe_max_dims(int64_t Mmax, int64_t E, int64_t U, int64_t* tiles, int64_t* rows) {
    *tiles = *rows = 0;
    for (int64_t m = 1; m <= Mmax; ++m) {
        const int64_t t = moe_tiles_max(m, E, U);
        *tiles = std::max(*tiles, t);
        *rows = std::max(*rows, t * moe_tile_rows(m, E, U));
    }
}

int64_t moe_rows_max(int64_t Mmax, int64_t E, int64_t U) {
    int64_t t, r;
    moe_max_dims(Mmax, E, U, &t, &r);
    return r;
}

size_t moe_route_bytes(int64_t Mmax, int64_t E, int64_t U) {
    int64_t T, R;
    moe_max_dims(Mmax, E, U, &T, &R);
    return align256((size_t)(1 + 2 * T) * 4) + align256((size_t)R * 4) +
           align256((size_t)(Mmax * U) * 4) * 4 + 256;
}

MoeRoute moe_route_view(void* buf, int64_t Mmax, int64_t E, int64_t U) {
    int64_t T, R;
    moe_max_dims(Mmax, E, U, &T, &R);
    uint8_t* p = (uint8_t*)buf;
    MoeRoute r;
    r.tab = (int32_t*)p;
    p += align256((size_t)(1 + 2 * T) * 4);
    r.slot_tok = (int32_t*)p;
    p += align256((size_t)R * 4);
    r.comb_slot = (int32_t*)p;
    p += align256((size_t)(Mmax * U) * 4);
    r.comb_w = (float*)p;
    p += align256((size_t)(Mmax * U) * 4);
    r.te = (int32_t*)p;
    p += align256((size_t)(Mmax * U) * 4);
    r.tw = (float*)p;
    p += align256((size_t)(Mmax * U) * 4);
    r.done = (uint32_t*)p;
    return r;
}

hipError_t launch_moe_route(hipStream_t st, const float* x, const float* normw, float eps,
                            float* xn, int64_t K, const uint8_t* W, int dt, int64_t row_bytes,
                            const float* rbias, int64_t M, int64_t E, int64_t U,
                            const MoeRoute& r) {
    if (M < 1 || M > MOE_MAXM || E < 2 || E > MOE_MAXE || U < 1 || U > MOE_MAXU || U > E ||
        K < 8 || K % 8 || K > 256 * 16 * MOE_GB || (K + E) * 4 > 65536 ||
        (dt == FTX_F32 && ((uintptr_t)W & 15)) || (dt == FTX_F32 && row_bytes % 16))
        return hipErrorInvalidValue;
    const size_t lds = (size_t)(K + E) * sizeof(float);
    const int nb = (int)((K + 4095) / 4096);
    auto kern = nb == 1 ? k_moe_gate<1> : nb == 2 ? k_moe_gate<2> : nb == 3 ? k_moe_gate<3> : k_moe_gate<4>;
    hipLaunchKernelGGL(kern, dim3((unsigned)M), dim3(256), lds, st, x, K, normw, eps, xn, W,
                       dt, row_bytes, rbias, (int)E, (int)U, (int)moe_tiles_max(M, E, U),
                       (int)moe_tile_rows(M, E, U), r);
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
    if (S < 1) S = 1;
    // every split a whole number of chunks, and none empty
    const int64_t per = ((G + S - 1) / S + MOE_CG - 1) / MOE_CG * MOE_CG;
    return (int)((G + per - 1) / per);
}

hipError_t launch_moe_down(hipStream_t st, const uint8_t* tiled, int dt, int64_t F, int64_t K,
                           const _Float16* ah, const _Float16* al, const int32_t* xtab,
                           int64_t ntile_max, int64_t trows, int S, float* part,
                           size_t part_floats) {
    if (!moe_down_supported(dt, F, K) || ntile_max < 1 || S < 1 || (trows != 16 && trows != 64) ||
        (size_t)S * (size_t)(ntile_max * trows) * (size_t)K > part_floats)
        return hipErrorInvalidValue;
    MoeDownArgs a{};
    a.W = tiled;
    a.ah = ah;
    a.al = al;
    a.xtab = xtab;
    a.F = F;
    a.K = K;
    a.rows = ntile_max * trows;
    a.trows = (int)trows;
    a.part = part;
    const int64_t G = F / 32;
    const int cg = trows == 16 ? MOE_CGS<1> : MOE_CGS<4>;
    a.g_per_split = (int)(((G + S - 1) / S + cg - 1) / cg * cg);
    // the real split count: splits past the last row group would leave
    // their partial rows unwritten
    if ((int64_t)a.g_per_split * (S - 1) >= G) return hipErrorInvalidValue;
    a.plane = (K / 64) * G * MOE_TB;
    const bool small = trows == 16;
    const size_t lds = 2 * (size_t)(small ? MOE_BUF<1> : MOE_BUF<4>);
    const void* kern = small ? (const void*)k_moe_down<1> : (const void*)k_moe_down<4>;
    static bool lds_set[2] = {};
    if (!lds_set[small]) {
        hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        lds_set[small] = true;
    }
    const dim3 grid((unsigned)(K / 256), (unsigned)ntile_max, (unsigned)S);
    if (small)
        ktimed_launch(k_moe_down<1>, grid, dim3(256), (uint32_t)lds, st, a);
    else
        ktimed_launch(k_moe_down<4>, grid, dim3(256), (uint32_t)lds, st, a);
    return hipGetLastError();
}

hipError_t launch_moe_combine(hipStream_t st, const float* part, int S, int64_t rows, int64_t K,
                              const MoeRoute& r, int64_t M, int64_t U, float* y, int accum) {
    if (M < 1 || K < 1 || S < 1 || U < 1 || U > MOE_MAXU) return hipErrorInvalidValue;
    auto kern = U <= 2 ? k_moe_combine<2> : U <= 4 ? k_moe_combine<4> : k_moe_combine<MOE_MAXU>;
    hipLaunchKernelGGL(kern, dim3((unsigned)((K + 255) / 256), (unsigned)M), dim3(256), 0,
                       st, part, S, rows, K, r, (int)U, y, accum);
    return hipGetLastError();
}

hipError_t launch_add(hipStream_t st, const float* x, float* y, int64_t n) {
    if (n < 1) return hipSuccess;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
    return hipGetLastError();
}
