// k_attn.hip -- tree-masked GQA attention over the fp16 KV cache on MFMA,
// split over chunks of the context (flash-decoding) and combined in a second
// pass (one partial per chunk, or per group of chunks on long contexts with
// many query rows).
//
// Semantics of Impl::attn (src/engine.cpp:137-177) with the draft-tree mask:
// query row m of head h attends to cache slots [0, npast) and to the tree
// slots npast + j of its ancestors j (itself included); kv head =
// h / (n_head / n_kv); scores are q.k / sqrt(hd); softmax; sum of p * v.
//
// One workgroup handles one kv head, one chunk of hd slots and one tile of
// 32 query rows of the GQA group (row r -> token r / gqa, head kvh * gqa +
// r % gqa) with hd / 16 waves.  Wave w first computes the scores of slots
// 16w .. 16w+15 with v_mfma_f32_16x16x32_f16: S^T = K . Q^T (K rows are the A
// operand, exact fp16; Q arrives split into fp16 hi + lo so the scores keep
// fp32 accuracy).  The chunk's row maxima meet in LDS, each wave writes its
// p = e^(s - max) as fp16 hi + lo into an LDS tile P[query row][slot], and
// wave w then forms output dims 16w .. 16w+15 over the whole chunk, O = P . V
// on v_mfma_f32_16x16x16_f16 with V kept transposed in the cache ([kv head]
// [dim][slot]) so its B operand is one 8-byte load.  The chunk partial (max,
// sum, O) goes straight from the MFMA registers to memory.
#include "ftx_internal.h"
#include "mm_dev.h"
#include "xq_dev.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

// waves per workgroup for head size 128 (16 waves, one score tile and one
// output tile per wave, measured slower)
constexpr int ATTN_WAVES_128 = 8;
// slots per chunk (one workgroup of hd / 16 waves) for head size hd (64-slot
// chunks measured slower for hd 128)
__host__ __device__ constexpr int chunk_slots(int hd) { return hd; }

// The workgroup (chunk c, kv head kvh, query tile qtile) of one sequence's
// attention; nch = the sequence's chunk count (its partials' stride).
template <int HD, int CHK, int NWV>
__device__ __forceinline__ void attn_mfma_wg(const AttnMArgs& a, int c, int kvh, int qtile,
                                             int nch) {
    constexpr int NDT = HD / 16;  // 16-dim output tiles
    constexpr int NST = CHK / 16; // 16-slot tiles of the chunk
    // score tiles (slot tile, query tile) per wave: pair p = w PPW + i takes
    // slot tile p / 2 and query tile p % 2
    constexpr int PPW = 2 * NST / NWV;
    static_assert(PPW == 1 || PPW == 2, "a wave takes one or two score tiles of one slot tile");
    // output tiles (dim tile, query tile) per wave: dim tile w % NDT, query
    // tiles all (QPW = 2) or w / NDT (QPW = 1)
    constexpr int QPW = 2 * NDT / NWV;
    static_assert(QPW == 1 || QPW == 2, "a wave takes one or two query tiles of one dim tile");
    constexpr int NDC = HD / 32;  // 32-dim chunks of the score contraction
    constexpr int QP = HD + 8;    // padded query row (halves)
    constexpr int PP = CHK + 8;   // padded P row (halves)
    constexpr int QV = (2 * 32 * HD / 8) / (64 * NWV);  // staged 16-byte query vectors per thread
    __shared__ _Float16 qs[2][32][QP];  // query hi / lo [part][row][dim]
    __shared__ _Float16 ps[2][32][PP];  // P hi / lo [part][query row][slot]
    __shared__ float smax[NST][32], ssum[NST][32], cmax[32];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, col = lane & 15, g = lane >> 4;
    const int64_t npast = a.npast;
    const int64_t total = npast + a.M;
    const int64_t slot0 = (int64_t)c * CHK;
    if (slot0 >= total) return;
    const int gqa = a.n_head / a.n_kv;
    const int qrows = a.M * gqa;
    const int qbase = qtile * 32;  // first query row of this tile
    const int64_t kdim = (int64_t)a.n_kv * HD;
    const int sst = (w * PPW) >> 1;          // this wave's slot tile
    const int64_t ws0 = slot0 + 16 * sst;    // its score slots
    const int dt = w % NDT;  // this wave's output dims 16 dt .. 16 dt + 15
    // ---- every operand load issued up front, in the order of use, with
    // clamped (always valid) addresses and no branch, so that each use waits
    // only for its own loads: the query vectors this thread stages (2 parts
    // x 32 rows x HD / 8; rows past qrows repeat the last valid row, whose
    // scores are masked and never stored), the ancestor-mask words of the
    // wave's query rows, K rows (A of S^T: slot ws0 + col, dims 32 dc + 8 g
    // ..), V^T rows (B of O: dim 16 dt + col, slots slot0 + 16 st + 4 g ..)
    v8h qv[QV];
#pragma unroll
    for (int k = 0; k < QV; ++k) {
        const int v = tid + 64 * NWV * k;
        const int part = v / (32 * HD / 8), r = (v / (HD / 8)) % 32, dv = v % (HD / 8);
        const int rq = min(qbase + r, qrows - 1);
        const int64_t qo = ((int64_t)(rq / gqa) * a.n_head + kvh * gqa + rq % gqa) * HD + 8 * dv;
        qv[k] = *(const v8h*)((part ? a.ql16 : a.qh16) + qo);
    }
    const int64_t j0 = ws0 + 4 * g - npast;  // tree index of this lane's first score slot
    const int wsel = (int)min(max(j0, (int64_t)0) >> 5, (int64_t)a.anc_words - 1);
    const int wnext = min(wsel + 1, a.anc_words - 1);
    uint32_t aw0[PPW], aw1[PPW];
#pragma unroll
    for (int pi = 0; pi < PPW; ++pi) {
        const int qt = (w * PPW + pi) & 1;
        const int rq = min(qbase + qt * 16 + col, qrows - 1);
        const uint32_t* an = a.anc + (int64_t)(rq / gqa) * a.anc_words;
        aw0[pi] = an[wsel];
        aw1[pi] = an[wnext];
    }
    v8h kf[NDC];
    {
        const _Float16* krow = a.kc + (ws0 + col) * kdim + (int64_t)kvh * HD + 8 * g;
#pragma unroll
        for (int dc = 0; dc < NDC; ++dc) kf[dc] = *(const v8h*)(krow + 32 * dc);
    }
    v4h vf[NST];
    {
        const _Float16* vrow = a.vt + ((int64_t)kvh * HD + 16 * dt + col) * a.cap + slot0 + 4 * g;
#pragma unroll
        for (int st = 0; st < NST; ++st) vf[st] = *(const v4h*)(vrow + 16 * st);
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the first use
#pragma unroll
    for (int k = 0; k < QV; ++k) {
        const int v = tid + 64 * NWV * k;
        const int part = v / (32 * HD / 8), r = (v / (HD / 8)) % 32, dv = v % (HD / 8);
        *(v8h*)&qs[part][r][8 * dv] = qv[k];
    }
    __syncthreads();
    // ---- S^T = K . Q^T for the wave's query tiles (every query fragment
    // read from LDS first); lane (col, g) then holds S^T[slot ws0 + 4g + r]
    // [query row qt * 16 + col]
    v8h qf[PPW][NDC][2];
#pragma unroll
    for (int pi = 0; pi < PPW; ++pi) {
        const int qt = (w * PPW + pi) & 1;
#pragma unroll
        for (int dc = 0; dc < NDC; ++dc) {
            qf[pi][dc][0] = *(const v8h*)&qs[0][qt * 16 + col][32 * dc + 8 * g];
            qf[pi][dc][1] = *(const v8h*)&qs[1][qt * 16 + col][32 * dc + 8 * g];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    v4f sc[PPW];
#pragma unroll
    for (int pi = 0; pi < PPW; ++pi) {
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dc = 0; dc < NDC; ++dc) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[dc], qf[pi][dc][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[dc], qf[pi][dc][1], acc, 0, 0, 0);
        }
        sc[pi] = acc;
    }
    // masked, scaled scores and this wave's row maxima
    const float scale = 1.f / sqrtf((float)HD);
#pragma unroll
    for (int pi = 0; pi < PPW; ++pi) {
        const int qt = (w * PPW + pi) & 1;
        const bool qvalid = qbase + qt * 16 + col < qrows;
        const uint64_t win = aw0[pi] | ((uint64_t)aw1[pi] << 32);
        float m_ = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            // committed slot, or tree slot j whose ancestor bit is set (bit
            // j - 32 wsel of the two-word window)
            const int64_t j = j0 + r;
            const bool tree_ok = j >= 0 && j < a.M && ((win >> ((j - 32 * wsel) & 63)) & 1u);
            const bool ok = qvalid && (j < 0 || tree_ok);
            const float sv = ok ? sc[pi][r] * scale : -INFINITY;
            sc[pi][r] = sv;
            m_ = fmaxf(m_, sv);
        }
        m_ = fmaxf(m_, __shfl_xor(m_, 16, 64));
        m_ = fmaxf(m_, __shfl_xor(m_, 32, 64));
        if (g == 0) smax[sst][qt * 16 + col] = m_;
    }
    __syncthreads();
    // ---- p = e^(s - chunk max); row sums per slot tile; P hi / lo into LDS
#pragma unroll
    for (int pi = 0; pi < PPW; ++pi) {
        const int qt = (w * PPW + pi) & 1;
        const int q = qt * 16 + col;
        float mx = smax[0][q];
#pragma unroll
        for (int k = 1; k < NST; ++k) mx = fmaxf(mx, smax[k][q]);
        float s_ = 0.f;
        v4h ph, pl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = sc[pi][r] == -INFINITY ? 0.f : expf(sc[pi][r] - mx);
            s_ += e;
            const _Float16 h = (_Float16)e;
            ph[r] = h;
            pl[r] = (_Float16)(e - (float)h);
        }
        s_ += __shfl_xor(s_, 16, 64);
        s_ += __shfl_xor(s_, 32, 64);
        if (g == 0) {
            ssum[sst][q] = s_;
            if (sst == 0) cmax[q] = mx;
        }
        *(v4h*)&ps[0][q][16 * sst + 4 * g] = ph;
        *(v4h*)&ps[1][q][16 * sst + 4 * g] = pl;
    }
    __syncthreads();
    // ---- O[:, 16 dt .. 16 dt + 15] = P . V over the chunk: A = P (query row
    // col, slots 16 st + 4g ..), B = V^T rows; lane then holds O[query row
    // qt * 16 + 4g + r][dim 16 dt + col]
#pragma unroll
    for (int qi = 0; qi < QPW; ++qi) {
        const int qt = QPW == 2 ? qi : w / NDT;
        v4h ph[NST], pl[NST];
#pragma unroll
        for (int st = 0; st < NST; ++st) {
            ph[st] = *(const v4h*)&ps[0][qt * 16 + col][16 * st + 4 * g];
            pl[st] = *(const v4h*)&ps[1][qt * 16 + col][16 * st + 4 * g];
        }
        __builtin_amdgcn_sched_barrier(0);
        v4f o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < NST; ++st) {
            o = __builtin_amdgcn_mfma_f32_16x16x16f16(ph[st], vf[st], o, 0, 0, 0);
            o = __builtin_amdgcn_mfma_f32_16x16x16f16(pl[st], vf[st], o, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rq = qbase + qt * 16 + 4 * g + r;
            if (rq >= qrows) continue;
            const int64_t qrow = (int64_t)(rq / gqa) * a.n_head + kvh * gqa + rq % gqa;
            a.pout[(qrow * nch + c) * HD + 16 * dt + col] = o[r];
        }
    }
    // chunk statistics of query row lane (wave 0)
    if (w == 0 && lane < 32 && qbase + lane < qrows) {
        const int rq = qbase + lane;
        const int64_t qi = (int64_t)(rq / gqa) * a.n_head + kvh * gqa + rq % gqa;
        float den = ssum[0][lane];
#pragma unroll
        for (int k = 1; k < NST; ++k) den += ssum[k][lane];
        a.pmax[qi * nch + c] = cmax[lane];
        a.psum[qi * nch + c] = den;
    }
}

// The workgroup (group grp of nc consecutive chunks, kv head kvh, query
// tile qtile) of one sequence's attention, for long contexts with many
// query rows: the group's chunks in turn with a running row maximum and sum
// (flash attention: O <- e^(m_old - m_new) O + P V with P = e^(s - m_new)),
// one partial per group (ngrp = the sequence's group count, the partials'
// stride).  The query is staged once; per chunk the same score / P / output
// steps as attn_mfma_wg, with each chunk's K / V rows and mask words loaded
// while the previous chunk's P . V runs.
template <int HD, int CHK, int NWV>
__device__ __forceinline__ void attn_mfma_wg_mc(const AttnMArgs& a, int grp, int kvh, int qtile,
                                                int ngrp) {
    constexpr int NDT = HD / 16, NST = CHK / 16;
    constexpr int PPW = 2 * NST / NWV;
    static_assert(PPW == 1 || PPW == 2, "a wave takes one or two score tiles of one slot tile");
    constexpr int QPW = 2 * NDT / NWV;
    static_assert(QPW == 1 || QPW == 2, "a wave takes one or two query tiles of one dim tile");
    constexpr int NDC = HD / 32, QP = HD + 8, PP = CHK + 8;
    constexpr int QV = (2 * 32 * HD / 8) / (64 * NWV);
    __shared__ _Float16 qs[2][32][QP];
    __shared__ _Float16 ps[2][32][PP];
    __shared__ float smax[NST][32], ssum[NST][32];
    __shared__ float rmax[32], rsum[32], ralpha[32];  // running max, sum; this chunk's rescale
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, col = lane & 15, g = lane >> 4;
    const int64_t npast = a.npast, total = npast + a.M;
    const int64_t gslot0 = (int64_t)grp * a.nc * CHK;
    if (gslot0 >= total) return;
    // chunks of the group holding slots below total (block-uniform)
    const int nck = (int)min((int64_t)a.nc, (total - gslot0 + CHK - 1) / CHK);
    const int gqa = a.n_head / a.n_kv, qrows = a.M * gqa, qbase = qtile * 32;
    const int64_t kdim = (int64_t)a.n_kv * HD;
    const int sst = (w * PPW) >> 1, dt = w % NDT;
    // query staging (once)
    {
        v8h qv[QV];
#pragma unroll
        for (int k = 0; k < QV; ++k) {
            const int v = tid + 64 * NWV * k;
            const int part = v / (32 * HD / 8), r = (v / (HD / 8)) % 32, dv = v % (HD / 8);
            const int rq = min(qbase + r, qrows - 1);
            const int64_t qo = ((int64_t)(rq / gqa) * a.n_head + kvh * gqa + rq % gqa) * HD + 8 * dv;
            qv[k] = *(const v8h*)((part ? a.ql16 : a.qh16) + qo);
        }
#pragma unroll
        for (int k = 0; k < QV; ++k) {
            const int v = tid + 64 * NWV * k;
            const int part = v / (32 * HD / 8), r = (v / (HD / 8)) % 32, dv = v % (HD / 8);
            *(v8h*)&qs[part][r][8 * dv] = qv[k];
        }
    }
    if (tid < 32) {
        rmax[tid] = -INFINITY;
        rsum[tid] = 0.f;
    }
    // a chunk's operands: mask words of the wave's query rows, K rows, V^T rows
    auto load = [&](int64_t slot0, uint32_t* aw0, uint32_t* aw1, v8h* kf, v4h* vf) {
        const int64_t ws0 = slot0 + 16 * sst;
        const int64_t j0 = ws0 + 4 * g - npast;
        const int wsel = (int)min(max(j0, (int64_t)0) >> 5, (int64_t)a.anc_words - 1);
        const int wnext = min(wsel + 1, a.anc_words - 1);
#pragma unroll
        for (int pi = 0; pi < PPW; ++pi) {
            const int qt = (w * PPW + pi) & 1;
            const int rq = min(qbase + qt * 16 + col, qrows - 1);
            const uint32_t* an = a.anc + (int64_t)(rq / gqa) * a.anc_words;
            aw0[pi] = an[wsel];
            aw1[pi] = an[wnext];
        }
        const _Float16* krow = a.kc + (ws0 + col) * kdim + (int64_t)kvh * HD + 8 * g;
#pragma unroll
        for (int dc = 0; dc < NDC; ++dc) kf[dc] = *(const v8h*)(krow + 32 * dc);
        const _Float16* vrow = a.vt + ((int64_t)kvh * HD + 16 * dt + col) * a.cap + slot0 + 4 * g;
#pragma unroll
        for (int st = 0; st < NST; ++st) vf[st] = *(const v4h*)(vrow + 16 * st);
    };
    uint32_t aw0[PPW], aw1[PPW];
    v8h kf[NDC];
    v4h vf[NST];
    load(gslot0, aw0, aw1, kf, vf);
    v4f oacc[QPW];
#pragma unroll
    for (int qi = 0; qi < QPW; ++qi) oacc[qi] = v4f{0.f, 0.f, 0.f, 0.f};
    const float scale = 1.f / sqrtf((float)HD);
    for (int ci = 0; ci < nck; ++ci) {
        const int64_t slot0 = gslot0 + (int64_t)ci * CHK;
        const int64_t ws0 = slot0 + 16 * sst;
        const int64_t j0 = ws0 + 4 * g - npast;
        const int wsel = (int)min(max(j0, (int64_t)0) >> 5, (int64_t)a.anc_words - 1);
        __syncthreads();  // the query staged / every wave done with the last chunk's LDS
        v8h qf[PPW][NDC][2];
#pragma unroll
        for (int pi = 0; pi < PPW; ++pi) {
            const int qt = (w * PPW + pi) & 1;
#pragma unroll
            for (int dc = 0; dc < NDC; ++dc) {
                qf[pi][dc][0] = *(const v8h*)&qs[0][qt * 16 + col][32 * dc + 8 * g];
                qf[pi][dc][1] = *(const v8h*)&qs[1][qt * 16 + col][32 * dc + 8 * g];
            }
        }
        v4f sc[PPW];
#pragma unroll
        for (int pi = 0; pi < PPW; ++pi) {
            v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dc = 0; dc < NDC; ++dc) {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[dc], qf[pi][dc][0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[dc], qf[pi][dc][1], acc, 0, 0, 0);
            }
            sc[pi] = acc;
        }
#pragma unroll
        for (int pi = 0; pi < PPW; ++pi) {
            const int qt = (w * PPW + pi) & 1;
            const bool qvalid = qbase + qt * 16 + col < qrows;
            const uint64_t win = aw0[pi] | ((uint64_t)aw1[pi] << 32);
            float m_ = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t j = j0 + r;
                const bool tree_ok = j >= 0 && j < a.M && ((win >> ((j - 32 * wsel) & 63)) & 1u);
                const bool ok = qvalid && (j < 0 || tree_ok);
                const float sv = ok ? sc[pi][r] * scale : -INFINITY;
                sc[pi][r] = sv;
                m_ = fmaxf(m_, sv);
            }
            m_ = fmaxf(m_, __shfl_xor(m_, 16, 64));
            m_ = fmaxf(m_, __shfl_xor(m_, 32, 64));
            if (g == 0) smax[sst][qt * 16 + col] = m_;
        }
        __syncthreads();
        // p = e^(s - m_new), m_new = max(running max, this chunk's max)
#pragma unroll
        for (int pi = 0; pi < PPW; ++pi) {
            const int qt = (w * PPW + pi) & 1;
            const int q = qt * 16 + col;
            float mx = rmax[q];
#pragma unroll
            for (int k = 0; k < NST; ++k) mx = fmaxf(mx, smax[k][q]);
            float s_ = 0.f;
            v4h ph, pl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = sc[pi][r] == -INFINITY ? 0.f : expf(sc[pi][r] - mx);
                s_ += e;
                const _Float16 h = (_Float16)e;
                ph[r] = h;
                pl[r] = (_Float16)(e - (float)h);
            }
            s_ += __shfl_xor(s_, 16, 64);
            s_ += __shfl_xor(s_, 32, 64);
            if (g == 0) ssum[sst][q] = s_;
            *(v4h*)&ps[0][q][16 * sst + 4 * g] = ph;
            *(v4h*)&ps[1][q][16 * sst + 4 * g] = pl;
        }
        // this chunk's V rows stay in vc; the next chunk's operands go out
        // now and land during this chunk's P . V
        v4h vc[NST];
#pragma unroll
        for (int st = 0; st < NST; ++st) vc[st] = vf[st];
        if (ci + 1 < nck) load(slot0 + CHK, aw0, aw1, kf, vf);
        __syncthreads();
        if (tid < 32) {  // running statistics of row tid
            const float mo = rmax[tid];
            float mn = mo, ls = 0.f;
#pragma unroll
            for (int k = 0; k < NST; ++k) mn = fmaxf(mn, smax[k][tid]);
#pragma unroll
            for (int k = 0; k < NST; ++k) ls += ssum[k][tid];
            const float al = mo == -INFINITY ? 0.f : expf(mo - mn);
            rsum[tid] = al * rsum[tid] + ls;
            rmax[tid] = mn;
            ralpha[tid] = al;
        }
        __syncthreads();
        // O <- alpha O + P . V over the chunk for the wave's dim tile
#pragma unroll
        for (int qi = 0; qi < QPW; ++qi) {
            const int qt = QPW == 2 ? qi : w / NDT;
            v4h ph[NST], pl[NST];
#pragma unroll
            for (int st = 0; st < NST; ++st) {
                ph[st] = *(const v4h*)&ps[0][qt * 16 + col][16 * st + 4 * g];
                pl[st] = *(const v4h*)&ps[1][qt * 16 + col][16 * st + 4 * g];
            }
            v4f o = oacc[qi];
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] *= ralpha[qt * 16 + 4 * g + r];
#pragma unroll
            for (int st = 0; st < NST; ++st) {
                o = __builtin_amdgcn_mfma_f32_16x16x16f16(ph[st], vc[st], o, 0, 0, 0);
                o = __builtin_amdgcn_mfma_f32_16x16x16f16(pl[st], vc[st], o, 0, 0, 0);
            }
            oacc[qi] = o;
        }
    }
    // the group's partial: O, the running max and sum of each valid row
#pragma unroll
    for (int qi = 0; qi < QPW; ++qi) {
        const int qt = QPW == 2 ? qi : w / NDT;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rq = qbase + qt * 16 + 4 * g + r;
            if (rq >= qrows) continue;
            const int64_t qrow = (int64_t)(rq / gqa) * a.n_head + kvh * gqa + rq % gqa;
            a.pout[(qrow * ngrp + grp) * HD + 16 * dt + col] = oacc[qi][r];
        }
    }
    if (w == 0 && lane < 32 && qbase + lane < qrows) {
        const int rq = qbase + lane;
        const int64_t qi = (int64_t)(rq / gqa) * a.n_head + kvh * gqa + rq % gqa;
        a.pmax[qi * ngrp + grp] = rmax[lane];
        a.psum[qi * ngrp + grp] = rsum[lane];
    }
}

// More than 16 query rows per kv head (chains of several tokens, draft
// trees, batches of trees): one workgroup of FA_WAVES waves takes 16 query
// rows per wave of one kv head over a group of a.pslots slots (whole
// 64-slot chunks, at least one chunk_slots(HD) block; one partial each), so each
// K / V row is read by ceil(rows / 128) workgroups instead of one per 32
// rows.  The group's 64-slot chunks are copied to LDS by direct
// global->LDS loads one chunk ahead (double buffer, one barrier per chunk),
// in MFMA fragment order: block (st, dc) of K holds, at lane l's 16 bytes,
// K[slot pi(st, l % 16)][32 dc + 8 (l / 16) ..], with the slot permutation
// pi(st, m) = 32 (st / 2) + 8 (m / 4) + 4 (st % 2) + m % 4; block (dt, sp)
// of V^T holds V^T[16 dt + l % 16][32 sp + 8 (l / 16) ..].  Every operand
// read is one conflict-free 16-byte LDS load per lane.
// A wave keeps its rows' query as the B operand (fp16 hi + lo), the running
// row maximum and sum, and O^T (dims x rows) in registers:
//   S^T = K . Q^T on v_mfma_f32_16x16x32_f16: C lane (col, kq) holds the
//   scores of row col at slots pi(st, 4 kq + r), r < 4 -- for the two tiles
//   st = 2 sp, 2 sp + 1 these are slots 32 sp + 8 kq + e, e < 8, which is
//   exactly the K index run 8 kq .. 8 kq + 7 of lane (col, kq) in a B
//   operand; so P^T passes from the score registers to the
//   O^T += V^T . P^T MFMAs (K = 32 slots) without LDS, and the row maximum
//   and sum are a lane's own values plus two shuffles.
// Flash attention per chunk: m_new = max(m, max_chunk s), O <- e^(m - m_new)
// O + P V, l <- e^(m - m_new) l + sum P, P = e^(s - m_new) split fp16 hi +
// lo (computed as 2^(s c - m c), c = log2(e) / sqrt(hd)).  One partial
// (O, m, l) per row and group, in the layout of attn_mfma_wg_mc, combined by
// k_attn_combine (or k_attn_combine_xq).
// Measured: 8 waves (two per SIMD) beat 16 (four per SIMD) and 32 rows per
// wave on the 52-node tree and the 70B batch; the workgroup's MFMAs and
// softmax arithmetic do not overlap, so its time is their sum.
constexpr int FA_WAVES = 8;
constexpr int FA_CHK = 64;  // slots per chunk
typedef __attribute__((address_space(3))) void lds_void;

template <int HD>
__host__ __device__ constexpr size_t fa_lds_bytes() {
    return 2 * (size_t)(HD / 8 + HD / 8) * 1024;  // two buffers of K and V^T blocks
}

template <int HD>
__device__ __forceinline__ void attn_fa_wg(const AttnMArgs& a, int grp, int kvh, int qsplit,
                                           int ngrp) {
    constexpr int NDC = HD / 32;     // 32-dim steps of the score contraction
    constexpr int NDT = HD / 16;     // 16-dim tiles of O^T
    constexpr int KB = 4 * NDC;      // K blocks per chunk: (st, dc)
    constexpr int NB = KB + 2 * NDT; // with the V^T blocks (dt, sp)
    constexpr int BPW = NB / FA_WAVES;
    static_assert(NB % FA_WAVES == 0 && NDC % BPW == 0 && BPW % 2 == 0,
                  "a wave copies blocks of one slot tile of K, or whole dim tiles of V^T");
    constexpr int BUF = NB * 1024;
    static_assert(chunk_slots(HD) % FA_CHK == 0, "whole chunks per block");
    extern __shared__ __attribute__((aligned(16))) uint8_t fa_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int64_t npast = a.npast, total = npast + a.M;
    const int64_t gslot0 = (int64_t)grp * a.pslots;
    if (gslot0 >= total) return;  // block-uniform
    const int nck = (int)min((int64_t)(a.pslots / FA_CHK), (total - gslot0 + FA_CHK - 1) / FA_CHK);
    const int gqa = a.n_head / a.n_kv, qrows = a.M * gqa;
    const int rbase = (qsplit * FA_WAVES + w) * 16;  // the wave's first query row
    const bool wlive = rbase < qrows;                // wave-uniform

    // the wave's blocks b0 + i, b0 = BPW w: K blocks (st, dc0 + i) or V^T
    // blocks (dt0 + i / 2, i % 2).  Block i of a chunk at slot0 comes from
    // lbase + slot0 * sstride + ioff(i) (K rows: kdim apart; V^T rows:
    // contiguous)
    const int b0 = BPW * w;
    const bool kwave = b0 < KB;  // wave-uniform
    const int64_t sstride = kwave ? (int64_t)a.n_kv * HD : 1;
    const int st0 = b0 / NDC, dc0 = b0 % NDC, dt0 = (b0 - KB) >> 1;
    const _Float16* lbase =
        kwave ? a.kc + (32 * (st0 >> 1) + 8 * (col >> 2) + 4 * (st0 & 1) + (col & 3)) * sstride +
                    (int64_t)kvh * HD + 32 * dc0 + 8 * kq
              : a.vt + ((int64_t)kvh * HD + 16 * dt0 + col) * a.cap + 8 * kq;
    auto ioff = [&](int i) -> int64_t { return kwave ? 32 * i : 16 * (i >> 1) * a.cap + 32 * (i & 1); };
    auto stage = [&](int64_t slot0, int buf) {
        uint8_t* dst = fa_lds + buf * BUF + BPW * w * 1024;
        const _Float16* src = lbase + slot0 * sstride;
#pragma unroll
        for (int i = 0; i < BPW; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(src + ioff(i)),
                                             (lds_void*)(dst + i * 1024), 16, 0, 0);
    };
    stage(gslot0, 0);

    // the rows' B operands (rows past qrows repeat the last valid row: their
    // results stay in their own O^T columns and are never stored)
    v8h qf[NDC][2];
    const int rq0 = min(rbase + col, qrows - 1), node = rq0 / gqa;
    {
        const int64_t qo = ((int64_t)node * a.n_head + kvh * gqa + rq0 % gqa) * HD + 8 * kq;
#pragma unroll
        for (int dc = 0; dc < NDC; ++dc) {
            qf[dc][0] = wlive ? *(const v8h*)(a.qh16 + qo + 32 * dc) : v8h{};
            qf[dc][1] = wlive ? *(const v8h*)(a.ql16 + qo + 32 * dc) : v8h{};
        }
    }
    const float c2 = 1.4426950408889634f / sqrtf((float)HD);
    float mrun = -INFINITY, lrun = 0.f;  // running maximum of the raw scores, running sum
    v4f o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < nck; ++c) {
        const int64_t slot0 = gslot0 + (int64_t)c * FA_CHK;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's copies of chunk c
        __syncthreads();                     // every wave's copies; the other buffer free
        // chunks reaching into the draft (block-uniform): the ancestor words
        // of the lane's two 8-slot runs, loaded before the next chunk's copies
        const bool tree = wlive && slot0 + FA_CHK > npast;
        uint32_t aw[2][2];
        int j0[2] = {0, 0}, wsel[2] = {0, 0};
        if (tree) {
            const uint32_t* an = a.anc + node * a.anc_words;
#pragma unroll
            for (int sp = 0; sp < 2; ++sp) {
                j0[sp] = (int)(slot0 - npast) + 32 * sp + 8 * kq;
                wsel[sp] = min(max(j0[sp], 0) >> 5, a.anc_words - 1);
                aw[sp][0] = an[wsel[sp]];
                aw[sp][1] = an[min(wsel[sp] + 1, a.anc_words - 1)];
            }
        }
        if (c + 1 < nck) stage(slot0 + FA_CHK, (c + 1) & 1);
        if (!wlive) continue;
        const uint8_t* bufp = fa_lds + (c & 1) * BUF;
        // raw scores S^T
        v4f s[4];
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int dc = 0; dc < NDC; ++dc) {
                const v8h kf = *(const v8h*)(bufp + (st * NDC + dc) * 1024 + lane * 16);
                s[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    kf, qf[dc][0], dc == 0 ? v4f{0.f, 0.f, 0.f, 0.f} : s[st], 0, 0, 0);
                s[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[dc][1], s[st], 0, 0, 0);
            }
        if (tree) {
            // slot 8 kq + e of run sp: allowed iff before the draft, or a
            // draft slot j < M whose ancestor bit is set
#pragma unroll
            for (int sp = 0; sp < 2; ++sp) {
                const uint64_t win = aw[sp][0] | ((uint64_t)aw[sp][1] << 32);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int j = j0[sp] + e;
                    const bool ok = (j < 0) | ((j < a.M) & (((win >> ((j - 32 * wsel[sp]) & 63)) & 1u) != 0));
                    const float v = s[2 * sp + (e >> 2)][e & 3];
                    s[2 * sp + (e >> 2)][e & 3] = ok ? v : -INFINITY;
                }
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[st][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mn = fmaxf(mrun, mx);
        // every score so far masked: p = 0, nothing to rescale
        const float mc = mn == -INFINITY ? 0.f : mn * c2;
        const float al = __builtin_amdgcn_exp2f(mrun * c2 - mc);  // 0 while mrun = -inf
        float sum = 0.f;
        v8h ph[2], pl[2];
#pragma unroll
        for (int sp = 0; sp < 2; ++sp)
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                // a pair: split_hl2 (one conversion, two mixed fmas)
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * sp + (e >> 2)][e & 3], c2, -mc));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * sp + (e >> 2)][(e & 3) + 1], c2, -mc));
                sum += p0;
                sum += p1;
                v2h hh, ll;
                split_hl2(p0, p1, hh, ll);
                ph[sp][e] = hh[0];
                ph[sp][e + 1] = hh[1];
                pl[sp][e] = ll[0];
                pl[sp][e + 1] = ll[1];
            }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        lrun = al * lrun + sum;
        mrun = mn;
        if (__builtin_amdgcn_ballot_w64(al != 1.f))  // a maximum moved (wave-uniform)
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) o[dt] *= al;
        // O^T += V^T . P^T
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int sp = 0; sp < 2; ++sp) {
                const v8h vf = *(const v8h*)(bufp + (KB + 2 * dt + sp) * 1024 + lane * 16);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph[sp], o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[sp], o[dt], 0, 0, 0);
            }
    }
    const int rq = rbase + col;
    if (!wlive || rq >= qrows) return;
    // the group's partial (m in natural-log units, as the combine expects):
    // lane (col, kq) of tile dt holds dims 16 dt + 4 kq + r of row col
    const int64_t qrow = (int64_t)(rq / gqa) * a.n_head + kvh * gqa + rq % gqa;
    float* po = a.pout + (qrow * ngrp + grp) * HD + 4 * kq;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) *(v4f*)(po + 16 * dt) = o[dt];
    if (kq == 0) {
        a.pmax[qrow * ngrp + grp] = mrun == -INFINITY ? -INFINITY : mrun * (c2 * 0.6931471805599453f);
        a.psum[qrow * ngrp + grp] = lrun;
    }
}

template <int HD>
__global__ void __launch_bounds__(64 * FA_WAVES) k_attn_fa(AttnMArgs a) {
    attn_fa_wg<HD>(a, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x);
}

// several sequences: grid.z runs over every sequence's query splits
// (sequence s owns splits qt0[s] .. qt0[s + 1] - 1)
template <int HD>
__global__ void __launch_bounds__(64 * FA_WAVES) k_attn_fa_batch(AttnMBatch b) {
    int s = 0;
    while (s + 1 < b.nseq && (int)blockIdx.z >= b.qt0[s + 1]) ++s;
    const AttnMArgs a = b.s[s];  // loaded once
    attn_fa_wg<HD>(a, blockIdx.x, blockIdx.y, (int)blockIdx.z - b.qt0[s], b.nch[s]);
}

template <int HD, int CHK, int NWV>
__global__ void __launch_bounds__(64 * NWV) k_attn_mfma(AttnMArgs a) {
    attn_mfma_wg<HD, CHK, NWV>(a, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x);
}

// groups of a.nc chunks per workgroup (grid.x = the group count)
template <int HD, int CHK, int NWV>
__global__ void __launch_bounds__(64 * NWV) k_attn_mfma_mc(AttnMArgs a) {
    attn_mfma_wg_mc<HD, CHK, NWV>(a, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x);
}

// several sequences in one launch: grid.z runs over every sequence's query
// tiles (sequence s owns tiles qt0[s] .. qt0[s + 1] - 1); chunks past a
// sequence's own end return at once
template <int HD, int CHK, int NWV, bool MC>
__global__ void __launch_bounds__(64 * NWV) k_attn_mfma_batch(AttnMBatch b) {
    int s = 0;
    while (s + 1 < b.nseq && (int)blockIdx.z >= b.qt0[s + 1]) ++s;
    if constexpr (MC)
        attn_mfma_wg_mc<HD, CHK, NWV>(b.s[s], blockIdx.x, blockIdx.y, (int)blockIdx.z - b.qt0[s],
                                      b.nch[s]);
    else
        attn_mfma_wg<HD, CHK, NWV>(b.s[s], blockIdx.x, blockIdx.y, (int)blockIdx.z - b.qt0[s],
                                   b.nch[s]);
}

// out[m][h*hd + d] = sum_c e^(max_c - M) O_c[d] / sum_c e^(max_c - M) sum_c
// one block per query row; the chunk weights are formed once in LDS so the
// output loop is a stream of independent loads
__device__ __forceinline__ void attn_combine_row(const AttnMArgs& a, int64_t qi, int nch) {
    // Every load of the common case is issued at entry, branch-free (indices
    // clamped): the first CPF partials of this thread's dim and the statistics
    // of partial `lane`.  Each wave then forms the weights, their maximum and
    // the denominator itself (shuffles, no workgroup barrier); weights of the
    // first CPF partials are read from their lanes (v_readlane), later ones
    // (more than CPF partials) through the wave's own LDS copy.
    constexpr int CPF = 8;
    __shared__ float wsh[2][1024];  // chunk weights (nch <= 1024) per wave
    const int d = threadIdx.x, wv = d >> 6, lane = d & 63;
    const int64_t npast = a.npast;
    const int ch = a.pslots;  // slots per partial
    const int nvalid = (int)((npast + a.M + ch - 1) / ch);
    const float* pm = a.pmax + qi * nch;
    const float* pz = a.psum + qi * nch;
    const float* po = a.pout + qi * nch * a.hd + min(d, a.hd - 1);
    float pv[CPF];
#pragma unroll
    for (int i = 0; i < CPF; ++i) pv[i] = po[(int64_t)min(i, nvalid - 1) * a.hd];
    const int cl = min(lane, nvalid - 1);
    const float m0 = pm[cl], z0 = pz[cl];
    float M = lane < nvalid ? m0 : -INFINITY;
    for (int c = lane + 64; c < nvalid; c += 64) M = fmaxf(M, pm[c]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    const float w0 = lane < nvalid && m0 != -INFINITY ? expf(m0 - M) : 0.f;
    float den = w0 * z0;
    for (int c = lane + 64; c < nvalid; c += 64) {
        const float mc = pm[c];
        const float w = mc == -INFINITY ? 0.f : expf(mc - M);
        wsh[wv][c] = w;
        den += w * pz[c];
    }
    if (nvalid > CPF) wsh[wv][lane] = w0;  // wave-uniform
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
    // the weights written by the wave's other lanes (LDS in program order
    // within a wave; the fence keeps the compiler's order too)
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const float* wl = wsh[wv];
    float num = 0.f;
#pragma unroll
    for (int i = 0; i < CPF; ++i) {
        const float wi = lane_f(w0, i);
        if (i < nvalid) num += wi * pv[i];
    }
    for (int c = CPF; c < nvalid; ++c) num += wl[c] * po[(int64_t)c * a.hd];
    if (d < a.hd) {  // whole waves (hd = 64 or 128)
        const float v = num / den;
        if (!a.frag.xh) {
            a.out[qi * a.hd + d] = v;
            return;
        }
        // the o projection's operand (k_mm_prep without a norm): element k
        // = h hd + d of operand row row0 + m, and the 32-element sums
        const int64_t R = a.frag.row0 + qi / a.n_head, k = (qi % a.n_head) * a.hd + d;
        _Float16 h, l;
        split_hl(v, h, l);
        const int64_t at = frag_at(R, k, a.frag.K, a.frag.inter != 0);
        a.frag.xh[at] = h;
        a.frag.xl[at] = l;
        float s = v;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o, 64);
        if ((d & 31) == 0) {
            split_hl(s, h, l);
            const int64_t sa = frag_sum_at(R, k / 32, a.frag.K);
            a.frag.sh[sa] = h;
            a.frag.sl[sa] = l;
        }
    }
}

__global__ void __launch_bounds__(128) k_attn_combine(AttnMArgs a, int nch) {
    attn_combine_row(a, blockIdx.x, nch);  // query row m * n_head + h
}

// several sequences: sequence s owns blocks qi0[s] .. qi0[s + 1] - 1
__global__ void __launch_bounds__(128) k_attn_combine_batch(AttnMBatch b) {
    int s = 0;
    while (s + 1 < b.nseq && (int)blockIdx.x >= b.qi0[s + 1]) ++s;
    attn_combine_row(b.s[s], (int64_t)blockIdx.x - b.qi0[s], b.nch[s]);
}

// The combine of k_attn_combine fused with the activation prep of the
// output projection: workgroup (sb, m) forms elements 256 sb .. 256 sb + 255
// of attention output row m (the HPB = 256 / HD heads 256 sb / HD ..) and
// writes them as the GEMV's activation operand (xq_dev.h) instead of fp32.
// Wave h < HPB forms head h's chunk weights; then wave w adds chunks
// w, w + 4, ... into per-lane partial numerators (lane l: elements 4l ..
// 4l+3), which wave 0 sums in wave order and quantises.  Rows m >= M are
// written as zeros.
template <int HD, bool L16>
__global__ void __launch_bounds__(256) k_attn_combine_xq(AttnMArgs a, int nch, XqPtrs o) {
    constexpr int HPB = 256 / HD;
    constexpr int CPF = 8;  // chunk partials per thread held in registers
    __shared__ float wsh[HPB][1024];  // chunk weights (nch <= 1024)
    __shared__ float sden[HPB];
    __shared__ float4 red[4][64];
    const int64_t sb = blockIdx.x;
    const int m = blockIdx.y, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int ch = a.pslots;  // slots per partial
    const int nvalid = (int)((a.npast + a.M + ch - 1) / ch);
    const int hh = (4 * l) / HD, d = (4 * l) % HD;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (m < a.M) {
        // the common case's loads issued together, branch-free (chunk
        // indices clamped): chunk statistics of head min(w, HPB - 1), chunk l,
        // and this thread's partials of chunks w + 4k, k < CPF
        const int64_t qw = (int64_t)m * a.n_head + sb * HPB + min(w, HPB - 1);
        const int cl = min(l, nvalid - 1);
        const float pm = a.pmax[qw * nch + cl], pz = a.psum[qw * nch + cl];
        const int64_t qi = (int64_t)m * a.n_head + sb * HPB + hh;
        const float* po = a.pout + qi * nch * HD + d;
        float4 pf[CPF];
#pragma unroll
        for (int k = 0; k < CPF; ++k) pf[k] = *(const float4*)(po + (int64_t)min(w + 4 * k, nvalid - 1) * HD);
        __builtin_amdgcn_sched_barrier(0);
        if (w < HPB) {
            float mx = l < nvalid ? pm : -INFINITY;
            for (int c = l + 64; c < nvalid; c += 64) mx = fmaxf(mx, a.pmax[qw * nch + c]);
#pragma unroll
            for (int s = 32; s > 0; s >>= 1) mx = fmaxf(mx, __shfl_xor(mx, s, 64));
            float den = 0.f;
            if (l < nvalid) {
                const float wc = pm == -INFINITY ? 0.f : expf(pm - mx);
                wsh[w][l] = wc;
                den = wc * pz;
            }
            for (int c = l + 64; c < nvalid; c += 64) {
                const float mc = a.pmax[qw * nch + c];
                const float wc = mc == -INFINITY ? 0.f : expf(mc - mx);
                wsh[w][c] = wc;
                den += wc * a.psum[qw * nch + c];
            }
#pragma unroll
            for (int s = 32; s > 0; s >>= 1) den += __shfl_xor(den, s, 64);
            if (l == 0) sden[w] = den;
        }
        __syncthreads();
        // chunks in the order w, w + 4, w + 8, ..
        float4 num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < CPF; ++k) {
            if (w + 4 * k < nvalid) {  // wave-uniform
                const float wc = wsh[hh][w + 4 * k];
                num.x += wc * pf[k].x;
                num.y += wc * pf[k].y;
                num.z += wc * pf[k].z;
                num.w += wc * pf[k].w;
            }
        }
#pragma unroll 4
        for (int c = w + 4 * CPF; c < nvalid; c += 4) {
            const float wc = wsh[hh][c];
            const float4 p = *(const float4*)(po + (int64_t)c * HD);
            num.x += wc * p.x;
            num.y += wc * p.y;
            num.z += wc * p.z;
            num.w += wc * p.w;
        }
        red[w][l] = num;
        __syncthreads();
        if (w == 0) {
            float4 t = red[0][l];
#pragma unroll
            for (int k = 1; k < 4; ++k) {
                const float4 r = red[k][l];
                t.x += r.x;
                t.y += r.y;
                t.z += r.z;
                t.w += r.w;
            }
            const float den = sden[hh];
            v[0] = t.x / den;
            v[1] = t.y / den;
            v[2] = t.z / den;
            v[3] = t.w / den;
        }
    }
    if (w == 0) {
        if constexpr (L16)
            xq16_emit(v, sb, m, l, o);
        else
            xq_emit(v, sb, m, l, o);
    }
}

}  // namespace

bool attn_combine_xq_supported(int64_t hd, int64_t n_head) {
    const int64_t K = hd * n_head;
    return (hd == 64 || hd == 128) && K % 512 == 0 && K <= 16384;
}

bool attn_mfma_supported(int64_t hd, int kv_f16, int64_t M, int64_t n_head, int64_t n_kv) {
    return kv_f16 && (hd == 64 || hd == 128) && M >= 1 && (M * (n_head / n_kv)) <= 32 * 16;
}

size_t attn_part_floats(int64_t M, int64_t n_head, int64_t hd, int64_t cap_alloc) {
    const int64_t nch = (cap_alloc + chunk_slots((int)hd) - 1) / chunk_slots((int)hd);
    return (size_t)(M * n_head * nch) * (size_t)(hd + 2);
}

// chunks per workgroup: doubled from 1 while the grid keeps at least 256
// workgroups, at most 16: the partials (and the combine's reads of them)
// shrink by that factor.  Measured: the 52-node tree at context 4096 (1848
// one-chunk workgroups) 1.68 -> 1.54 ms of attention per step at 4 chunks,
// 2.08 ms at 8; the 70B batch the same at 8 and 16; grids of at most 511
// workgroups (the 8-token chains, the 4 x 8-token MoE batch) keep one chunk
static int attn_chunks_per_wg(int64_t wgs) {
    int nc = 1;
    while (nc < 16 && wgs / (2 * nc) >= 256) nc *= 2;
    return nc;
}

// The many-row kernel (k_attn_fa) takes sequences with more than 16 query
// rows per kv head (measured: the 8-token chain of 32 rows per kv head at
// context 2048 gains a little, the trees and batches most)
static bool attn_fa_rows(int64_t qrows) { return qrows > 16; }
static int attn_fa_splits(int64_t qrows) { return (int)((qrows + 16 * FA_WAVES - 1) / (16 * FA_WAVES)); }

// 64-slot chunks per workgroup (and per partial) for the many-row kernel:
// sequence s has nchk[s] live chunks and splits[s] row splits; with g
// chunks per workgroup the live workgroups run in rounds of 256, a round
// costing about 3 + g chunk times (measured: ~3 us of start and ~1-2 us per
// chunk, the chunk's MFMAs and softmax); the cheapest g in [gmin, 32], the
// largest on ties (fewer partials for the combine).  gmin = the chunks of
// one chunk_slots(hd) block, so the partials fit the buffer sized per block.
// Whole chunks rather than whole blocks let the 52-node tree at context
// 4096 take 224 workgroups of 5 chunks instead of 176 of 6.
static int attn_fa_chunks_per_wg(const int64_t* nchk, const int* splits, int nseq, int n_kv,
                                 int gmin) {
    int best = gmin;
    int64_t best_cost = -1;
    for (int g = gmin; g <= 32; ++g) {
        int64_t wgs = 0;
        for (int s = 0; s < nseq; ++s) wgs += (nchk[s] + g - 1) / g * n_kv * splits[s];
        const int64_t cost = (wgs + 255) / 256 * (3 + (int64_t)g);
        if (best_cost < 0 || cost <= best_cost) {
            best_cost = cost;
            best = g;
        }
    }
    return best;
}

template <int HD, typename A>
static hipError_t launch_fa(void (*kern)(A), const dim3& grid, hipStream_t st, const A& args) {
    static bool lds_set = false;
    if (!lds_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)fa_lds_bytes<HD>());
        if (e != hipSuccess) return e;
        lds_set = true;
    }
    ktimed_launch(kern, grid, dim3(64 * FA_WAVES), (uint32_t)fa_lds_bytes<HD>(), st, args);
    return hipGetLastError();
}

hipError_t launch_attn_mfma(hipStream_t st, AttnMArgs a, float* part, int8_t* xq, int xq16) {
    // whole chunks of the allocation: every slot a chunk reads is allocated
    const int ch = chunk_slots(a.hd);
    if (a.cap % ch) return hipErrorInvalidValue;
    const int nch = (int)(a.cap / ch);
    if (nch > 1024) return hipErrorInvalidValue;  // combine weights live in LDS
    const int64_t qi = (int64_t)a.M * a.n_head;
    const int64_t qrows = (int64_t)a.M * (a.n_head / a.n_kv);
    if (attn_fa_rows(qrows)) {
        const int qs = attn_fa_splits(qrows);
        const int64_t nchk = (a.npast + a.M + FA_CHK - 1) / FA_CHK;
        // the combine that writes the GEMV operand takes one block per
        // partial (the 8-token chain: 136 workgroups of two chunks)
        const int g = xq ? ch / FA_CHK : attn_fa_chunks_per_wg(&nchk, &qs, 1, a.n_kv, ch / FA_CHK);
        a.pslots = g * FA_CHK;
        const int ngrp = (int)((a.cap + a.pslots - 1) / a.pslots);  // the partials' stride
        a.pmax = part;
        a.psum = part + qi * ngrp;
        a.pout = part + 2 * qi * ngrp;
        const dim3 grid((unsigned)ngrp, (unsigned)a.n_kv, (unsigned)qs);
        hipError_t e;
        if (a.hd == 128)
            e = launch_fa<128>(k_attn_fa<128>, grid, st, a);
        else
            e = launch_fa<64>(k_attn_fa<64>, grid, st, a);
        if (e != hipSuccess) return e;
        if (xq) {
            const int64_t K = (int64_t)a.n_head * a.hd;
            const dim3 cg((unsigned)(K / 256), 8);
            const auto kc = a.hd == 128 ? (xq16 ? k_attn_combine_xq<128, true> : k_attn_combine_xq<128, false>)
                                        : (xq16 ? k_attn_combine_xq<64, true> : k_attn_combine_xq<64, false>);
            hipLaunchKernelGGL(kc, cg, dim3(256), 0, st, a, ngrp, xq_ptrs(xq, K));
        } else {
            hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)qi), dim3(128), 0, st, a, ngrp);
        }
        return hipGetLastError();
    }
    // one workgroup per (chunk or group of chunks, kv head, tile of 32 query rows)
    const int qtiles = (int)((a.M * (a.n_head / a.n_kv) + 31) / 32);
    const int64_t nvalid = (a.npast + a.M + ch - 1) / ch;
    a.nc = xq ? 1 : attn_chunks_per_wg(nvalid * a.n_kv * qtiles);
    a.pslots = a.nc * ch;
    const int ngrp = (nch + a.nc - 1) / a.nc;  // the partials' stride
    a.pmax = part;
    a.psum = part + qi * ngrp;
    a.pout = part + 2 * qi * ngrp;
    const dim3 grid((unsigned)ngrp, (unsigned)a.n_kv, (unsigned)qtiles);
    if (a.hd == 128 && a.nc > 1)
        ktimed_launch(k_attn_mfma_mc<128, chunk_slots(128), ATTN_WAVES_128>, grid,
                      dim3(64 * ATTN_WAVES_128), 0, st, a);
    else if (a.hd == 128)
        ktimed_launch(k_attn_mfma<128, chunk_slots(128), ATTN_WAVES_128>, grid,
                           dim3(64 * ATTN_WAVES_128), 0, st, a);
    else if (a.hd == 64 && a.nc > 1)
        ktimed_launch(k_attn_mfma_mc<64, chunk_slots(64), 4>, grid, dim3(64 * 4), 0, st, a);
    else if (a.hd == 64)
        ktimed_launch(k_attn_mfma<64, chunk_slots(64), 4>, grid, dim3(64 * 4), 0, st, a);
    else
        return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (xq) {
        if (!attn_combine_xq_supported(a.hd, a.n_head)) return hipErrorInvalidValue;
        const int64_t K = (int64_t)a.n_head * a.hd;
        const dim3 cg((unsigned)(K / 256), 8);
        const auto kc = a.hd == 128 ? (xq16 ? k_attn_combine_xq<128, true> : k_attn_combine_xq<128, false>)
                                    : (xq16 ? k_attn_combine_xq<64, true> : k_attn_combine_xq<64, false>);
        hipLaunchKernelGGL(kc, cg, dim3(256), 0, st, a, ngrp, xq_ptrs(xq, K));
    } else {
        hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)qi), dim3(128), 0, st, a, ngrp);
    }
    return hipGetLastError();
}

hipError_t launch_attn_mfma_batch(hipStream_t st, const AttnMArgs* as, const float* const* parts,
                                  int nseq) {
    if (nseq < 1 || nseq > FTX_MAX_SEQ) return hipErrorInvalidValue;
    AttnMBatch b{};
    b.nseq = nseq;
    int hd = as[0].hd, nkv = as[0].n_kv, maxch = 0, qt = 0, qi = 0;
    // the many-row kernel when every sequence has the rows for it
    bool fa = true;
    for (int s = 0; s < nseq; ++s) fa = fa && attn_fa_rows((int64_t)as[s].M * (as[s].n_head / nkv));
    int64_t wgs = 0;  // the one-block grid's live workgroups
    int64_t nblk[FTX_MAX_SEQ], nchk[FTX_MAX_SEQ];
    int splits[FTX_MAX_SEQ];
    for (int s = 0; s < nseq; ++s) {
        const int ch = chunk_slots(as[s].hd);
        if (as[s].hd != hd || as[s].n_kv != nkv || as[s].cap % ch) return hipErrorInvalidValue;
        const int64_t r = (int64_t)as[s].M * (as[s].n_head / nkv);
        nblk[s] = (as[s].npast + as[s].M + ch - 1) / ch;
        nchk[s] = (as[s].npast + as[s].M + FA_CHK - 1) / FA_CHK;
        splits[s] = fa ? attn_fa_splits(r) : (int)((r + 31) / 32);
        wgs += nblk[s] * nkv * splits[s];
    }
    // many-row: g chunks per partial; otherwise nc blocks
    const int g = fa ? attn_fa_chunks_per_wg(nchk, splits, nseq, nkv, chunk_slots(hd) / FA_CHK) : 0;
    const int nc = fa ? 1 : attn_chunks_per_wg(wgs);
    for (int s = 0; s < nseq; ++s) {
        AttnMArgs a = as[s];
        const int ch = chunk_slots(a.hd);
        if (a.cap / ch > 1024) return hipErrorInvalidValue;  // combine weights live in LDS
        a.nc = nc;
        a.pslots = fa ? g * FA_CHK : nc * ch;
        const int nch = (int)((a.cap + a.pslots - 1) / a.pslots);  // the partials' stride
        const int64_t q = (int64_t)a.M * a.n_head;
        float* part = const_cast<float*>(parts[s]);
        a.pmax = part;
        a.psum = part + q * nch;
        a.pout = part + 2 * q * nch;
        b.s[s] = a;
        b.nch[s] = nch;
        b.qt0[s] = qt;
        b.qi0[s] = qi;
        qt += splits[s];
        qi += (int)q;
        maxch = nch > maxch ? nch : maxch;
    }
    b.qt0[nseq] = qt;
    b.qi0[nseq] = qi;
    const dim3 grid((unsigned)maxch, (unsigned)nkv, (unsigned)qt);
    if (fa) {
        hipError_t e;
        if (hd == 128)
            e = launch_fa<128>(k_attn_fa_batch<128>, grid, st, b);
        else if (hd == 64)
            e = launch_fa<64>(k_attn_fa_batch<64>, grid, st, b);
        else
            return hipErrorInvalidValue;
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_attn_combine_batch, dim3((unsigned)qi), dim3(128), 0, st, b);
        return hipGetLastError();
    }
    if (hd == 128 && nc > 1)
        ktimed_launch(k_attn_mfma_batch<128, chunk_slots(128), ATTN_WAVES_128, true>, grid,
                      dim3(64 * ATTN_WAVES_128), 0, st, b);
    else if (hd == 128)
        ktimed_launch(k_attn_mfma_batch<128, chunk_slots(128), ATTN_WAVES_128, false>, grid,
                      dim3(64 * ATTN_WAVES_128), 0, st, b);
    else if (hd == 64 && nc > 1)
        ktimed_launch(k_attn_mfma_batch<64, chunk_slots(64), 4, true>, grid, dim3(64 * 4), 0, st, b);
    else if (hd == 64)
        ktimed_launch(k_attn_mfma_batch<64, chunk_slots(64), 4, false>, grid, dim3(64 * 4), 0, st, b);
    else
        return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine_batch, dim3((unsigned)qi), dim3(128), 0, st, b);
    return hipGetLastError();
}
