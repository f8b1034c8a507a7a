// verify.hip -- the device-resident verify step: Engine::forward for M
// draft tokens (src/engine.cpp:461-596, extend_verify 669-674) with every op
// on the GPU, plus the acceptance sampler entry point.
#include <algorithm>
#include <cmath>
#include <new>

#include "ftx_internal.h"

#include <cstring>
#include "quant_dev.h"

struct ftx_model {
    ftx_ctx* ctx = nullptr;
    ftx_model_desc d{};
    std::vector<const ftx_tensor*> layers;
    int64_t qdim = 0, kdim = 0, ldq = 0, Mmax = 0;
    // F32 copies of the norm vectors
    float* norms = nullptr;  // [n_layer*2 + 1][n_embd]
    // activations
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *h = nullptr;
    float* part = nullptr;
    size_t part_floats = 0;
    // per-step arguments, one device block filled by one copy per step (the
    // pointers below are views into it, laid out as the pinned host block)
    uint8_t* args = nullptr;
    int32_t* toks = nullptr;
    int32_t* depth = nullptr;
    uint32_t* anc = nullptr;
    int64_t* npast = nullptr;
    // int8-MFMA GEMV activation operand
    int8_t* xq = nullptr;
    // rotated q as fp16 hi + lo parts for the MFMA attention, [M][n_head][hd] each
    _Float16* qhl = nullptr;
    // RoPE cos / sin per (token, pair) of the current step, [M][hd / 2][2]
    float* rcs = nullptr;  // (a view into args)
    // rope_vec's frequencies f_p = theta^(-2p / hd), p < hd / 2 (formed once;
    // a step computes only its angles' cos / sin)
    std::vector<double> rope_f;
    // per-layer re-tiled ffn_down copies for the MFMA down kernel (or null)
    std::vector<uint8_t*> down_tiled;
    // tiled copies for the int8-MFMA row-dot kernel, [layer * LAYER_TENSORS +
    // tensor] and the LM head last (null where the kernel does not apply)
    std::vector<uint8_t*> mvt;
    std::vector<int> mvt_rpt;
    // planar copies of Q8_0 / Q4_0 projections for the generic kernels (same
    // indexing; null where they do not apply) and their internal dtypes
    std::vector<uint8_t*> pln;
    std::vector<int> pln_dt;
    // the one-pass GEMM's re-tiled copies of Q8_0 / Q4_0 projections (same
    // indexing; null where they do not apply) and their internal dtypes
    std::vector<uint8_t*> mmt;
    std::vector<int> mmt_dt;
    float* downpart = nullptr;
    // large-M path (more than 8 tokens, or several sequences): activation
    // operands and split-sum partials of the k_gemm.hip launches
    _Float16* mm_act = nullptr;
    float* mm_part = nullptr;
    size_t mm_part_n = 0;
    // optional per-layer tensors (layer_ext) and what the device keeps of
    // them: any attention extra or MoE layer sends every step through
    // verify_large
    std::vector<const ftx_tensor*> ext;
    bool has_ext = false;
    std::vector<float*> attn_bias;  // [qdim + 2 kdim] q | k | v bias per layer, or null
    std::vector<float*> qnorm, knorm;  // [hd] per layer, or null
    // MoE layers: planar copies of the gate and up expert planes, the
    // re-tiled down planes, the router bias as F32; shared buffers for the
    // routing tables, the gathered operand, the down operand, split partials,
    // and tmpo for shared experts
    std::vector<uint8_t*> moe_gate, moe_up, moe_down;
    std::vector<int> moe_gu_dt;
    std::vector<float*> moe_rbias;
    void* route = nullptr;
    _Float16* moe_act = nullptr;
    _Float16* moe_h = nullptr;
    float* moe_part = nullptr;
    size_t moe_part_n = 0;
    float* tmpo = nullptr;
    int64_t F_alloc = 0;  // columns of h (the widest of n_ff and the shared experts')
    // pinned host argument blocks, used in turn; an event recorded after a
    // block's copy to the device guards its reuse, so the host prepares the
    // next step while earlier steps still run
    static constexpr int PIN_RING = 4;
    uint8_t* pin[PIN_RING] = {};
    hipEvent_t pin_ev[PIN_RING] = {};
    int pin_next = 0;
};

// Per-step argument block (pinned host copy and device copy share the
// layout): tokens [M] | depth [M] | ancestor masks [M][aw] | npast [nseq]
// (8-byte aligned) | RoPE cos / sin [M][hd / 2][2].  M counts the tokens of
// every sequence; a mask row holds bits of its own sequence's nodes.
struct StepArgsLayout {
    size_t depth, anc, np, cs, bytes;
};
static StepArgsLayout step_args_layout(int64_t M, int64_t hd, int64_t aw, int64_t nseq = 1) {
    StepArgsLayout L;
    L.depth = (size_t)M * 4;
    L.anc = L.depth + (size_t)M * 4;
    L.np = (L.anc + (size_t)(M * aw) * 4 + 7) & ~(size_t)7;
    L.cs = L.np + 8 * (size_t)nseq;
    L.bytes = L.cs + (size_t)(M * (hd / 2) * 2) * 4;
    return L;
}
static size_t step_args_bytes(int64_t Mmax, int64_t hd) {
    return step_args_layout(Mmax, hd, (Mmax + 31) / 32, FTX_MAX_SEQ).bytes;
}

// the MFMA row-dot path applies to every segment of a projection, or none
static bool mv_all(const ftx_tensor* const* ts, int n, int64_t K, int64_t M) {
    for (int i = 0; i < n; ++i)
        if (!mv_supported(ts[i]->dtype, K, M)) return false;
    return true;
}

// whether the 16x16x32 row-dot kernel (launch_rd) takes a projection whose
// segments have tiled copies with rpt[i] rows per tile
static bool rd_use(const ftx_tensor* const* ts, const int* rpt, int n, int64_t K, int64_t M,
                   int epi, int cu_count) {
    int dts[3];
    int64_t Ns[3];
    for (int i = 0; i < n && i < 3; ++i) {
        dts[i] = ts[i]->dtype;
        Ns[i] = ts[i]->nrows;
    }
    return n <= 3 && rd_take(dts, Ns, rpt, n, K, M, epi, cu_count);
}

struct ftx_kv {
    ftx_ctx* ctx = nullptr;
    int64_t n_layer = 0, cap = 0, kdim = 0, n_kv = 0, hd = 0;
    // the creating model's query heads and largest step: attn_part is sized
    // for them
    int64_t n_head = 0, mmax = 0;
    int64_t cap_alloc = 0;  // slots allocated per layer, a multiple of 128
    int kv_f16 = 1;
    void* k = nullptr;      // [n_layer][cap_alloc][kdim]
    void* v = nullptr;      // [n_layer][n_kv][hd][cap_alloc]
    float* attn_part = nullptr;  // chunk partials of the MFMA attention
    int64_t npast = 0;
};

static void model_release(ftx_model* m) {
    if (!m) return;
    void* bufs[] = {m->norms, m->x, m->xn, m->qkv, m->att, m->h, m->part, m->args, m->xq, m->qhl};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    for (uint8_t* b : m->down_tiled)
        if (b) (void)hipFree(b);
    for (uint8_t* b : m->mvt)
        if (b) (void)hipFree(b);
    for (uint8_t* b : m->pln)
        if (b) (void)hipFree(b);
    for (uint8_t* b : m->mmt)
        if (b) (void)hipFree(b);
    if (m->downpart) (void)hipFree(m->downpart);
    if (m->mm_act) (void)hipFree(m->mm_act);
    if (m->mm_part) (void)hipFree(m->mm_part);
    for (auto* v : {&m->attn_bias, &m->qnorm, &m->knorm, &m->moe_rbias})
        for (float* b : *v)
            if (b) (void)hipFree(b);
    for (auto* v : {&m->moe_gate, &m->moe_up, &m->moe_down})
        for (uint8_t* b : *v)
            if (b) (void)hipFree(b);
    void* mb[] = {m->route, m->moe_act, m->moe_h, m->moe_part, m->tmpo};
    for (void* b : mb)
        if (b) (void)hipFree(b);
    for (int i = 0; i < ftx_model::PIN_RING; ++i) {
        if (m->pin[i]) (void)hipHostFree(m->pin[i]);
        if (m->pin_ev[i]) (void)hipEventDestroy(m->pin_ev[i]);
    }
    delete m;
}

template <typename T>
static bool dalloc(T** p, size_t n) {
    if (hipMalloc((void**)p, n * sizeof(T) + 256) != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return false;
    }
    return true;
}

// The verify step for more than 8 tokens or for several sequences: every
// projection over the tokens of all sequences at once, through the one-pass
// GEMMs of k_gemm.hip where the weights allow (tiled Q4_K, planar Q8_0 /
// Q4_0 copies) and the generic kernels otherwise; RoPE, the KV write and
// attention per sequence against its own cache (Engine::forward,
// src/engine.cpp:461-596, per sequence).  The caller has checked the
// arguments.
static int verify_large(ftx_ctx* ctx, ftx_model* m, const ftx_seq_args* sq, int64_t nseq) {
    const ftx_model_desc& d = m->d;
    const int64_t D = d.n_embd, F = d.n_ff, V = d.vocab, hd = d.head_dim;
    int64_t row0[FTX_MAX_SEQ + 1];
    int64_t Mt = 0, Mmx = 0;
    for (int64_t s = 0; s < nseq; ++s) {
        row0[s] = Mt;
        Mt += sq[s].M;
        Mmx = std::max(Mmx, sq[s].M);
    }
    row0[nseq] = Mt;
    const int aw = (int)((Mmx + 31) / 32);
    const int64_t hd2 = hd / 2;
    const StepArgsLayout AL = step_args_layout(Mt, hd, aw, nseq);
    const int slot = m->pin_next;
    uint8_t* pin = m->pin[slot];
    FTX_HIP(ctx, hipEventSynchronize(m->pin_ev[slot]));
    int32_t* toks = (int32_t*)pin;
    int32_t* depth = (int32_t*)(pin + AL.depth);
    uint32_t* anc = (uint32_t*)(pin + AL.anc);
    int64_t* np = (int64_t*)(pin + AL.np);
    float* cs = (float*)(pin + AL.cs);
    for (int64_t s = 0; s < nseq; ++s) {
        const int64_t r0 = row0[s], M = sq[s].M, npast = sq[s].kv->npast;
        np[s] = npast;
        for (int64_t i = 0; i < M; ++i) {
            const int32_t t = sq[s].tokens[i];
            if (t < 0 || t >= d.vocab) return ftx_fail(ctx, FTX_E_RANGE, "token id out of range");
            const int32_t p = sq[s].parents ? sq[s].parents[i] : (int32_t)i - 1;
            if (p < -1 || p >= i) return ftx_fail(ctx, FTX_E_INVALID, "parents[i] must be in [-1, i)");
            toks[r0 + i] = t;
            depth[r0 + i] = p < 0 ? 0 : depth[r0 + p] + 1;
            uint32_t* row = anc + (r0 + i) * aw;
            for (int w = 0; w < aw; ++w) row[w] = p >= 0 ? anc[(r0 + p) * aw + w] : 0u;
            row[i / 32] |= 1u << (i % 32);
            // rope_vec's angles (src/engine.cpp:43-60) at npast + depth
            // (sincos: the values of cos and sin, in one call)
            for (int64_t q = 0; q < hd2; ++q) {
                const double ang = (double)(npast + depth[r0 + i]) * m->rope_f[(size_t)q];
                double sn, cn;
                sincos(ang, &sn, &cn);
                cs[((r0 + i) * hd2 + q) * 2] = (float)cn;
                cs[((r0 + i) * hd2 + q) * 2 + 1] = (float)sn;
            }
        }
    }
    hipStream_t st = ctx->stream;
    int32_t* d_toks = (int32_t*)m->args;
    int32_t* d_depth = (int32_t*)(m->args + AL.depth);
    uint32_t* d_anc = (uint32_t*)(m->args + AL.anc);
    int64_t* d_np = (int64_t*)(m->args + AL.np);
    float* d_cs = (float*)(m->args + AL.cs);
    FTX_HIP(ctx, hipMemcpyAsync(m->args, pin, AL.bytes, hipMemcpyHostToDevice, st));
    FTX_HIP(ctx, hipEventRecord(m->pin_ev[slot], st));
    m->pin_next = (slot + 1) % ftx_model::PIN_RING;

    const float eps = d.rms_eps;
    const double f4 = 4.0, Md = (double)Mt;
    auto wbytes = [](const ftx_tensor* t) { return (double)(t->row_bytes * t->nrows); };
#define TRACED_L(kind, bytes, call)           \
    do {                                      \
        TraceScope ts_(ctx);                  \
        FTX_HIP(ctx, call);                   \
        ts_.end((kind), (double)(bytes));     \
    } while (0)
    TRACED_L(TK_EMBED, Md * d.tok_embd->row_bytes + Md * D * f4,
             launch_embed(st, d.tok_embd->data, d.tok_embd->dtype, d.tok_embd->row_bytes, D,
                          d_toks, Mt, m->x));
    // the k_mm operand of tensor index i, if it has one
    auto mm_seg = [&](size_t i, const ftx_tensor* w, MmSeg& sg) -> bool {
        if (w->dtype == FTX_Q4_K && m->mvt[i] && mm_supported(FTX_Q4_K, w->ne[0])) {
            sg = MmSeg{m->mvt[i], FTX_Q4_K, w->nrows, m->mvt_rpt[i], 0};
            return true;
        }
        if (m->mmt[i] && mm_supported(m->mmt_dt[i], w->ne[0])) {
            sg = MmSeg{m->mmt[i], m->mmt_dt[i], w->nrows, 0, w->row_bytes};
            return true;
        }
        return false;
    };
    auto out1 = [&](float* y, int64_t ld, int accum) {
        MmOut o{};
        o.nseq = 1;
        o.base[0] = y;
        o.row0[0] = 0;
        o.row0[1] = Mt;
        o.ld = ld;
        o.accum = accum;
        return o;
    };
    // the split partials of the last o / ffn_down GEMM not yet added into x
    // (they stay in mm_part): the next activation prep over x adds them as it
    // reads x; any other reader of x first adds them by a reduce launch
    MmPend xpend{};
    auto flush_x = [&]() -> int {
        if (xpend.S > 0)
            TRACED_L(TK_XQ_PREP, (xpend.S + 2.0) * Md * D * f4, launch_mm_fold(st, xpend, Mt, m->x, D));
        xpend = MmPend{};
        return FTX_OK;
    };
    // one projection of rows [r0, r0 + Mr) of xin: [RMSNorm ->] segments ->
    // out (k_mm) or gs (generic kernels, whose outputs are the segments' y);
    // pend: an accumulating k_mm GEMM may leave its partials there
    auto project = [&](int kind, double bytes, const float* xin, int64_t ldx, const float* normw,
                       const size_t* idx, const ftx_tensor* const* ts, GemvSeg* gs, int nseg,
                       int64_t K, int epi, const MmOut& out, int64_t Mr,
                       MmPend* pend = nullptr, bool act_ready = false) -> int {
        MmSeg sg[3];
        bool all = true;
        for (int i = 0; i < nseg; ++i) all = all && mm_seg(idx[i], ts[i], sg[i]);
        for (int i = 1; all && i < nseg; ++i) all = sg[i].dt == sg[0].dt;
        if (all) {
            const MmAct act = mm_act(m->mm_act, mm_pad_tokens(Mr), K);
            if (act_ready) {
                // the producer wrote the operand
            } else if (xpend.S > 0 && xin == m->x && Mr == Mt && ldx == D) {
                TRACED_L(TK_XQ_PREP, (xpend.S + 2.0) * Mr * K * f4 + 4.0 * mm_pad_tokens(Mr) * K,
                         launch_mm_prep_fold(st, m->x, ldx, normw, eps, Mr, act, sg[0].dt, xpend));
                xpend = MmPend{};
            } else {
                if (xin >= m->x && xin < m->x + Mt * D) {
                    const int fr = flush_x();
                    if (fr) return fr;
                }
                TRACED_L(TK_XQ_PREP, Mr * K * f4 + 4.0 * mm_pad_tokens(Mr) * K,
                         launch_mm_prep(st, xin, ldx, normw, eps, Mr, act, sg[0].dt));
            }
            TRACED_L(kind, bytes,
                     launch_mm(st, sg, nseg, act, Mr, epi, out, m->mm_part, m->mm_part_n,
                               ctx->cu_count, pend));
            return FTX_OK;
        }
        // the other kernels read x as it is
        if (xin >= m->x && xin < m->x + Mt * D) {
            const int fr = flush_x();
            if (fr) return fr;
        }
        // tiled K-quants the one-pass kernels do not take (Q6_K): the
        // row-dot MFMA kernel on 8-row chunks (one activation prep for all)
        bool tiled_all = mv_all(ts, nseg, K, 8) && (epi != EPI_SWIGLU || mv_swiglu_supported(K));
        for (int i = 0; tiled_all && i < nseg; ++i) tiled_all = m->mvt[idx[i]] != nullptr;
        if (tiled_all) {
            int rpts[3] = {0, 0, 0};
            for (int i = 0; i < nseg; ++i) rpts[i] = m->mvt_rpt[idx[i]];
            const bool rd = rd_use(ts, rpts, nseg, K, 8, epi, ctx->cu_count);
            auto chunks = [&]() -> hipError_t {
                hipError_t e = launch_xq_prep(st, (float*)xin, ldx, normw, nullptr, 0, D, K, Mr, m->xq,
                                              rd);
                if (e != hipSuccess) return e;
                for (int64_t c0 = 0; c0 < Mr; c0 += 8) {
                    const int64_t mc = Mr - c0 < 8 ? Mr - c0 : 8;
                    GemvSeg cs[3];
                    for (int i = 0; i < nseg; ++i) {
                        cs[i] = gs[i];
                        cs[i].W = m->mvt[idx[i]];
                        cs[i].tiled = 1;
                        cs[i].rpt = m->mvt_rpt[idx[i]];
                        if (cs[i].y) cs[i].y += c0 * cs[i].ldy;
                    }
                    const int8_t* xc = m->xq + (c0 / 8) * (int64_t)xq_chunk_bytes(K);
                    e = rd ? launch_rd(st, cs, nseg, xc, K, mc, epi, normw != nullptr, eps)
                           : launch_mv(st, cs, nseg, xc, K, mc, epi, ctx->cu_count, normw != nullptr,
                                       eps, nullptr);
                    if (e != hipSuccess) return e;
                }
                return hipSuccess;
            };
            TRACED_L(kind, bytes, chunks());
            return FTX_OK;
        }
        bool pl_all = true;
        for (int i = 0; i < nseg; ++i) pl_all = pl_all && m->pln[idx[i]] != nullptr;
        for (int i = 0; pl_all && i < nseg; ++i) {
            gs[i].W = m->pln[idx[i]];
            gs[i].dt = m->pln_dt[idx[i]];
        }
        const float* src = xin;
        int64_t lds = ldx;
        if (normw) {
            TRACED_L(TK_RMSNORM, 2 * Mr * K * f4, launch_rmsnorm(st, xin, normw, K, Mr, eps, m->xn));
            src = m->xn;
            lds = K;
        }
        if (epi == EPI_SWIGLU)
            TRACED_L(kind, bytes,
                     launch_gemv_swiglu(st, gs[0].W, gs[1].W, gs[0].dt, gs[0].row_bytes, gs[0].N,
                                        src, lds, K, Mr, gs[0].y, gs[0].ldy, true));
        else
            TRACED_L(kind, bytes, launch_gemv(st, gs, nseg, src, lds, K, Mr, epi, true));
        return FTX_OK;
    };
    auto seg = [](const ftx_tensor* t, float* y, int64_t ldy) {
        return GemvSeg{t->data, t->dtype, t->row_bytes, t->nrows, y, ldy};
    };
    _Float16* qh = m->qhl;
    _Float16* ql = m->qhl + Mt * m->qdim;
    // The MoE FFN of layer l (src/engine.cpp:179-258), added into x: ffn_norm
    // rows, router logits, routing, the routed experts' gate / up (one-pass
    // GEMM over the gathered rows, SwiGLU into the down operand), their down,
    // the weighted sum in first-use order; a shared expert's FFN is added to
    // that sum before the sum goes into x (src/engine.cpp:243-257, 577-579).
    auto moe_layer = [&](int64_t l, const ftx_tensor* const* X) -> int {
        const int64_t E = d.n_expert, U = d.n_expert_used;
        const int64_t TR = moe_tile_rows(Mt, E, U), T = moe_tiles_max(Mt, E, U), rows = T * TR;
        const int64_t Mp = mm_pad_tokens(rows);
        const ftx_tensor* gi = X[FTX_X_GATE_INP];
        const ftx_tensor *ge = X[FTX_X_GATE_EXPS], *de = X[FTX_X_DOWN_EXPS];
        const MoeRoute rt = moe_route_view(m->route, m->Mmax, E, U);
        TRACED_L(TK_MOE_ROUTE, wbytes(gi) + 2 * Md * D * f4 + 4.0 * Md * U * f4,
                 launch_moe_route(st, m->x, m->norms + (l * 2 + 1) * D, eps, m->xn, D, gi->data,
                                  gi->dtype, gi->row_bytes, m->moe_rbias[l], Mt, E, U, rt));
        const int gdt = m->moe_gu_dt[l];
        const MmAct act = mm_act(m->moe_act, Mp, D);
        TRACED_L(TK_XQ_PREP, Md * U * D * f4 + 4.0 * rows * D,
                 launch_mm_prep(st, m->xn, D, nullptr, eps, rows, act, gdt, rt.slot_tok));
        // every plane is read at most once; the routed planes are what moves
        const double plane_gu = (double)(ge->row_bytes * F);
        const double used = (double)std::min<int64_t>(E, Mt * U);
        MmSeg gs[2] = {MmSeg{m->moe_gate[l], gdt, F, 0, ge->row_bytes},
                       MmSeg{m->moe_up[l], gdt, F, 0, ge->row_bytes}};
        const int64_t pb = (int64_t)mm_tiled_bytes(gdt, F, D);
        const int64_t plane[2] = {pb, pb};
        MmFragOut fo{m->moe_h, m->moe_h + Mp * F, 1.f, F};
        TRACED_L(TK_GEMV_SWIGLU, 2 * used * plane_gu + Md * U * D * 4.0 + Md * U * F * 4.0,
                 launch_mm_experts(st, gs, 2, plane, act, rt.tab, T, TR, fo, m->moe_part,
                                   m->moe_part_n, ctx->cu_count));
        const int S = moe_down_splits(F, D, T, ctx->cu_count);
        TRACED_L(TK_DOWN, used * (double)(de->row_bytes * F) + Md * U * F * 4.0 + S * Md * U * D * f4,
                 launch_moe_down(st, m->moe_down[l], de->dtype, F, D, fo.h, fo.l, rt.tab, T, TR,
                                 S, m->moe_part, m->moe_part_n));
        const ftx_tensor *sg = X[FTX_X_GATE_SH], *su = X[FTX_X_UP_SH], *sd = X[FTX_X_DOWN_SH];
        TRACED_L(TK_MOE_COMBINE, S * Md * U * D * f4 + 2 * Md * D * f4,
                 launch_moe_combine(st, m->moe_part, S, rows, D, rt, Mt, U, sg ? m->tmpo : m->x,
                                    sg ? 0 : 1));
        if (sg) {
            // the shared expert over all rows (generic kernels), into tmpo
            const int64_t FS = sg->nrows;
            TRACED_L(TK_GEMV_SWIGLU, wbytes(sg) + wbytes(su) + Md * D * f4 + Md * FS * f4,
                     launch_gemv_swiglu(st, sg->data, su->data, sg->dtype, sg->row_bytes, FS,
                                        m->xn, D, D, Mt, m->h, FS, true));
            TRACED_L(TK_DOWN, wbytes(sd) + Md * FS * f4 + 2 * Md * D * f4,
                     launch_down(st, sd->data, sd->dtype, sd->row_bytes, FS, D, m->h, FS, Mt,
                                 m->tmpo, D, m->part));
            TRACED_L(TK_MOE_COMBINE, 3 * Md * D * f4, launch_add(st, m->tmpo, m->x, Mt * D));
        }
        return FTX_OK;
    };
    int rc;
    for (int64_t l = 0; l < d.n_layer; ++l) {
        const int64_t lt = l * FTX_LAYER_TENSORS;
        const ftx_tensor* const* T = m->layers.data() + lt;
        // q / k / v into qkv [Mt][ldq] (its split partials, if any, summed
        // by RoPE)
        MmPend qpend{};
        {
            const ftx_tensor* ts[3] = {T[FTX_T_Q], T[FTX_T_K], T[FTX_T_V]};
            const size_t idx[3] = {(size_t)(lt + FTX_T_Q), (size_t)(lt + FTX_T_K),
                                   (size_t)(lt + FTX_T_V)};
            GemvSeg gs[3] = {seg(T[FTX_T_Q], m->qkv, m->ldq),
                             seg(T[FTX_T_K], m->qkv + m->qdim, m->ldq),
                             seg(T[FTX_T_V], m->qkv + m->qdim + m->kdim, m->ldq)};
            rc = project(TK_GEMV_QKV,
                         wbytes(ts[0]) + wbytes(ts[1]) + wbytes(ts[2]) + Md * D * f4 +
                             Md * m->ldq * f4,
                         m->x, D, m->norms + (l * 2) * D, idx, ts, gs, 3, D, EPI_STORE,
                         out1(m->qkv, m->ldq, 0), Mt, &qpend);
            if (rc) return rc;
        }
        // RoPE, the KV write and attention: one launch each over all
        // sequences when every sequence takes the MFMA attention, else per
        // sequence
        bool all_mattn = nseq > 1;
        for (int64_t s = 0; s < nseq && all_mattn; ++s)
            all_mattn = attn_mfma_supported(hd, sq[s].kv->kv_f16, sq[s].M, d.n_head, d.n_head_kv);
        // the attention combine writes the o projection's one-pass GEMM
        // operand when every sequence takes the MFMA attention (its prep is
        // then skipped)
        MmFragDst ofd{};
        {
            MmSeg oseg;
            bool of = mm_seg((size_t)(lt + FTX_T_O), T[FTX_T_O], oseg);
            for (int64_t s = 0; s < nseq && of; ++s)
                of = attn_mfma_supported(hd, sq[s].kv->kv_f16, sq[s].M, d.n_head, d.n_head_kv);
            if (of) {
                const MmAct oact = mm_act(m->mm_act, mm_pad_tokens(Mt), m->qdim);
                ofd = MmFragDst{oact.xh, oact.xl, oact.sh, oact.sl, 0, m->qdim,
                                oseg.dt == FTX_Q4_0_MMT ? 1 : 0};
            }
        }
        if (all_mattn) {
            RopeArgs ras[FTX_MAX_SEQ];
            AttnMArgs ams[FTX_MAX_SEQ];
            const float* parts[FTX_MAX_SEQ];
            int64_t Ms[FTX_MAX_SEQ];
            double rope_b = 0.0, attn_b = 0.0;
            for (int64_t s = 0; s < nseq; ++s) {
                ftx_kv* kv = sq[s].kv;
                const int64_t r0 = row0[s], M = sq[s].M, npast = kv->npast;
                const size_t kvel = 2;
                uint8_t* kl = (uint8_t*)kv->k + (size_t)(l * kv->cap_alloc * kv->kdim) * kvel;
                uint8_t* vl = (uint8_t*)kv->v + (size_t)(l * kv->cap_alloc * kv->kdim) * kvel;
                RopeArgs ra{m->qkv + r0 * m->ldq, m->ldq,  d.n_head,   d.n_head_kv, hd,
                            d_depth + r0,         d_np + s, d.rope_theta, d.rope_neox, kl,
                            vl,                   kv->kv_f16, kv->cap_alloc};
                ra.bias = m->attn_bias[l];
                ra.qnorm = m->qnorm[l];
                ra.knorm = m->knorm[l];
                ra.eps = eps;
                ra.qh16 = qh + r0 * m->qdim;
                ra.ql16 = ql + r0 * m->qdim;
                if (qpend.S > 0) {
                    ra.part = qpend.part + r0 * qpend.ldp;
                    ra.split_stride = qpend.split_stride;
                    ra.ldp = qpend.ldp;
                    ra.S = qpend.S;
                }
                ra.cs = d_cs + r0 * hd2 * 2;
                ras[s] = ra;
                Ms[s] = M;
                AttnMArgs am{};
                am.qkv = m->qkv + r0 * m->ldq;
                am.ldq = m->ldq;
                am.qh16 = ra.qh16;
                am.ql16 = ra.ql16;
                am.kc = (const _Float16*)kl;
                am.vt = (const _Float16*)vl;
                am.cap = kv->cap_alloc;
                am.npast = npast;
                am.anc = d_anc + r0 * aw;
                am.anc_words = aw;
                am.M = (int)M;
                am.n_head = (int)d.n_head;
                am.n_kv = (int)d.n_head_kv;
                am.hd = (int)hd;
                am.out = m->att + r0 * m->qdim;
                am.frag = ofd;
                am.frag.row0 = r0;
                ams[s] = am;
                parts[s] = kv->attn_part;
                rope_b += 2.0 * M * m->ldq * f4 + 2.0 * M * m->kdim * (double)kvel;
                attn_b += 2.0 * (double)(npast + M) * m->kdim * (double)kvel + 2.0 * M * m->qdim * f4;
            }
            TRACED_L(TK_ROPE_KV, rope_b, launch_rope_kv_batch(st, ras, Ms, (int)nseq));
            TRACED_L(TK_ATTENTION, attn_b, launch_attn_mfma_batch(st, ams, parts, (int)nseq));
        }
        for (int64_t s = 0; s < nseq && !all_mattn; ++s) {
            ftx_kv* kv = sq[s].kv;
            const int64_t r0 = row0[s], M = sq[s].M, npast = kv->npast;
            const size_t kvel = kv->kv_f16 ? 2 : 4;
            uint8_t* kl = (uint8_t*)kv->k + (size_t)(l * kv->cap_alloc * kv->kdim) * kvel;
            uint8_t* vl = (uint8_t*)kv->v + (size_t)(l * kv->cap_alloc * kv->kdim) * kvel;
            const bool mattn = attn_mfma_supported(hd, kv->kv_f16, M, d.n_head, d.n_head_kv);
            RopeArgs ra{m->qkv + r0 * m->ldq, m->ldq,  d.n_head,   d.n_head_kv, hd,
                        d_depth + r0,         d_np + s, d.rope_theta, d.rope_neox, kl,
                        vl,                   kv->kv_f16, kv->cap_alloc};
            ra.bias = m->attn_bias[l];
            ra.qnorm = m->qnorm[l];
            ra.knorm = m->knorm[l];
            ra.eps = eps;
            if (qpend.S > 0) {
                ra.part = qpend.part + r0 * qpend.ldp;
                ra.split_stride = qpend.split_stride;
                ra.ldp = qpend.ldp;
                ra.S = qpend.S;
            }
            ra.cs = d_cs + r0 * hd2 * 2;
            if (mattn) {
                ra.qh16 = qh + r0 * m->qdim;
                ra.ql16 = ql + r0 * m->qdim;
            }
            TRACED_L(TK_ROPE_KV, 2.0 * M * m->ldq * f4 + 2.0 * M * m->kdim * (double)kvel,
                     launch_rope_kv(st, ra, M));
            const double attn_b =
                2.0 * (double)(npast + M) * m->kdim * (double)kvel + 2.0 * M * m->qdim * f4;
            if (mattn) {
                AttnMArgs am{};
                am.qkv = m->qkv + r0 * m->ldq;
                am.ldq = m->ldq;
                am.qh16 = ra.qh16;
                am.ql16 = ra.ql16;
                am.kc = (const _Float16*)kl;
                am.vt = (const _Float16*)vl;
                am.cap = kv->cap_alloc;
                am.npast = npast;
                am.anc = d_anc + r0 * aw;
                am.anc_words = aw;
                am.M = (int)M;
                am.n_head = (int)d.n_head;
                am.n_kv = (int)d.n_head_kv;
                am.hd = (int)hd;
                am.out = m->att + r0 * m->qdim;
                am.frag = ofd;
                am.frag.row0 = r0;
                TRACED_L(TK_ATTENTION, attn_b, launch_attn_mfma(st, am, kv->attn_part, nullptr));
            } else {
                AttnArgs aa{m->qkv + r0 * m->ldq, m->ldq, kl, vl, kv->kv_f16, d_np + s,
                            d_anc + r0 * aw, aw, d.n_head, d.n_head_kv, hd, npast + M,
                            m->att + r0 * m->qdim, kv->cap_alloc};
                TRACED_L(TK_ATTENTION, attn_b, launch_attention(st, aa, M));
            }
        }
        const ftx_tensor* const* X = m->ext.data() + l * FTX_LAYER_EXT;
        // o, added into x (a dense FFN's prep adds its partials)
        {
            const size_t idx[1] = {(size_t)(lt + FTX_T_O)};
            GemvSeg gs[1] = {seg(T[FTX_T_O], m->x, D)};
            if (const int fr = flush_x()) return fr;
            rc = project(TK_GEMV_O, wbytes(T[FTX_T_O]) + Md * m->qdim * f4 + 2 * Md * D * f4, m->att,
                         m->qdim, nullptr, idx, &T[FTX_T_O], gs, 1, m->qdim, EPI_ACCUM,
                         out1(m->x, D, 1), Mt, X[FTX_X_GATE_INP] ? nullptr : &xpend,
                         ofd.xh != nullptr);
            if (rc) return rc;
        }
        if (X[FTX_X_GATE_INP]) {
            rc = moe_layer(l, X);
            if (rc) return rc;
            continue;
        }
        // gate / up with SwiGLU into h
        {
            const ftx_tensor* ts[2] = {T[FTX_T_GATE], T[FTX_T_UP]};
            const size_t idx[2] = {(size_t)(lt + FTX_T_GATE), (size_t)(lt + FTX_T_UP)};
            GemvSeg gs[2] = {seg(T[FTX_T_GATE], m->h, F), seg(T[FTX_T_UP], nullptr, 0)};
            rc = project(TK_GEMV_SWIGLU,
                         wbytes(ts[0]) + wbytes(ts[1]) + Md * D * f4 + Md * F * f4, m->x, D,
                         m->norms + (l * 2 + 1) * D, idx, ts, gs, 2, D, EPI_SWIGLU,
                         out1(m->h, F, 0), Mt);
            if (rc) return rc;
        }
        // ffn_down, added into x
        const ftx_tensor* dn = T[FTX_T_DOWN];
        const double down_b = wbytes(dn) + Md * F * f4 + 2 * Md * D * f4;
        if (const int fr = flush_x()) return fr;
        if (m->down_tiled[l] && mm_down_supported(dn->dtype, F, D)) {
            // added into x by the next prep
            TRACED_L(TK_DOWN, down_b,
                     launch_mm_down(st, m->down_tiled[l], F, D, m->h, F, Mt, out1(m->x, D, 1),
                                    m->mm_part, m->mm_part_n, ctx->cu_count, &xpend));
        } else if (m->down_tiled[l] && down_mfma_supported(dn->dtype, F, D, 8)) {
            // the MFMA down kernel on 8-row chunks, every chunk's split
            // partials added into x by one reduce
            auto chunks = [&]() -> hipError_t {
                int S = 0;
                for (int64_t c0 = 0; c0 < Mt; c0 += 8) {
                    const int64_t mc = Mt - c0 < 8 ? Mt - c0 : 8;
                    float* pc = m->downpart + (S ? (c0 / 8) * (int64_t)S * 8 * D : 0);
                    hipError_t e = launch_down_mfma(st, dn->dtype, m->down_tiled[l], F, D,
                                                    m->h + c0 * F, F, mc, m->x + c0 * D, D, pc,
                                                    ctx->cu_count, &S);
                    if (e != hipSuccess) return e;
                }
                return launch_part_reduce(st, m->downpart, S, D, Mt, m->x, D);
            };
            TRACED_L(TK_DOWN, down_b, chunks());
        } else {
            TRACED_L(TK_DOWN, down_b,
                     launch_down(st, dn->data, dn->dtype, dn->row_bytes, F, D, m->h, F, Mt, m->x,
                                 D, m->part));
        }
    }
    // the LM head, each sequence's rows into its own logits (without one,
    // x is left complete)
    if (!sq[0].logits) {
        if (const int fr = flush_x()) return fr;
    }
    if (sq[0].logits) {
        const ftx_tensor* lm = d.output ? d.output : d.tok_embd;
        const size_t idx[1] = {(size_t)(d.n_layer * FTX_LAYER_TENSORS)};
        MmSeg probe;
        if (mm_seg(idx[0], lm, probe) || nseq == 1) {
            MmOut o{};
            o.nseq = (int)nseq;
            for (int64_t s = 0; s < nseq; ++s) {
                o.base[s] = sq[s].logits;
                o.row0[s] = row0[s];
            }
            o.row0[nseq] = Mt;
            o.ld = V;
            GemvSeg gs[1] = {seg(lm, sq[0].logits, V)};
            rc = project(TK_HEAD, wbytes(lm) + Md * D * f4 + Md * V * f4, m->x, D,
                         m->norms + (d.n_layer * 2) * D, idx, &lm, gs, 1, D, EPI_STORE, o, Mt);
            if (rc) return rc;
        } else {
            // the generic head per sequence (its weights are read once each)
            if (const int fr = flush_x()) return fr;
            for (int64_t s = 0; s < nseq; ++s) {
                const int64_t M = sq[s].M;
                GemvSeg gs[1] = {seg(lm, sq[s].logits, V)};
                rc = project(TK_HEAD, wbytes(lm) + M * D * f4 + M * V * f4, m->x + row0[s] * D,
                             D, m->norms + (d.n_layer * 2) * D, idx, &lm, gs, 1, D, EPI_STORE,
                             out1(sq[s].logits, V, 0), M);
                if (rc) return rc;
            }
        }
    }
#undef TRACED_L
    for (int64_t s = 0; s < nseq; ++s)
        if (sq[s].advance) sq[s].kv->npast += sq[s].M;
    return FTX_OK;
}

// checks of one sequence's arguments against the model and its cache
static int check_seq(ftx_ctx* ctx, const ftx_model* m, const ftx_kv* kv, int64_t M,
                     const int32_t* tokens) {
    const ftx_model_desc& d = m->d;
    if (!kv || !tokens) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (M < 1 || M > m->Mmax) return ftx_fail(ctx, FTX_E_INVALID, "M out of range");
    if (kv->n_layer != d.n_layer || kv->kdim != m->kdim || kv->n_kv != d.n_head_kv ||
        kv->hd != d.head_dim || kv->n_head != d.n_head)
        return ftx_fail(ctx, FTX_E_INVALID, "kv cache does not match the model");
    if (M > kv->mmax)
        return ftx_fail(ctx, FTX_E_INVALID, "M above the max_tokens of the kv cache's model");
    if (kv->npast + M > kv->cap) return ftx_fail(ctx, FTX_E_RANGE, "kv capacity exceeded");
    return FTX_OK;
}

extern "C" {

int ftx_model_create(ftx_ctx* ctx, const ftx_model_desc* d, ftx_model** out) {
    if (!ctx || !d || !out || !d->layers || !d->tok_embd || !d->out_norm)
        return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    *out = nullptr;
    if (d->n_layer < 1 || d->n_embd < 1 || d->n_head < 1 || d->n_head_kv < 1 ||
        d->n_head % d->n_head_kv || d->head_dim < 2 || d->head_dim % 2 || d->n_ff < 1 ||
        d->vocab < 1)
        return ftx_fail(ctx, FTX_E_INVALID, "bad model hyper-parameters");
    const int64_t Mmax = d->max_tokens > 0 ? d->max_tokens : 64;
    if (Mmax > 256) return ftx_fail(ctx, FTX_E_INVALID, "max_tokens above 256");
    const int64_t D = d->n_embd, qdim = d->n_head * d->head_dim, kdim = d->n_head_kv * d->head_dim;
    auto need = [&](const ftx_tensor* t, int64_t cols, int64_t rows, const char* nm) -> int {
        if (!t) return ftx_fail(ctx, FTX_E_INVALID, std::string("missing tensor ") + nm);
        if (t->ne[0] != cols || t->nrows != rows)
            return ftx_fail(ctx, FTX_E_INVALID, std::string("bad shape of tensor ") + nm);
        return FTX_OK;
    };
    int rc;
    if ((rc = need(d->tok_embd, D, d->vocab, "tok_embd"))) return rc;
    if ((rc = need(d->out_norm, D, 1, "out_norm"))) return rc;
    if (d->output && (rc = need(d->output, D, d->vocab, "output"))) return rc;
    // a vector of n values (stored [n] or [1, n])
    auto need_vec = [&](const ftx_tensor* t, int64_t n, const char* nm) -> int {
        if (t->ne[0] * t->nrows != n)
            return ftx_fail(ctx, FTX_E_INVALID, std::string("bad shape of tensor ") + nm);
        return FTX_OK;
    };
    const int64_t E = d->n_expert, U = d->n_expert_used;
    bool any_moe = false, any_ext = false;
    int64_t F_sh = 0;
    for (int64_t l = 0; l < d->n_layer; ++l) {
        const ftx_tensor* const* T = d->layers + l * FTX_LAYER_TENSORS;
        const ftx_tensor* const* X = d->layer_ext ? d->layer_ext + l * FTX_LAYER_EXT : nullptr;
        auto x = [&](int i) { return X ? X[i] : nullptr; };
        if ((rc = need(T[FTX_T_ATTN_NORM], D, 1, "attn_norm")) ||
            (rc = need(T[FTX_T_Q], D, qdim, "attn_q")) ||
            (rc = need(T[FTX_T_K], D, kdim, "attn_k")) ||
            (rc = need(T[FTX_T_V], D, kdim, "attn_v")) ||
            (rc = need(T[FTX_T_O], qdim, D, "attn_output")) ||
            (rc = need(T[FTX_T_FFN_NORM], D, 1, "ffn_norm")))
            return rc;
        const int64_t vn[5] = {qdim, kdim, kdim, d->head_dim, d->head_dim};
        static const char* const vnm[5] = {"attn_q.bias", "attn_k.bias", "attn_v.bias",
                                           "attn_q_norm", "attn_k_norm"};
        for (int i = 0; i < 5; ++i)
            if (x(i)) {
                if ((rc = need_vec(x(i), vn[i], vnm[i]))) return rc;
                any_ext = true;
            }
        if (x(FTX_X_GATE_INP)) {
            // MoE layer (src/engine.cpp:348-369)
            any_moe = true;
            if (E < 2 || E > 256 || U < 1 || U > 8 || U > E || (D + E) * 4 > 65536)
                return ftx_fail(ctx, FTX_E_UNSUPPORTED,
                                "MoE: n_expert must be in [2, 256], n_expert_used in [1, min(8, "
                                "n_expert)], n_embd + n_expert <= 16384");
            const ftx_tensor *ge = x(FTX_X_GATE_EXPS), *ue = x(FTX_X_UP_EXPS), *de = x(FTX_X_DOWN_EXPS);
            if ((rc = need(x(FTX_X_GATE_INP), D, E, "ffn_gate_inp"))) return rc;
            if (!ge || !ue || !de)
                return ftx_fail(ctx, FTX_E_INVALID, "incomplete MoE tensors at a layer");
            for (const ftx_tensor* t : {ge, ue, de})
                if (t->ne[0] != D || t->ne[1] != d->n_ff || t->ne[2] != E || t->ne[3] != 1)
                    return ftx_fail(ctx, FTX_E_INVALID, "bad shape of an expert tensor");
            if (ge->dtype != ue->dtype || (ge->dtype != FTX_Q4_0 && ge->dtype != FTX_Q8_0) ||
                !mm_supported(mm_tiled_dtype(ge->dtype, D), D))
                return ftx_fail(ctx, FTX_E_UNSUPPORTED,
                                "MoE gate / up experts must share Q4_0 or Q8_0 with n_embd % 256 == 0");
            if (!moe_down_supported(de->dtype, d->n_ff, D))
                return ftx_fail(ctx, FTX_E_UNSUPPORTED,
                                "MoE down experts must be Q4_0 with n_ff % 32 == 0, n_embd % 256 == 0");
            if (x(FTX_X_ROUTER_BIAS) && (rc = need_vec(x(FTX_X_ROUTER_BIAS), E, "exp_probs_b")))
                return rc;
            const ftx_tensor *sg = x(FTX_X_GATE_SH), *su = x(FTX_X_UP_SH), *sd = x(FTX_X_DOWN_SH);
            if (sg || su || sd) {
                if (!sg || !su || !sd) return ftx_fail(ctx, FTX_E_INVALID, "incomplete shared expert");
                const int64_t fs = sg->nrows;
                if ((rc = need(sg, D, fs, "ffn_gate_shexp")) || (rc = need(su, D, fs, "ffn_up_shexp")) ||
                    (rc = need(sd, D, fs, "ffn_down_shexp")))
                    return rc;
                if (sg->dtype != su->dtype)
                    return ftx_fail(ctx, FTX_E_UNSUPPORTED, "shared gate and up must share a dtype");
                F_sh = std::max(F_sh, fs);
            }
            continue;
        }
        if ((rc = need(T[FTX_T_GATE], D, d->n_ff, "ffn_gate")) ||
            (rc = need(T[FTX_T_UP], D, d->n_ff, "ffn_up")) ||
            (rc = need(T[FTX_T_DOWN], D, d->n_ff, "ffn_down")))
            return rc;
        if (T[FTX_T_GATE]->dtype != T[FTX_T_UP]->dtype)
            return ftx_fail(ctx, FTX_E_UNSUPPORTED, "ffn_gate and ffn_up must share a dtype");
    }
    ftx_model* m = new (std::nothrow) ftx_model;
    if (!m) return ftx_fail(ctx, FTX_E_NOMEM, "host allocation failed");
    m->ctx = ctx;
    m->d = *d;
    // (the same expression as rope_vec's, src/engine.cpp:43-60)
    m->rope_f.resize((size_t)(d->head_dim / 2));
    for (int64_t p = 0; p < d->head_dim / 2; ++p)
        m->rope_f[(size_t)p] = std::pow(d->rope_theta, -2.0 * (double)p / (double)d->head_dim);
    m->layers.assign(d->layers, d->layers + d->n_layer * FTX_LAYER_TENSORS);
    m->d.layers = nullptr;
    m->ext.assign((size_t)(d->n_layer * FTX_LAYER_EXT), nullptr);
    if (d->layer_ext) m->ext.assign(d->layer_ext, d->layer_ext + d->n_layer * FTX_LAYER_EXT);
    m->d.layer_ext = nullptr;
    m->has_ext = any_moe || any_ext;
    m->F_alloc = std::max(d->n_ff, F_sh);
    m->qdim = qdim;
    m->kdim = kdim;
    m->ldq = qdim + 2 * kdim;
    m->Mmax = Mmax;
    m->part_floats = down_scratch_floats(Mmax, d->n_ff, D);
    if (F_sh) m->part_floats = std::max(m->part_floats, down_scratch_floats(Mmax, F_sh, D));
    const size_t nn = (size_t)(d->n_layer * 2 + 1);
    bool ok = dalloc(&m->norms, nn * D) && dalloc(&m->x, Mmax * D) && dalloc(&m->xn, Mmax * D) &&
              dalloc(&m->qkv, Mmax * m->ldq) && dalloc(&m->att, Mmax * qdim) &&
              dalloc(&m->h, Mmax * m->F_alloc) && dalloc(&m->part, m->part_floats) &&
              dalloc(&m->args, step_args_bytes(Mmax, d->head_dim));
    for (int i = 0; ok && i < ftx_model::PIN_RING; ++i) {
        ok = hipHostMalloc((void**)&m->pin[i], step_args_bytes(Mmax, d->head_dim),
                           hipHostMallocDefault) == hipSuccess &&
             hipEventCreateWithFlags(&m->pin_ev[i], hipEventDisableTiming) == hipSuccess;
        if (!ok) (void)hipGetLastError();
    }
    if (ok) {
        const int64_t Kmax = std::max(D, qdim);
        ok = dalloc(&m->xq, (size_t)((Mmax + 7) / 8) * xq_chunk_bytes(Kmax)) &&
             dalloc(&m->qhl, (size_t)(2 * Mmax * qdim));
    }
    // re-tiled ffn_down copies (same bytes, MFMA-friendly order)
    m->down_tiled.assign((size_t)d->n_layer, nullptr);
    bool any_tiled = false;
    for (int64_t l = 0; ok && l < d->n_layer; ++l) {
        const ftx_tensor* dn = d->layers[l * FTX_LAYER_TENSORS + FTX_T_DOWN];
        if (!dn || !down_mfma_supported(dn->dtype, d->n_ff, D, 1)) continue;
        uint8_t* buf = nullptr;
        if (!dalloc(&buf, down_tiled_bytes(dn->dtype, d->n_ff, D))) {
            ok = false;
            break;
        }
        m->down_tiled[l] = buf;
        any_tiled = true;
        if (launch_down_tile(ctx->stream, dn->data, dn->row_bytes, dn->dtype, d->n_ff, D, buf) !=
            hipSuccess)
            ok = false;
    }
    if (ok && any_tiled) {
        size_t pf = 0;
        for (int dt : {FTX_Q4_K, FTX_Q6_K})
            pf = std::max(pf, down_mfma_part_floats(dt, d->n_ff, D, Mmax, ctx->cu_count));
        ok = dalloc(&m->downpart, pf);
    }
    // row-dot projections and the LM head: tiled copies for the MFMA kernel
    const size_t nmvt = (size_t)(d->n_layer * FTX_LAYER_TENSORS + 1);
    m->mvt.assign(nmvt, nullptr);
    m->mvt_rpt.assign(nmvt, 0);
    for (size_t i = 0; ok && i < nmvt; ++i) {
        const int t = (int)(i % FTX_LAYER_TENSORS);
        const bool head = i + 1 == nmvt;
        if (!head && t != FTX_T_Q && t != FTX_T_K && t != FTX_T_V && t != FTX_T_O &&
            t != FTX_T_GATE && t != FTX_T_UP)
            continue;
        const ftx_tensor* w = head ? (d->output ? d->output : d->tok_embd) : d->layers[i];
        if (!w || !mv_supported(w->dtype, w->ne[0], 1)) continue;
        const int rpt = mv_tile_rows(w->nrows, ctx->cu_count);
        uint8_t* buf = nullptr;
        if (!dalloc(&buf, mv_tiled_bytes(w->dtype, w->nrows, w->ne[0], rpt))) {
            ok = false;
            break;
        }
        m->mvt[i] = buf;
        m->mvt_rpt[i] = rpt;
        if (launch_mv_tile(ctx->stream, w->data, w->row_bytes, w->dtype, w->nrows, w->ne[0], rpt,
                           buf) != hipSuccess)
            ok = false;
    }
    m->pln.assign(nmvt, nullptr);
    m->pln_dt.assign(nmvt, -1);
    for (size_t i = 0; ok && i < nmvt; ++i) {
        const int t = (int)(i % FTX_LAYER_TENSORS);
        const bool head = i + 1 == nmvt;
        if (!head && t != FTX_T_Q && t != FTX_T_K && t != FTX_T_V && t != FTX_T_O &&
            t != FTX_T_GATE && t != FTX_T_UP)
            continue;
        const ftx_tensor* w = head ? (d->output ? d->output : d->tok_embd) : d->layers[i];
        if (!w) continue;
        const int pdt = planar_dtype(w->dtype, w->ne[0]);
        if (pdt < 0 || w->row_bytes * 32 != w->ne[0] * (w->dtype == FTX_Q8_0 ? 34 : 18)) continue;
        uint8_t* buf = nullptr;
        if (!dalloc(&buf, (size_t)(w->row_bytes * w->nrows))) {
            ok = false;
            break;
        }
        m->pln[i] = buf;
        m->pln_dt[i] = pdt;
        if (launch_planar(ctx->stream, w->data, w->dtype, w->nrows, w->ne[0], buf) != hipSuccess)
            ok = false;
    }
    m->mmt.assign(nmvt, nullptr);
    m->mmt_dt.assign(nmvt, -1);
    for (size_t i = 0; ok && i < nmvt; ++i) {
        const int t = (int)(i % FTX_LAYER_TENSORS);
        const bool head = i + 1 == nmvt;
        if (!head && t != FTX_T_Q && t != FTX_T_K && t != FTX_T_V && t != FTX_T_O &&
            t != FTX_T_GATE && t != FTX_T_UP)
            continue;
        const ftx_tensor* w = head ? (d->output ? d->output : d->tok_embd) : d->layers[i];
        if (!w) continue;
        const int mdt = mm_tiled_dtype(w->dtype, w->ne[0]);
        if (mdt < 0 || !mm_supported(mdt, w->ne[0])) continue;
        if (mdt == FTX_Q6_K_MMT && m->Mmax <= 8) continue;  // only the large-M path reads it
        uint8_t* buf = nullptr;
        if (!dalloc(&buf, mm_tiled_bytes(mdt, w->nrows, w->ne[0]))) {
            ok = false;
            break;
        }
        m->mmt[i] = buf;
        m->mmt_dt[i] = mdt;
        if (launch_mm_tile(ctx->stream, w->data, w->dtype, w->nrows, 1, w->ne[0], buf) != hipSuccess)
            ok = false;
    }
    // the large-M path (more than 8 tokens, or several sequences):
    // activation operands for the widest contraction and split-sum partials
    // for the widest projection (SwiGLU's gate and up sums always pass
    // through them)
    if (ok) {
        const int64_t Mp = mm_pad_tokens(Mmax), Kmax = std::max(D, qdim);
        const int cu = ctx->cu_count;
        size_t pf = (size_t)Mp * 2 * (size_t)d->n_ff;
        auto upd = [&](int64_t N, int64_t K) {
            pf = std::max(pf, mm_part_floats(Mp, N, K / 256, (N + 255) / 256, cu));
        };
        upd(qdim + 2 * kdim, D);
        upd(D, qdim);
        upd(2 * d->n_ff, D);
        pf = std::max(pf, mm_down_part_floats(Mp, d->n_ff, D, cu));
        ok = dalloc(&m->mm_act, mm_act_halves(Mp, Kmax)) && dalloc(&m->mm_part, pf);
        m->mm_part_n = pf;
    }
    // attention extras as F32 vectors (absent parts of a present bias are zero)
    m->attn_bias.assign((size_t)d->n_layer, nullptr);
    m->qnorm.assign((size_t)d->n_layer, nullptr);
    m->knorm.assign((size_t)d->n_layer, nullptr);
    auto vec_f32 = [&](const ftx_tensor* t, float* dst) {
        return launch_dequant(ctx->stream, t->data, t->dtype, t->row_bytes, t->ne[0], t->nrows,
                              dst) == hipSuccess;
    };
    for (int64_t l = 0; ok && l < d->n_layer; ++l) {
        const ftx_tensor* const* X = m->ext.data() + l * FTX_LAYER_EXT;
        if (X[FTX_X_Q_BIAS] || X[FTX_X_K_BIAS] || X[FTX_X_V_BIAS]) {
            ok = dalloc(&m->attn_bias[l], (size_t)m->ldq) &&
                 hipMemsetAsync(m->attn_bias[l], 0, (size_t)m->ldq * 4, ctx->stream) == hipSuccess;
            const int64_t at[3] = {0, qdim, qdim + kdim};
            for (int i = 0; ok && i < 3; ++i)
                if (X[FTX_X_Q_BIAS + i]) ok = vec_f32(X[FTX_X_Q_BIAS + i], m->attn_bias[l] + at[i]);
        }
        if (ok && X[FTX_X_Q_NORM])
            ok = dalloc(&m->qnorm[l], (size_t)d->head_dim) && vec_f32(X[FTX_X_Q_NORM], m->qnorm[l]);
        if (ok && X[FTX_X_K_NORM])
            ok = dalloc(&m->knorm[l], (size_t)d->head_dim) && vec_f32(X[FTX_X_K_NORM], m->knorm[l]);
    }
    // MoE: per-layer copies and the shared buffers
    m->moe_gate.assign((size_t)d->n_layer, nullptr);
    m->moe_up.assign((size_t)d->n_layer, nullptr);
    m->moe_down.assign((size_t)d->n_layer, nullptr);
    m->moe_gu_dt.assign((size_t)d->n_layer, -1);
    m->moe_rbias.assign((size_t)d->n_layer, nullptr);
    for (int64_t l = 0; ok && any_moe && l < d->n_layer; ++l) {
        const ftx_tensor* const* X = m->ext.data() + l * FTX_LAYER_EXT;
        if (!X[FTX_X_GATE_INP]) continue;
        const ftx_tensor *ge = X[FTX_X_GATE_EXPS], *ue = X[FTX_X_UP_EXPS], *de = X[FTX_X_DOWN_EXPS];
        m->moe_gu_dt[l] = mm_tiled_dtype(ge->dtype, D);
        const size_t gub = E * mm_tiled_bytes(m->moe_gu_dt[l], d->n_ff, D);
        ok = dalloc(&m->moe_gate[l], gub) && dalloc(&m->moe_up[l], gub) &&
             dalloc(&m->moe_down[l], moe_down_tiled_bytes(de->dtype, d->n_ff, D, E));
        ok = ok &&
             launch_mm_tile(ctx->stream, ge->data, ge->dtype, d->n_ff, E, D, m->moe_gate[l]) ==
                 hipSuccess &&
             launch_mm_tile(ctx->stream, ue->data, ue->dtype, d->n_ff, E, D, m->moe_up[l]) ==
                 hipSuccess &&
             launch_moe_down_tile(ctx->stream, de->data, de->dtype, d->n_ff, D, E, m->moe_down[l]) ==
                 hipSuccess;
        if (ok && X[FTX_X_ROUTER_BIAS])
            ok = dalloc(&m->moe_rbias[l], (size_t)E) && vec_f32(X[FTX_X_ROUTER_BIAS], m->moe_rbias[l]);
    }
    if (ok && any_moe) {
        const int64_t rows = mm_pad_tokens(moe_rows_max(Mmax, E, U));
        const int cu = ctx->cu_count;
        // gate / up partials and the down partials share one buffer, sized
        // for every step size up to Mmax (the split counts depend on it)
        size_t pn = 0;
        for (int64_t mt = 1; mt <= Mmax; ++mt) {
            const int64_t t = moe_tiles_max(mt, E, U), r = t * moe_tile_rows(mt, E, U);
            const int S = moe_down_splits(d->n_ff, D, t, cu);
            // (the gate / up launch's splits depend on its tile count; 64
            // rows per tile bounds its operand rows)
            const size_t gu =
                mm_part_floats(t * 64, 2 * d->n_ff, D / 256, (2 * d->n_ff + 255) / 256, cu);
            pn = std::max({pn, gu, (size_t)mm_pad_tokens(r) * 2 * (size_t)d->n_ff,
                           (size_t)S * r * D});
        }
        m->moe_part_n = pn;
        ok = dalloc((uint8_t**)&m->route, moe_route_bytes(Mmax, E, U)) &&
             dalloc(&m->moe_act, mm_act_halves(rows, D)) &&
             dalloc(&m->moe_h, (size_t)(2 * rows * d->n_ff)) && dalloc(&m->moe_part, m->moe_part_n) &&
             (!F_sh || dalloc(&m->tmpo, (size_t)(Mmax * D)));
        // the router's finished-workgroup counter starts at zero
        ok = ok && hipMemset(m->route, 0, moe_route_bytes(Mmax, E, U)) == hipSuccess;
    }
    if (!ok) {
        model_release(m);
        return ftx_fail(ctx, FTX_E_NOMEM, "activation allocation failed");
    }
    // norm vectors as F32 (any stored dtype is dequantised once)
    for (int64_t l = 0; l <= d->n_layer; ++l) {
        for (int k = 0; k < 2; ++k) {
            if (l == d->n_layer && k == 1) break;
            const ftx_tensor* t =
                l == d->n_layer ? d->out_norm
                                : d->layers[l * FTX_LAYER_TENSORS + (k ? FTX_T_FFN_NORM : FTX_T_ATTN_NORM)];
            hipError_t e = launch_dequant(ctx->stream, t->data, t->dtype, t->row_bytes, D, 1,
                                          m->norms + (l * 2 + k) * D);
            if (e != hipSuccess) {
                model_release(m);
                return ftx_fail(ctx, FTX_E_DEVICE, "norm dequant failed");
            }
        }
    }
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
        model_release(m);
        return ftx_fail(ctx, FTX_E_DEVICE, "norm dequant failed");
    }
    *out = m;
    return FTX_OK;
}

int ftx_model_free(ftx_model* m) {
    if (m && m->ctx) (void)hipStreamSynchronize(m->ctx->stream);
    model_release(m);
    return FTX_OK;
}

int ftx_kv_create(ftx_ctx* ctx, const ftx_model* m, int64_t cap, int kv_dtype, ftx_kv** out) {
    if (!ctx || !m || !out) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (cap < 1) return ftx_fail(ctx, FTX_E_INVALID, "cap must be >= 1");
    if (kv_dtype != FTX_KV_F16 && kv_dtype != FTX_KV_F32)
        return ftx_fail(ctx, FTX_E_UNSUPPORTED, "kv dtype");
    ftx_kv* kv = new (std::nothrow) ftx_kv;
    if (!kv) return ftx_fail(ctx, FTX_E_NOMEM, "host allocation failed");
    kv->ctx = ctx;
    kv->n_layer = m->d.n_layer;
    kv->cap = cap;
    kv->cap_alloc = (cap + 127) / 128 * 128;  // whole attention chunks
    kv->kdim = m->kdim;
    kv->n_kv = m->d.n_head_kv;
    kv->hd = m->d.head_dim;
    kv->n_head = m->d.n_head;
    kv->mmax = m->Mmax;
    kv->kv_f16 = kv_dtype == FTX_KV_F16;
    const size_t bytes = (size_t)(kv->n_layer * kv->cap_alloc * kv->kdim) * (kv->kv_f16 ? 2 : 4);
    const size_t pf = attn_part_floats(m->Mmax, m->d.n_head, m->d.head_dim, kv->cap_alloc);
    if (hipMalloc(&kv->k, bytes) != hipSuccess || hipMalloc(&kv->v, bytes) != hipSuccess ||
        hipMalloc((void**)&kv->attn_part, pf * sizeof(float)) != hipSuccess) {
        (void)hipGetLastError();
        if (kv->k) (void)hipFree(kv->k);
        if (kv->v) (void)hipFree(kv->v);
        delete kv;
        return ftx_fail(ctx, FTX_E_NOMEM, "kv allocation failed");
    }
    // finite contents everywhere: masked slots still meet the P.V product
    (void)hipMemset(kv->k, 0, bytes);
    (void)hipMemset(kv->v, 0, bytes);
    *out = kv;
    return FTX_OK;
}

int ftx_kv_free(ftx_kv* kv) {
    if (!kv) return FTX_OK;
    if (kv->ctx) (void)hipStreamSynchronize(kv->ctx->stream);
    if (kv->k) (void)hipFree(kv->k);
    if (kv->v) (void)hipFree(kv->v);
    if (kv->attn_part) (void)hipFree(kv->attn_part);
    delete kv;
    return FTX_OK;
}

// host arrays in the canonical [n_layer][cap][n_kv*hd] layout
static int kv_copy(ftx_kv* kv, void* kh, void* vh, bool to_device) {
    ftx_ctx* ctx = kv->ctx;
    const int eb = kv->kv_f16 ? 2 : 4;
    const size_t row = (size_t)kv->kdim * eb;
    const size_t canon = (size_t)(kv->n_layer * kv->cap) * row;
    const size_t dev = (size_t)(kv->n_layer * kv->cap_alloc) * row;
    void* tmp;
    int rc = ftx_workspace(ctx, dev, &tmp);
    if (rc) return rc;
    hipStream_t st = ctx->stream;
    const hipMemcpyKind kind = to_device ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
    // K: the same layout with cap_alloc rows per layer
    if (to_device)
        FTX_HIP(ctx, hipMemcpy2DAsync(kv->k, (size_t)kv->cap_alloc * row, kh, (size_t)kv->cap * row,
                                      (size_t)kv->cap * row, (size_t)kv->n_layer, kind, st));
    else
        FTX_HIP(ctx, hipMemcpy2DAsync(kh, (size_t)kv->cap * row, kv->k, (size_t)kv->cap_alloc * row,
                                      (size_t)kv->cap * row, (size_t)kv->n_layer, kind, st));
    // V: canonical rows staged with cap_alloc rows per layer, then transposed
    if (to_device) {
        FTX_HIP(ctx, hipMemsetAsync(tmp, 0, dev, st));
        FTX_HIP(ctx, hipMemcpy2DAsync(tmp, (size_t)kv->cap_alloc * row, vh, (size_t)kv->cap * row,
                                      (size_t)kv->cap * row, (size_t)kv->n_layer, kind, st));
        FTX_HIP(ctx, launch_v_layout(st, tmp, kv->v, kv->n_layer, kv->cap_alloc, kv->n_kv, kv->hd,
                                     eb, 1));
    } else {
        FTX_HIP(ctx, launch_v_layout(st, kv->v, tmp, kv->n_layer, kv->cap_alloc, kv->n_kv, kv->hd,
                                     eb, 0));
        FTX_HIP(ctx, hipMemcpy2DAsync(vh, (size_t)kv->cap * row, tmp, (size_t)kv->cap_alloc * row,
                                      (size_t)kv->cap * row, (size_t)kv->n_layer, kind, st));
    }
    FTX_HIP(ctx, hipStreamSynchronize(st));
    (void)canon;
    return FTX_OK;
}

int ftx_kv_write(ftx_kv* kv, const void* k, const void* v) {
    if (!kv || !k || !v) return FTX_E_INVALID;
    return kv_copy(kv, (void*)k, (void*)v, true);
}

int ftx_kv_read(ftx_kv* kv, void* k, void* v) {
    if (!kv || !k || !v) return FTX_E_INVALID;
    return kv_copy(kv, k, v, false);
}

int ftx_kv_pointers(ftx_kv* kv, void** k, void** v, int64_t* npast) {
    if (!kv) return FTX_E_INVALID;
    if (k) *k = kv->k;
    if (v) *v = kv->v;
    if (npast) *npast = kv->npast;
    return FTX_OK;
}

int ftx_kv_truncate(ftx_kv* kv, int64_t npast) {
    if (!kv) return FTX_E_INVALID;
    if (npast < 0 || npast > kv->cap) return ftx_fail(kv->ctx, FTX_E_RANGE, "npast out of range");
    kv->npast = npast;
    return FTX_OK;
}

int ftx_kv_commit(ftx_kv* kv, const int32_t* nodes, int64_t n) {
    if (!kv || (n > 0 && !nodes)) return FTX_E_INVALID;
    ftx_ctx* ctx = kv->ctx;
    if (n < 0 || n > 256) return ftx_fail(ctx, FTX_E_INVALID, "kv_commit: path length out of range");
    if (kv->npast + n > kv->cap) return ftx_fail(ctx, FTX_E_RANGE, "kv_commit: capacity exceeded");
    KvCommitArgs a{};
    a.npast = kv->npast;
    a.cap = kv->cap_alloc;
    a.n_layer = kv->n_layer;
    a.n_kv = (int)kv->n_kv;
    a.hd = (int)kv->hd;
    a.n = (int)n;
    bool moves = false;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t j = nodes[i];
        if (j < i || (i > 0 && j <= nodes[i - 1]))
            return ftx_fail(ctx, FTX_E_INVALID,
                            "kv_commit: nodes must be strictly increasing with nodes[i] >= i");
        if (kv->npast + j >= kv->cap) return ftx_fail(ctx, FTX_E_RANGE, "kv_commit: node out of range");
        a.nodes[i] = j;
        moves |= j != i;
    }
    if (moves) FTX_HIP(ctx, launch_kv_commit(ctx->stream, a, kv->k, kv->v, kv->kv_f16));
    kv->npast += n;
    return FTX_OK;
}

int ftx_verify_batch(ftx_ctx* ctx, ftx_model* m, const ftx_seq_args* seqs, int64_t nseq) {
    if (!ctx || !m || !seqs) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (nseq < 1 || nseq > FTX_MAX_SEQ)
        return ftx_fail(ctx, FTX_E_INVALID, "nseq out of range (1 .. FTX_MAX_SEQ)");
    if (nseq == 1) {
        const ftx_verify_args a{seqs[0].M, seqs[0].tokens, seqs[0].parents, seqs[0].logits,
                                seqs[0].advance, 0};
        return ftx_verify_step(ctx, m, seqs[0].kv, &a);
    }
    int64_t Mt = 0;
    for (int64_t s = 0; s < nseq; ++s) {
        int rc = check_seq(ctx, m, seqs[s].kv, seqs[s].M, seqs[s].tokens);
        if (rc) return rc;
        if ((seqs[s].logits != nullptr) != (seqs[0].logits != nullptr))
            return ftx_fail(ctx, FTX_E_INVALID, "logits must be given for every sequence or none");
        for (int64_t r = 0; r < s; ++r)
            if (seqs[r].kv == seqs[s].kv)
                return ftx_fail(ctx, FTX_E_INVALID, "two sequences share a kv cache");
        Mt += seqs[s].M;
    }
    if (Mt > m->Mmax) return ftx_fail(ctx, FTX_E_INVALID, "tokens of all sequences above max_tokens");
    return verify_large(ctx, m, seqs, nseq);
}

int ftx_verify_step(ftx_ctx* ctx, ftx_model* m, ftx_kv* kv, const ftx_verify_args* a) {
    if (!ctx || !m || !kv || !a || !a->tokens)
        return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    const ftx_model_desc& d = m->d;
    const int64_t M = a->M;
    {
        int rc = check_seq(ctx, m, kv, M, a->tokens);
        if (rc) return rc;
    }
    if (M > 8 || m->has_ext) {
        const ftx_seq_args sa{kv, M, a->tokens, a->parents, a->logits, a->advance, 0};
        return verify_large(ctx, m, &sa, 1);
    }
    const int64_t npast = kv->npast;
    // host-side argument prep: tokens, depth, ancestor masks, npast
    const int aw = (int)((M + 31) / 32);
    const int64_t hd2 = d.head_dim / 2;
    const StepArgsLayout AL = step_args_layout(M, d.head_dim, aw);
    const int slot = m->pin_next;
    uint8_t* pin = m->pin[slot];
    FTX_HIP(ctx, hipEventSynchronize(m->pin_ev[slot]));  // this block's last copy is done
    int rc = FTX_OK;
    int32_t* toks = (int32_t*)pin;
    int32_t* depth = (int32_t*)(pin + AL.depth);
    uint32_t* anc = (uint32_t*)(pin + AL.anc);
    int64_t* np = (int64_t*)(pin + AL.np);
    float* cs = (float*)(pin + AL.cs);
    for (int64_t i = 0; i < M; ++i) {
        const int32_t t = a->tokens[i];
        if (t < 0 || t >= d.vocab) return ftx_fail(ctx, FTX_E_RANGE, "token id out of range");
        const int32_t p = a->parents ? a->parents[i] : (int32_t)i - 1;
        if (p < -1 || p >= i) return ftx_fail(ctx, FTX_E_INVALID, "parents[i] must be in [-1, i)");
        toks[i] = t;
        depth[i] = p < 0 ? 0 : depth[p] + 1;
        uint32_t* row = anc + i * aw;
        if (p >= 0)
            for (int w = 0; w < aw; ++w) row[w] = anc[p * aw + w];
        else
            for (int w = 0; w < aw; ++w) row[w] = 0;
        row[i / 32] |= 1u << (i % 32);
    }
    *np = npast;
    // rope_vec's angles (src/engine.cpp:43-60): f = theta^(-2i/hd) (the
    // model's table) and the angle in double, cos / sin rounded to float, at
    // position npast + depth (sincos: the values of cos and sin, in one call)
    for (int64_t i = 0; i < M; ++i)
        for (int64_t p = 0; p < hd2; ++p) {
            const double ang = (double)(npast + depth[i]) * m->rope_f[(size_t)p];
            double sn, cn;
            sincos(ang, &sn, &cn);
            cs[(i * hd2 + p) * 2] = (float)cn;
            cs[(i * hd2 + p) * 2 + 1] = (float)sn;
        }
    hipStream_t st = ctx->stream;
    m->toks = (int32_t*)m->args;
    m->depth = (int32_t*)(m->args + AL.depth);
    m->anc = (uint32_t*)(m->args + AL.anc);
    m->npast = (int64_t*)(m->args + AL.np);
    m->rcs = (float*)(m->args + AL.cs);
    FTX_HIP(ctx, hipMemcpyAsync(m->args, pin, AL.bytes, hipMemcpyHostToDevice, st));
    FTX_HIP(ctx, hipEventRecord(m->pin_ev[slot], st));
    m->pin_next = (slot + 1) % ftx_model::PIN_RING;

    const int64_t D = d.n_embd, F = d.n_ff, V = d.vocab;
    const float eps = d.rms_eps;
    const double f4 = 4.0, Md = (double)M;
    auto wbytes = [](const ftx_tensor* t) { return (double)(t->row_bytes * t->nrows); };
#define TRACED(kind, bytes, call)             \
    do {                                      \
        TraceScope ts_(ctx);                  \
        FTX_HIP(ctx, call);                   \
        ts_.end((kind), (double)(bytes));     \
    } while (0)
    // a launch whose outputs do not depend on its own earlier results
    // (no accumulate into its inputs): replayable by ftx_trace_replay
#define TRACED_IDEM(kind, bytes, call)                         \
    do {                                                       \
        TraceScope ts_(ctx);                                   \
        const int n_ = tr_repeats(ctx, (kind));                \
        for (int r_ = 0; r_ < n_; ++r_) FTX_HIP(ctx, call);     \
        ts_.end((kind), (double)(bytes) * n_, n_);             \
    } while (0)
    TRACED(TK_EMBED, Md * d.tok_embd->row_bytes + Md * D * f4,
           launch_embed(st, d.tok_embd->data, d.tok_embd->dtype, d.tok_embd->row_bytes, D,
                        m->toks, M, m->x));
    const size_t kvel = kv->kv_f16 ? 2 : 4;
    const double norm_b = 2 * Md * D * f4 + D * f4;
    // One projection: x (row stride ldx) [-> RMSNorm] -> weight segments.  The
    // int8-MFMA path runs when every segment qualifies (the norm is fused
    // into its activation prep); the generic kernels run otherwise.
    // split partials of the last ffn_down not yet added into x (folded by the
    // next projection's activation prep, or added here before a generic one)
    int fold_S = 0;
    auto project = [&](int kind, double bytes, float* xin, int64_t ldx, const float* normw,
                       const ftx_tensor* const* ts, GemvSeg* segs, int nseg, int64_t K, int epi,
                       int64_t tix0, const int* tix, const QkvEpi* qe = nullptr,
                       bool xq_ready = false) -> int {
        const bool fold = fold_S > 0 && xin == m->x;
        if (mv_all(ts, nseg, K, M) && (epi != EPI_SWIGLU || mv_swiglu_supported(K))) {
            // the tiled copies when every segment has one
            bool all = true;
            for (int i = 0; i < nseg; ++i) all = all && m->mvt[tix0 + tix[i]];
            for (int i = 0; all && i < nseg; ++i) {
                segs[i].W = m->mvt[tix0 + tix[i]];
                segs[i].tiled = 1;
                segs[i].rpt = m->mvt_rpt[tix0 + tix[i]];
            }
            // the 16x16x32 row-dot kernel over the tiled copies, else k_mv
            int rpts[3] = {0, 0, 0};
            for (int i = 0; all && i < nseg; ++i) rpts[i] = segs[i].rpt;
            const bool rd = all && rd_use(ts, rpts, nseg, K, M, epi, ctx->cu_count);
            if (!xq_ready && fold)  // adds the split partials into x: not replayable
                TRACED(TK_XQ_PREP, Md * K * f4 * (2.0 + fold_S) + 19.0 * K,
                       launch_xq_prep(st, xin, ldx, normw, m->downpart, fold_S, D, K, M, m->xq, rd));
            else if (!xq_ready)
                TRACED_IDEM(TK_XQ_PREP, Md * K * f4 + 19.0 * K,
                            launch_xq_prep(st, xin, ldx, normw, nullptr, 0, D, K, M, m->xq, rd));
            if (fold) fold_S = 0;
            auto gemv = [&]() -> hipError_t {
                return rd ? launch_rd(st, segs, nseg, m->xq, K, M, epi, normw != nullptr, eps, qe)
                          : launch_mv(st, segs, nseg, m->xq, K, M, epi, ctx->cu_count,
                                      normw != nullptr, eps, qe);
            };
            if (epi == EPI_ACCUM)
                TRACED(kind, bytes, gemv());
            else
                TRACED_IDEM(kind, bytes, gemv());
            return FTX_OK;
        }
        if (fold) {
            TRACED(TK_DOWN, Md * D * f4 * (2.0 + fold_S),
                   launch_part_reduce(st, m->downpart, fold_S, D, M, m->x, D));
            fold_S = 0;
        }
        // more than 8 tokens on tiled K-quant weights (not the fused qkv
        // epilogue): the row-dot MFMA kernel on 8-row chunks, each with its
        // own activation prep
        bool tiled_all = epi != EPI_QKV && M > 8 && mv_all(ts, nseg, K, 8) &&
                         (epi != EPI_SWIGLU || mv_swiglu_supported(K));
        for (int i = 0; tiled_all && i < nseg; ++i) tiled_all = m->mvt[tix0 + tix[i]] != nullptr;
        if (tiled_all) {
            auto chunks = [&]() -> hipError_t {
                // one prep for every chunk's operand, then a launch per chunk
                hipError_t e = launch_xq_prep(st, xin, ldx, normw, nullptr, 0, D, K, M, m->xq);
                if (e != hipSuccess) return e;
                for (int64_t c0 = 0; c0 < M; c0 += 8) {
                    const int64_t mc = M - c0 < 8 ? M - c0 : 8;
                    GemvSeg cs[3];
                    for (int i = 0; i < nseg; ++i) {
                        cs[i] = segs[i];
                        cs[i].W = m->mvt[tix0 + tix[i]];
                        cs[i].tiled = 1;
                        cs[i].rpt = m->mvt_rpt[tix0 + tix[i]];
                        if (cs[i].y) cs[i].y += c0 * cs[i].ldy;
                    }
                    e = launch_mv(st, cs, nseg, m->xq + (c0 / 8) * (int64_t)xq_chunk_bytes(K), K,
                                  mc, epi, ctx->cu_count, normw != nullptr, eps, nullptr);
                    if (e != hipSuccess) return e;
                }
                return hipSuccess;
            };
            TRACED(kind, bytes, chunks());
            return FTX_OK;
        }
        // the planar copies where every segment has one
        bool pl_all = true;
        for (int i = 0; i < nseg; ++i) pl_all = pl_all && m->pln[tix0 + tix[i]] != nullptr;
        for (int i = 0; pl_all && i < nseg; ++i) {
            segs[i].W = m->pln[tix0 + tix[i]];
            segs[i].dt = m->pln_dt[tix0 + tix[i]];
        }
        const float* src = xin;
        int64_t lds = ldx;
        if (normw) {
            TRACED(TK_RMSNORM, norm_b, launch_rmsnorm(st, xin, normw, K, M, eps, m->xn));
            src = m->xn;
            lds = K;
        }
        if (epi == EPI_SWIGLU)
            TRACED(kind, bytes,
                   launch_gemv_swiglu(st, segs[0].W, segs[1].W, segs[0].dt, segs[0].row_bytes,
                                      segs[0].N, src, lds, K, M, segs[0].y, segs[0].ldy, true));
        else
            TRACED(kind, bytes, launch_gemv(st, segs, nseg, src, lds, K, M, epi, true));
        return FTX_OK;
    };
    auto seg = [](const ftx_tensor* t, float* y, int64_t ldy) {
        return GemvSeg{t->data, t->dtype, t->row_bytes, t->nrows, y, ldy};
    };
    static const int ix_qkv[3] = {FTX_T_Q, FTX_T_K, FTX_T_V}, ix_o[1] = {FTX_T_O},
                     ix_gu[2] = {FTX_T_GATE, FTX_T_UP}, ix_head[1] = {0};
    for (int64_t l = 0; l < d.n_layer; ++l) {
        const int64_t lt = l * FTX_LAYER_TENSORS;
        const ftx_tensor* const* T = m->layers.data() + lt;
        const ftx_tensor* tqkv[3] = {T[FTX_T_Q], T[FTX_T_K], T[FTX_T_V]};
        GemvSeg qkv[3] = {seg(T[FTX_T_Q], m->qkv, m->ldq), seg(T[FTX_T_K], m->qkv + m->qdim, m->ldq),
                          seg(T[FTX_T_V], m->qkv + m->qdim + m->kdim, m->ldq)};
        uint8_t* kl = (uint8_t*)kv->k + (size_t)(l * kv->cap_alloc * kv->kdim) * kvel;
        uint8_t* vl = (uint8_t*)kv->v + (size_t)(l * kv->cap_alloc * kv->kdim) * kvel;
        const bool mattn = attn_mfma_supported(d.head_dim, kv->kv_f16, M, d.n_head, d.n_head_kv);
        // RoPE and the KV write ride on the projection's epilogue when the
        // MFMA kernels take both (interleaved pairs are adjacent outputs)
        const bool fuse = mattn && !d.rope_neox && mv_all(tqkv, 3, D, M);
        QkvEpi qe{};
        qe.cs = m->rcs;
        qe.qh = m->qhl;
        qe.ql = m->qhl + M * m->qdim;
        qe.kc = kl;
        qe.vc = vl;
        qe.slot0 = npast;
        qe.cap = kv->cap_alloc;
        qe.hd = (int)d.head_dim;
        qe.n_head = (int)d.n_head;
        qe.n_kv = (int)d.n_head_kv;
        qe.kv_f16 = kv->kv_f16;
        rc = project(TK_GEMV_QKV,
                     wbytes(T[FTX_T_Q]) + wbytes(T[FTX_T_K]) + wbytes(T[FTX_T_V]) + Md * D * f4 +
                         Md * m->ldq * f4,
                     m->x, D, m->norms + (l * 2) * D, tqkv, qkv, 3, D,
                     fuse ? EPI_QKV : EPI_STORE, lt, ix_qkv, fuse ? &qe : nullptr);
        if (rc) return rc;
        RopeArgs ra{m->qkv,       m->ldq,       d.n_head, d.n_head_kv, d.head_dim,   m->depth,
                    m->npast,     d.rope_theta, d.rope_neox, kl,       vl,           kv->kv_f16,
                    kv->cap_alloc};
        if (mattn) {
            ra.qh16 = qe.qh;
            ra.ql16 = qe.ql;
        }
        if (!fuse)
            TRACED(TK_ROPE_KV, 2 * Md * m->ldq * f4 + 2 * Md * m->kdim * (double)kvel,
                   launch_rope_kv(st, ra, M));
        const double attn_b =
            2.0 * (double)(npast + M) * m->kdim * (double)kvel + 2 * Md * m->qdim * f4;
        // the chunk combine writes the output projection's activation operand
        // directly when that projection takes the int8-MFMA path
        const bool o_xq = mattn && attn_combine_xq_supported(d.head_dim, d.n_head) &&
                          mv_all(&T[FTX_T_O], 1, m->qdim, M);
        // the o projection runs launch_rd (its operand in the layout16 form)
        // when its tiled copy exists and the kernel takes the shape
        const int o_rpt = m->mvt_rpt[lt + FTX_T_O];
        const bool o_rd = m->mvt[lt + FTX_T_O] &&
                          rd_use(&T[FTX_T_O], &o_rpt, 1, m->qdim, M, EPI_ACCUM, ctx->cu_count);
        if (mattn) {
            AttnMArgs am{};
            am.qkv = m->qkv;
            am.ldq = m->ldq;
            am.qh16 = ra.qh16;
            am.ql16 = ra.ql16;
            am.kc = (const _Float16*)kl;
            am.vt = (const _Float16*)vl;
            am.cap = kv->cap_alloc;
            am.npast = npast;
            am.anc = m->anc;
            am.anc_words = aw;
            am.M = (int)M;
            am.n_head = (int)d.n_head;
            am.n_kv = (int)d.n_head_kv;
            am.hd = (int)d.head_dim;
            am.out = m->att;
            TRACED_IDEM(TK_ATTENTION, attn_b,
                        launch_attn_mfma(st, am, kv->attn_part, o_xq ? m->xq : nullptr, o_rd));
        } else {
            AttnArgs aa{m->qkv,  m->ldq, kl,       vl,          kv->kv_f16, m->npast,
                        m->anc,  aw,     d.n_head, d.n_head_kv, d.head_dim, npast + M,
                        m->att,  kv->cap_alloc};
            TRACED(TK_ATTENTION, attn_b, launch_attention(st, aa, M));
        }
        GemvSeg o = seg(T[FTX_T_O], m->x, D);
        rc = project(TK_GEMV_O, wbytes(T[FTX_T_O]) + Md * m->qdim * f4 + 2 * Md * D * f4, m->att,
                     m->qdim, nullptr, &T[FTX_T_O], &o, 1, m->qdim, EPI_ACCUM, lt, ix_o, nullptr,
                     o_xq);
        if (rc) return rc;
        const ftx_tensor* tgu[2] = {T[FTX_T_GATE], T[FTX_T_UP]};
        GemvSeg gu[2] = {seg(T[FTX_T_GATE], m->h, F), seg(T[FTX_T_UP], nullptr, 0)};
        rc = project(TK_GEMV_SWIGLU,
                     wbytes(T[FTX_T_GATE]) + wbytes(T[FTX_T_UP]) + Md * D * f4 + Md * F * f4, m->x,
                     D, m->norms + (l * 2 + 1) * D, tgu, gu, 2, D, EPI_SWIGLU, lt, ix_gu);
        if (rc) return rc;
        const double down_b = wbytes(T[FTX_T_DOWN]) + Md * F * f4 + 2 * Md * D * f4;
        if (m->down_tiled[l] && down_mfma_supported(T[FTX_T_DOWN]->dtype, F, D, M)) {
            TRACED_IDEM(TK_DOWN, down_b,
                        launch_down_mfma(st, T[FTX_T_DOWN]->dtype, m->down_tiled[l], F, D, m->h,
                                         F, M, m->x, D, m->downpart, ctx->cu_count, &fold_S));
        } else if (m->down_tiled[l] && down_mfma_supported(T[FTX_T_DOWN]->dtype, F, D, 8)) {
            // more than 8 tokens: the MFMA down kernel on 8-row chunks, every
            // chunk's split partials added into x by one reduce
            auto chunks = [&]() -> hipError_t {
                int S = 0;
                for (int64_t c0 = 0; c0 < M; c0 += 8) {
                    const int64_t mc = M - c0 < 8 ? M - c0 : 8;
                    // chunk c's partials at downpart + c * S * 8 * D (S is the
                    // same for every chunk: it depends on the shape only)
                    float* pc = m->downpart + (S ? (c0 / 8) * (int64_t)S * 8 * D : 0);
                    hipError_t e = launch_down_mfma(st, T[FTX_T_DOWN]->dtype, m->down_tiled[l], F,
                                                    D, m->h + c0 * F, F, mc, m->x + c0 * D, D, pc,
                                                    ctx->cu_count, &S);
                    if (e != hipSuccess) return e;
                }
                return launch_part_reduce(st, m->downpart, S, D, M, m->x, D);
            };
            TRACED(TK_DOWN, down_b, chunks());
        } else {
            TRACED(TK_DOWN, down_b,
                   launch_down(st, T[FTX_T_DOWN]->data, T[FTX_T_DOWN]->dtype,
                               T[FTX_T_DOWN]->row_bytes, F, D, m->h, F, M, m->x, D, m->part));
        }
    }
    // the LM head (skipped without a logits buffer: every layer's K / V rows
    // are written by now, which is all a prefill chunk needs)
    if (a->logits) {
        const ftx_tensor* lm = d.output ? d.output : d.tok_embd;
        GemvSeg hs = seg(lm, a->logits, V);
        rc = project(TK_HEAD, wbytes(lm) + Md * D * f4 + Md * V * f4, m->x, D,
                     m->norms + (d.n_layer * 2) * D, &lm, &hs, 1, D, EPI_STORE,
                     d.n_layer * FTX_LAYER_TENSORS, ix_head);
        if (rc) return rc;
    }
#undef TRACED
    if (a->advance) kv->npast = npast + M;
    return FTX_OK;
}

int ftx_argmax_prob(ftx_ctx* ctx, const float* row, int64_t V, int32_t* token, float* prob) {
    if (!ctx || !row || !token || V < 1) return ftx_fail(ctx, FTX_E_INVALID, "null argument or V < 1");
    const size_t rs = (row_stats_scratch_bytes(1, V) + 255) & ~(size_t)255;
    uint8_t* ws;
    int rc = ftx_workspace(ctx, rs + 256, (void**)&ws);
    if (rc) return rc;
    int32_t* pin;
    rc = ftx_pinned(ctx, 8, (void**)&pin);
    if (rc) return rc;
    hipStream_t st = ctx->stream;
    int32_t* d_out = (int32_t*)(ws + rs);
    FTX_HIP(ctx, launch_argmax_prob(st, row, V, ws, d_out));
    FTX_HIP(ctx, hipMemcpyAsync(pin, d_out, 8, hipMemcpyDeviceToHost, st));
    FTX_HIP(ctx, hipStreamSynchronize(st));
    *token = pin[0];
    if (prob) std::memcpy(prob, &pin[1], 4);
    return FTX_OK;
}

}  // extern "C"

namespace {

// Checks of one acceptance's arguments (ftx_accept's contract).
int acc_validate(ftx_ctx* ctx, const ftx_accept_args* a) {
    if (!a || !a->base_row || !a->props || !a->rng || !a->accepted || !a->n_acc || !a->bonus)
        return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    const int64_t M = a->M, V = a->V;
    if (M < 0 || V < 1 || (M > 0 && !a->rows)) return ftx_fail(ctx, FTX_E_INVALID, "bad M or V");
    if (a->mode != FTX_ACCEPT_GREEDY && a->mode != FTX_ACCEPT_RATIO &&
        a->mode != FTX_ACCEPT_RESIDUAL)
        return ftx_fail(ctx, FTX_E_UNSUPPORTED, "unknown acceptance mode");
    if (a->mode == FTX_ACCEPT_RATIO && (!a->pd && M > 0))
        return ftx_fail(ctx, FTX_E_INVALID, "ratio mode needs pd");
    if (a->mode == FTX_ACCEPT_RESIDUAL && (!a->q && M > 0))
        return ftx_fail(ctx, FTX_E_INVALID, "residual mode needs q");
    if (!(a->temp > 0.f)) return ftx_fail(ctx, FTX_E_INVALID, "temperature must be > 0");
    if (a->mode == FTX_ACCEPT_RATIO) {
        // the device sampler: top-k of at most 64, or no top-k over at most
        // 64 tokens; rows of at most 4096 sub-chunks of 128
        if (!a->sampler_rng) return ftx_fail(ctx, FTX_E_INVALID, "ratio mode needs sampler_rng");
        const bool use_k = a->top_k > 0 && a->top_k < V;
        if ((use_k && a->top_k > 64) || (!use_k && V > 64) || (V + 127) / 128 > 4096)
            return ftx_fail(ctx, FTX_E_UNSUPPORTED,
                            "sampler: top_k must be in 1..64 (or V <= 64), V <= 524288");
    }
    for (int64_t i = 0; i < M; ++i) {
        const int32_t p = a->parents ? a->parents[i] : (int32_t)i - 1;
        if (p < -1 || p >= i) return ftx_fail(ctx, FTX_E_INVALID, "parents[i] must be in [-1, i)");
        if (a->props[i] < 0 || a->props[i] >= V)
            return ftx_fail(ctx, FTX_E_RANGE, "draft token out of range");
        if (a->mode == FTX_ACCEPT_RATIO && p != i - 1)
            return ftx_fail(ctx, FTX_E_INVALID, "ratio mode is chain only");
    }
    return FTX_OK;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace of one acceptance: stats [M+1], p [V] doubles (residual mode:
// two residual buffers and the kernel's barrier and partial sums), the small
// block (rng, margin, out ints | props, parents, pd: copied in, its head
// copied out), the chunk statistics of the M + 1 rows.
struct AccPlan {
    size_t off_p, off_small, head_b, small_b, off_rs, bytes;
};

AccPlan acc_plan(const ftx_accept_args* a) {
    const int64_t M = a->M, V = a->V;
    AccPlan P;
    P.off_p = align256((size_t)(M + 1) * sizeof(RowStats));
    const size_t pb = a->mode == FTX_ACCEPT_RESIDUAL
                          ? 2 * (size_t)V * 8 + 256 + accept_residual_scratch_bytes()
                          : 0;
    P.off_small = P.off_p + align256(pb);
    const size_t out_b = ((size_t)(M + 2) * 4 + 7) & ~(size_t)7;
    P.head_b = 24 + out_b;  // rng | sampler rng | margin | pad | out
    P.small_b = P.head_b + (size_t)M * 12 + 64;
    P.off_rs = P.off_small + align256(P.small_b);
    P.bytes = P.off_rs + align256(row_stats_scratch_bytes(M + 1, V)) + 256;
    return P;
}

// the small block of a in host memory: rng | sampler rng | margin | pad |
// out | props | parents | pd
void acc_fill_small(const ftx_accept_args* a, const AccPlan& P, uint8_t* pin) {
    const int64_t M = a->M;
    *(uint64_t*)pin = *a->rng;
    *(uint64_t*)(pin + 8) = a->sampler_rng ? *a->sampler_rng : 0;
    *(float*)(pin + 16) = INFINITY;
    int32_t* h_props = (int32_t*)(pin + P.head_b);
    int32_t* h_par = h_props + M;
    float* h_pd = (float*)(h_par + M);
    for (int64_t i = 0; i < M; ++i) {
        h_props[i] = a->props[i];
        h_par[i] = a->parents ? a->parents[i] : (int32_t)i - 1;
        h_pd[i] = a->pd ? a->pd[i] : 0.f;
    }
}

// the kernels' view of a: ws = its workspace, d_small = its small block on
// the device
AcceptDev acc_dev(const ftx_accept_args* a, const AccPlan& P, uint8_t* ws, uint8_t* d_small) {
    const int64_t M = a->M, V = a->V;
    AcceptDev ad{};
    ad.base_row = a->base_row;
    ad.rows = a->rows;
    ad.q = a->q;
    ad.rc = row_chunks(ws + P.off_rs, M + 1, V);
    ad.with_sum = a->mode != FTX_ACCEPT_GREEDY;
    ad.stats = (RowStats*)ws;
    ad.M = M;
    ad.V = V;
    ad.props = (const int32_t*)(d_small + P.head_b);
    ad.parents = ad.props + M;
    ad.pd = (const float*)(ad.parents + M);
    ad.mode = a->mode;
    ad.temp = a->temp;
    ad.rng = (uint64_t*)d_small;
    ad.sampler_rng = (uint64_t*)(d_small + 8);
    ad.top_k = a->top_k;
    ad.top_p = a->top_p;
    ad.p = (double*)(ws + P.off_p);
    ad.out = (int32_t*)(d_small + 24);
    ad.margin = (float*)(d_small + 16);
    return ad;
}

void* acc_res_scratch(const ftx_accept_args* a, const AccPlan& P, uint8_t* ws) {
    return ws + P.off_p + align256(2 * (size_t)a->V * 8);
}

int acc_row_stats(ftx_ctx* ctx, const ftx_accept_args* a, const AcceptDev& ad) {
    TraceScope ts(ctx);
    FTX_HIP(ctx, launch_row_stats(ctx->stream, a->base_row, a->rows, a->M + 1, a->V, a->temp,
                                  ad.with_sum, ad.rc));
    ts.end(TK_ROW_STATS, (double)(a->M + 1) * a->V * 4, ad.with_sum ? 2 : 1);
    return FTX_OK;
}

// the outputs of a from its small block's head, copied back to host memory
int acc_results(ftx_ctx* ctx, const ftx_accept_args* a, const uint8_t* pin) {
    const int32_t* h_out = (const int32_t*)(pin + 24);
    const int32_t na = h_out[0];
    if (na < 0 || na > a->M) return ftx_fail(ctx, FTX_E_DEVICE, "acceptance returned a bad count");
    *a->n_acc = na;
    *a->bonus = h_out[1];
    for (int32_t i = 0; i < na; ++i) a->accepted[i] = h_out[2 + i];
    *a->rng = *(const uint64_t*)pin;
    if (a->sampler_rng) *a->sampler_rng = *(const uint64_t*)(pin + 8);
    if (a->margin) *a->margin = *(const float*)(pin + 16);
    return FTX_OK;
}

}  // namespace

extern "C" {

int ftx_accept(ftx_ctx* ctx, const ftx_accept_args* a) {
    if (!ctx) return FTX_E_INVALID;
    int rc = acc_validate(ctx, a);
    if (rc) return rc;
    const AccPlan P = acc_plan(a);
    uint8_t* ws;
    rc = ftx_workspace(ctx, P.bytes, (void**)&ws);
    if (rc) return rc;
    uint8_t* pin;
    rc = ftx_pinned(ctx, P.small_b, (void**)&pin);
    if (rc) return rc;
    // (every user of the context's pinned block has waited for its copies
    // before returning, also on its error paths, so the block is filled
    // while the stream may still run earlier work: the acceptance's copies
    // and launches queue behind it without a host round trip)
    hipStream_t st = ctx->stream;
    acc_fill_small(a, P, pin);
    uint8_t* d_small = ws + P.off_small;
    FTX_HIP(ctx, hipMemcpyAsync(d_small, pin, P.small_b, hipMemcpyHostToDevice, st));
    const AcceptDev ad = acc_dev(a, P, ws, d_small);
    rc = acc_row_stats(ctx, a, ad);
    if (rc) return rc;
    int bar_err = 0;
    void* res_scratch = acc_res_scratch(a, P, ws);
    {
        TraceScope ts(ctx);
        if (a->mode == FTX_ACCEPT_RESIDUAL)
            FTX_HIP(ctx, launch_accept_residual(st, ad, res_scratch));
        else
            FTX_HIP(ctx, launch_accept(st, ad));
        ts.end(TK_ACCEPT, (double)a->V * 4);
    }
    FTX_HIP(ctx, hipMemcpyAsync(pin, d_small, P.head_b, hipMemcpyDeviceToHost, st));
    if (a->mode == FTX_ACCEPT_RESIDUAL && accept_residual_error(res_scratch, st, &bar_err)) {
        (void)hipStreamSynchronize(st);  // the copy into the pinned block has landed
        return ftx_fail(ctx, FTX_E_DEVICE, "acceptance: copy of the barrier state failed");
    }
    FTX_HIP(ctx, hipStreamSynchronize(st));
    if (bar_err)
        return ftx_fail(ctx, FTX_E_DEVICE, "acceptance: a grid barrier timed out");
    return acc_results(ctx, a, pin);
}

int ftx_accept_batch(ftx_ctx* ctx, const ftx_accept_args* args, int n) {
    if (!ctx) return FTX_E_INVALID;
    if (!args || n < 1 || n > FTX_MAX_SEQ)
        return ftx_fail(ctx, FTX_E_INVALID, "accept_batch: 1..FTX_MAX_SEQ acceptances");
    AccPlan P[FTX_MAX_SEQ];
    size_t ws_off[FTX_MAX_SEQ], pin_off[FTX_MAX_SEQ];
    size_t ws_total = 0, pin_total = 0;
    int nmulti = 0;
    for (int i = 0; i < n; ++i) {
        const int rc = acc_validate(ctx, &args[i]);
        if (rc) return rc;
        P[i] = acc_plan(&args[i]);
        ws_off[i] = ws_total;
        ws_total += align256(P[i].bytes);
        pin_off[i] = pin_total;
        pin_total += align256(P[i].small_b);
        nmulti += args[i].mode != FTX_ACCEPT_RESIDUAL;
    }
    // the small blocks, then the one-launch acceptances' descriptions, in
    // one pinned block copied to one device region (one copy each way)
    const size_t adv_off = pin_total;
    pin_total += align256((size_t)nmulti * sizeof(AcceptDev));
    uint8_t* ws;
    int rc = ftx_workspace(ctx, ws_total + pin_total, (void**)&ws);
    if (rc) return rc;
    uint8_t* pin;
    rc = ftx_pinned(ctx, pin_total, (void**)&pin);
    if (rc) return rc;
    uint8_t* d_small = ws + ws_total;
    hipStream_t st = ctx->stream;  // (filled without waiting: see ftx_accept)
    AcceptDev ad[FTX_MAX_SEQ];
    AcceptDev* h_adv = (AcceptDev*)(pin + adv_off);
    int k = 0;
    for (int i = 0; i < n; ++i) {
        acc_fill_small(&args[i], P[i], pin + pin_off[i]);
        ad[i] = acc_dev(&args[i], P[i], ws + ws_off[i], d_small + pin_off[i]);
        if (args[i].mode != FTX_ACCEPT_RESIDUAL) h_adv[k++] = ad[i];
    }
    FTX_HIP(ctx, hipMemcpyAsync(d_small, pin, pin_total, hipMemcpyHostToDevice, st));
    for (int i = 0; i < n; ++i) {
        rc = acc_row_stats(ctx, &args[i], ad[i]);
        if (rc) return rc;
    }
    int bar_err[FTX_MAX_SEQ] = {};
    for (int i = 0; i < n; ++i) {
        if (args[i].mode != FTX_ACCEPT_RESIDUAL) continue;
        TraceScope ts(ctx);
        FTX_HIP(ctx, launch_accept_residual(st, ad[i], acc_res_scratch(&args[i], P[i], ws + ws_off[i])));
        ts.end(TK_ACCEPT, (double)args[i].V * 4);
    }
    if (nmulti) {
        TraceScope ts(ctx);
        FTX_HIP(ctx, launch_accept_multi(st, (const AcceptDev*)(d_small + adv_off), nmulti));
        ts.end(TK_ACCEPT, (double)args[0].V * 4 * nmulti);
    }
    FTX_HIP(ctx, hipMemcpyAsync(pin, d_small, adv_off, hipMemcpyDeviceToHost, st));
    for (int i = 0; i < n; ++i)
        if (args[i].mode == FTX_ACCEPT_RESIDUAL &&
            accept_residual_error(acc_res_scratch(&args[i], P[i], ws + ws_off[i]), st, &bar_err[i])) {
            (void)hipStreamSynchronize(st);  // the copy into the pinned block has landed
            return ftx_fail(ctx, FTX_E_DEVICE, "acceptance: copy of the barrier state failed");
        }
    FTX_HIP(ctx, hipStreamSynchronize(st));
    for (int i = 0; i < n; ++i) {
        if (bar_err[i]) return ftx_fail(ctx, FTX_E_DEVICE, "acceptance: a grid barrier timed out");
        rc = acc_results(ctx, &args[i], pin + pin_off[i]);
        if (rc) return rc;
    }
    return FTX_OK;
}

}  // extern "C"
