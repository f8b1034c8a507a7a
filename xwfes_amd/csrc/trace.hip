// trace.hip -- per-kernel-class device time from HIP events recorded around
// each launch on the context's stream (ftx_trace / ftx_trace_read).
#include <cstdio>
#include <cstring>

#include "ftx_internal.h"

thread_local KernelTimer* g_ktimer = nullptr;

static const char* kTraceNames[TK_COUNT] = {
    "embed", "rmsnorm", "gemv_qkv", "rope_kv", "attention", "gemv_o",
    "gemv_swiglu", "down", "head", "row_stats", "accept", "xq_prep", "moe_route",
    "moe_combine", "event_pair"};

static void resolve(ftx_ctx* ctx) {
    if (ctx->pending.empty()) {
        ctx->next_event = 0;
        return;
    }
    (void)hipStreamSynchronize(ctx->stream);
    for (const TraceRec& r : ctx->pending) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, ctx->events[r.ev0], ctx->events[r.ev1]) != hipSuccess) {
            (void)hipGetLastError();
            continue;
        }
        if (r.kernel) {
            ctx->tr_klaunches[r.kind] += 1;
            ctx->tr_kms[r.kind] += ms;
            continue;
        }
        ctx->tr_launches[r.kind] += r.launches;
        ctx->tr_ms[r.kind] += ms;
        ctx->tr_bytes[r.kind] += r.bytes;
    }
    ctx->pending.clear();
    ctx->next_event = 0;
}

static int take_event(ftx_ctx* ctx) {
    if (ctx->next_event >= (int)ctx->events.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) {
            (void)hipGetLastError();
            return -1;
        }
        ctx->events.push_back(e);
    }
    return ctx->next_event++;
}

int tr_begin(ftx_ctx* ctx) {
    if (!ctx->trace) return -1;
    if (ctx->next_event > 4096) resolve(ctx);
    const int e = take_event(ctx);
    if (e < 0) return -1;
    if (hipEventRecord(ctx->events[e], ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    // arm the kernel timer for the first kernel of this call
    const int k0 = take_event(ctx), k1 = take_event(ctx);
    if (k0 >= 0 && k1 >= 0) {
        ctx->kt.e0 = ctx->events[k0];
        ctx->kt.e1 = ctx->events[k1];
        ctx->kt.armed = true;
        ctx->kt.fired = false;
        ctx->kt_ev0 = k0;
        ctx->kt_ev1 = k1;
        g_ktimer = &ctx->kt;
    }
    return e;
}

void tr_end(ftx_ctx* ctx, int token, int kind, double bytes, int launches) {
    if (token < 0 || !ctx->trace) return;
    if (ctx->kt.armed) {
        if (ctx->kt.fired)
            ctx->pending.push_back(TraceRec{kind, ctx->kt_ev0, ctx->kt_ev1, 0.0, 1, true});
        ctx->kt.armed = false;
        g_ktimer = nullptr;
    }
    const int e = take_event(ctx);
    if (e < 0) return;
    if (hipEventRecord(ctx->events[e], ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    ctx->pending.push_back(TraceRec{kind, token, e, bytes, launches});
}

void tr_abort(ftx_ctx* ctx) {
    if (!ctx) return;
    ctx->kt.armed = false;
    if (g_ktimer == &ctx->kt) g_ktimer = nullptr;
}

int tr_repeats(const ftx_ctx* ctx, int kind) {
    return ctx->trace && kind == ctx->replay_kind ? ctx->replay_n : 1;
}

extern "C" {

int ftx_trace(ftx_ctx* ctx, int enable) {
    if (!ctx) return FTX_E_INVALID;
    tr_abort(ctx);
    resolve(ctx);
    ctx->trace = enable != 0;
    if (enable) {
        for (int k = 0; k < TK_COUNT; ++k) {
            ctx->tr_launches[k] = 0;
            ctx->tr_ms[k] = 0;
            ctx->tr_bytes[k] = 0;
            ctx->tr_klaunches[k] = 0;
            ctx->tr_kms[k] = 0;
        }
        // the brackets' own time: 32 event pairs with nothing between them
        for (int i = 0; i < 32; ++i) tr_end(ctx, tr_begin(ctx), TK_EVENT_PAIR, 0.0, 1);
    }
    return FTX_OK;
}

int ftx_trace_replay(ftx_ctx* ctx, const char* kind, int times) {
    if (!ctx) return FTX_E_INVALID;
    if (!kind || times < 1) return ftx_fail(ctx, FTX_E_INVALID, "trace_replay: bad arguments");
    for (int k = 0; k < TK_COUNT; ++k)
        if (!strcmp(kind, kTraceNames[k])) {
            ctx->replay_kind = times > 1 ? k : -1;
            ctx->replay_n = times;
            return FTX_OK;
        }
    return ftx_fail(ctx, FTX_E_INVALID, "trace_replay: unknown kernel class");
}

int ftx_trace_read(ftx_ctx* ctx, ftx_trace_entry* out, int max, int* n) {
    if (!ctx || !n || (max > 0 && !out)) return FTX_E_INVALID;
    resolve(ctx);
    int c = 0;
    for (int k = 0; k < TK_COUNT; ++k) {
        if (!ctx->tr_launches[k]) continue;
        if (c < max) {
            memset(&out[c], 0, sizeof(out[c]));
            snprintf(out[c].name, sizeof(out[c].name), "%s", kTraceNames[k]);
            out[c].launches = ctx->tr_launches[k];
            out[c].ms = ctx->tr_ms[k];
            out[c].bytes = ctx->tr_bytes[k];
            out[c].kernel_launches = ctx->tr_klaunches[k];
            out[c].kernel_ms = ctx->tr_kms[k];
        }
        ++c;
    }
    *n = c < max ? c : max;
    return FTX_OK;
}

}  // extern "C"
