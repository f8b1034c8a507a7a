/*
 * ftx.h -- C ABI of the MI355X speculative-decoding verify path.
 *
 * One shared library (libftx.so, HIP for gfx950) behind plain C entry
 * points: opaque handles, plain pointers and sizes, int status codes, no
 * exceptions and no C++ types across the boundary.  Every function returns
 * FTX_OK (0) or a negative FTX_E_* code; ftx_last_error() returns the message
 * of the last failure on that context.
 *
 * Reference interface each entry point replaces (paths relative to
 * ft-igpu-src/ of Dark-hub-cat/xwfes):
 *   ftx_create / ftx_destroy / ftx_device_info
 *       IBackend construction and name()/info()/ready()
 *       (include/ft/backend.h:21-27; src/engine.cpp:291-300)
 *   ftx_tensor_upload
 *       the HostTensor that IBackend::matmul receives
 *       (include/ft/types.h:119-140), made resident on the device; callers
 *       key the handle by HostTensor::data
 *   ftx_dequant            dequant_row (include/ft/quant.h:10-84), whole tensor
 *   ftx_matmul             IBackend::matmul (include/ft/backend.h:29-30) as
 *                          CpuBackend::matmul (src/cpu_backend.cpp:90-104)
 *                          means it: y[m*N + n] per row (the reference sums
 *                          the M rows into y[n], cpu_backend.cpp:98-101)
 *   ftx_down_axpy          matmul_down_axpy (src/cpu_backend.cpp:60-75)
 *   ftx_expert_chunk       IBackend::run_expert_chunk (include/ft/backend.h:32;
 *                          ExpertChunkJob backend.h:7-19;
 *                          src/cpu_backend.cpp:106-149)
 *   ftx_alloc_staging / ftx_free_staging / ftx_stage / ftx_sync
 *                          IBackend staging and sync (include/ft/backend.h:34-39)
 *   ftx_model_create, ftx_kv_create, ftx_verify_step
 *                          Engine::extend_verify -> Engine::forward(M)
 *                          (src/engine.cpp:669-674, 461-596) over the KV cache
 *                          of include/ft/kv_cache.h:10-47, run on the device,
 *                          with optional draft-tree parents (the reference is
 *                          causal only, src/engine.cpp:152)
 *   ftx_kv_truncate        Engine::truncate_to / KvCache::set_npast
 *                          (src/engine.cpp:423-428; include/ft/kv_cache.h:31)
 *   ftx_kv_commit          the same for an accepted draft-tree path (rows of
 *                          the path's nodes gathered to the committed slots)
 *   ftx_accept             accept_chain_greedy / accept_chain_sampling
 *                          (src/spec.cpp:203-238) plus the bonus token of
 *                          generate() (src/spec.cpp:302-311), and tree and
 *                          residual-resampling modes (no reference
 *                          counterpart)
 */
#ifndef FTX_H
#define FTX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
enum {
    FTX_OK = 0,
    FTX_E_INVALID = -1,     /* bad argument, shape or dtype */
    FTX_E_UNSUPPORTED = -2, /* dtype or mode not implemented */
    FTX_E_DEVICE = -3,      /* HIP runtime error */
    FTX_E_NOMEM = -4,       /* device allocation failed */
    FTX_E_RANGE = -5        /* token id, position or capacity out of range */
};

/* ---- dtypes: the reference DType values (include/ft/types.h:20-27) plus
 * the ggml ids of the K-quants ---- */
enum {
    FTX_F32 = 0,
    FTX_F16 = 1,
    FTX_Q4_0 = 2,  /* 18 B / 32; element j = nibble (j&1) of byte j/2 (reference order) */
    FTX_Q4_1 = 3,  /* 20 B / 32; first fp16 added, second multiplies the nibble */
    FTX_Q8_0 = 8,  /* 34 B / 32 */
    FTX_Q4_K = 12, /* 144 B / 256: fp16 d, fp16 dmin, 12 B 6-bit (sc, m), 128 B qs */
    FTX_Q6_K = 14, /* 210 B / 256: 128 B ql, 64 B qh, 16 int8 sc, fp16 d */
    FTX_BF16 = 30
};

/* KV element types */
enum { FTX_KV_F32 = 0, FTX_KV_F16 = 1 };

/* acceptance modes */
enum {
    FTX_ACCEPT_GREEDY = 0,   /* argmax match, chain or tree */
    FTX_ACCEPT_RATIO = 1,    /* reference ratio test, scalar draft prob, chain only */
    FTX_ACCEPT_RESIDUAL = 2  /* multi-candidate speculative sampling, full draft dists */
};

typedef struct ftx_ctx ftx_ctx;
typedef struct ftx_tensor ftx_tensor;
typedef struct ftx_model ftx_model;
typedef struct ftx_kv ftx_kv;

typedef struct {
    char name[64];
    int64_t mem_bytes;  /* total device memory */
    int32_t compute_units;
    int32_t arch_major, arch_minor;
    int32_t pad_;
} ftx_device_info_t;

/* ---- context ---- */
/* A context on `device` with its own stream (IBackend construction,
 * src/engine.cpp:291-300).  Makes `device` the calling thread's current
 * device, as creating its stream requires. */
int ftx_create(int device, ftx_ctx** out);
int ftx_destroy(ftx_ctx* ctx);
int ftx_device_info(ftx_ctx* ctx, ftx_device_info_t* out);
const char* ftx_last_error(ftx_ctx* ctx);
/* Enqueue all following work on `stream` (a hipStream_t; NULL = the
 * context's own stream). */
int ftx_set_stream(ftx_ctx* ctx, void* stream);
int ftx_sync(ftx_ctx* ctx);

/* ---- tensors: rows of ne[0] elements, ne[1] rows, ne[2] planes ---- */
int64_t ftx_row_bytes(int dtype, int64_t ncols);
/* Copy `host` (row_stride bytes per row; 0 = dense) into a new resident
 * device tensor with dense rows. */
int ftx_tensor_upload(ftx_ctx* ctx, int dtype, const int64_t ne[4], int64_t row_stride,
                      const void* host, ftx_tensor** out);
/* A device tensor without data (filled by ftx_quantize or device copies). */
int ftx_tensor_alloc(ftx_ctx* ctx, int dtype, const int64_t ne[4], ftx_tensor** out);
int ftx_tensor_free(ftx_tensor* t);
void* ftx_tensor_data(ftx_tensor* t);
int64_t ftx_tensor_nbytes(const ftx_tensor* t);

/* Quantise ne1*ne2 rows of ne0 fp32 values at `src` (device) into t.
 * Synthetic-model builder: per-block symmetric fits for Q4_0/Q8_0, affine
 * 6-bit sub-block fits for Q4_K, int8 sub-block scales for Q6_K. */
int ftx_quantize(ftx_ctx* ctx, const float* src, ftx_tensor* t);

/* dst[i] = std * N(0,1) for i < n, as fp32 (FTX_F32) or fp16 (FTX_F16),
 * from a counter-based generator keyed by (seed, i): synthetic weights, KV
 * contents and activations without a host round trip. */
int ftx_fill_normal(ftx_ctx* ctx, void* dst, int dtype, int64_t n, uint64_t seed, float std);

/* ---- IBackend-level operations (synchronous, like the reference's) ---- */
/* out[r*ne0 + c] = dequant(W)[r, c] for every row, bit-exact with
 * dequant_row.  `out` may be host or device memory. */
int ftx_dequant(ftx_ctx* ctx, const ftx_tensor* W, float* out);
/* y[m*N + n] = sum_k x[m*K + k] * W[n, k], N = rows of W, K = W ne0.
 * x and y may be host or device memory. */
int ftx_matmul(ftx_ctx* ctx, const float* x, int64_t M, int64_t K, const ftx_tensor* W,
               float* y);
/* y[m*N + j] += sum_i x[m*n_in + i] * W[i, j]; W is n_in rows of N = ne0
 * columns (the reference's down orientation).  Host or device memory. */
int ftx_down_axpy(ftx_ctx* ctx, const float* x, int64_t M, int64_t n_in, const ftx_tensor* W,
                  float* y);

/* No counterpart in the reference: ftx_down_axpy for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  x and y must be device memory; the split partials
 * go to a file-scope device array of the library (16 MiB per GPU, held until
 * the process ends) instead of the context's workspace, so nothing is
 * allocated.  Shapes whose partials exceed that array return FTX_E_RANGE.
 * The result is stream-ordered: the call returns once its two kernels are
 * enqueued on the context's stream (ftx_sync, or any later synchronising
 * call, waits for them), so it may be recorded into a HIP graph.  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (several
 * streams or threads) race.  The array's address is looked up per device at
 * ftx_create; if that lookup fails, only this entry point fails
 * (FTX_E_DEVICE). */
int ftx_down_axpy_noalloc(ftx_ctx* ctx, const float* x, int64_t M, int64_t n_in,
                          const ftx_tensor* W, float* y);

/* ExpertChunkJob (include/ft/backend.h:7-19) with device pointers: gate,
 * up and down point at IC rows of resident expert weights. */
typedef struct {
    const float* x;    /* [M][K] */
    float* out;        /* [M][K], accumulated into */
    const void* gate;  /* IC rows of K cols */
    const void* up;    /* IC rows of K cols */
    const void* down;  /* IC rows of K cols (reference down orientation) */
    int32_t dt;
    int32_t pad_;
    int64_t M, K, IC;
    int64_t gate_up_row_stride, down_row_stride;  /* bytes */
} ftx_expert_job;
/* h[m,i] = silu(x_m . gate_i) * (x_m . up_i); out[m,:] += sum_i h[m,i] down_i.
 * x and out may be host or device memory; weights are device memory. */
int ftx_expert_chunk(ftx_ctx* ctx, const ftx_expert_job* job);

void* ftx_alloc_staging(ftx_ctx* ctx, size_t bytes);  /* device memory or NULL */
int ftx_free_staging(ftx_ctx* ctx, void* p);
int ftx_stage(ftx_ctx* ctx, void* dst, const void* src, size_t bytes);

/* ---- the device-resident verify step ---- */
/* per-layer tensor order in ftx_model_desc.layers[l*FTX_LAYER_TENSORS + i] */
enum {
    FTX_T_ATTN_NORM = 0,
    FTX_T_Q = 1,
    FTX_T_K = 2,
    FTX_T_V = 3,
    FTX_T_O = 4,
    FTX_T_FFN_NORM = 5,
    FTX_T_GATE = 6,
    FTX_T_UP = 7,
    FTX_T_DOWN = 8,  /* n_ff rows x n_embd cols (reference orientation) */
    FTX_LAYER_TENSORS = 9
};

/* optional per-layer tensors in ftx_model_desc.layer_ext[l*FTX_LAYER_EXT + i]
 * (NULL entries: absent).  Attention: bias vectors added after the q / k / v
 * projections and RMSNorm weights (head_dim) applied to every head of q and
 * k before RoPE (src/engine.cpp:519-542, loaded at 325-339).  MoE FFN
 * (src/engine.cpp:179-258, loaded at 348-369): a layer with a router runs
 * it instead of the dense FFN (its FTX_T_GATE / UP / DOWN are then NULL):
 * router n_expert rows of n_embd; expert planes ne = {n_embd, n_ff,
 * n_expert} (down in the reference orientation, n_ff rows of n_embd per
 * plane); optional router bias (n_expert) and shared expert (gate / up:
 * rows of n_embd; down: the same rows, reference orientation). */
enum {
    FTX_X_Q_BIAS = 0,
    FTX_X_K_BIAS = 1,
    FTX_X_V_BIAS = 2,
    FTX_X_Q_NORM = 3,
    FTX_X_K_NORM = 4,
    FTX_X_GATE_INP = 5,
    FTX_X_GATE_EXPS = 6,
    FTX_X_UP_EXPS = 7,
    FTX_X_DOWN_EXPS = 8,
    FTX_X_ROUTER_BIAS = 9,
    FTX_X_GATE_SH = 10,
    FTX_X_UP_SH = 11,
    FTX_X_DOWN_SH = 12,
    FTX_LAYER_EXT = 13
};

typedef struct {
    int64_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, vocab;
    float rms_eps;     /* the reference always ends up at 1e-5 (src/graph.cpp:42-43) */
    int32_t rope_neox; /* 0: interleaved pairs (2i, 2i+1); 1: (i, i + hd/2) */
    double rope_theta;
    const ftx_tensor* tok_embd;
    const ftx_tensor* out_norm;
    const ftx_tensor* output;  /* NULL: tied to tok_embd */
    const ftx_tensor* const* layers;  /* n_layer * FTX_LAYER_TENSORS */
    int64_t max_tokens;  /* largest M a verify step will use (<= 256) */
    const ftx_tensor* const* layer_ext;  /* NULL or n_layer * FTX_LAYER_EXT */
    /* MoE layers: experts per layer and experts routed per token
     * (ModelConfig::n_experts / n_expert_used, src/graph.cpp:48-50) */
    int64_t n_expert, n_expert_used;
} ftx_model_desc;

int ftx_model_create(ftx_ctx* ctx, const ftx_model_desc* desc, ftx_model** out);
int ftx_model_free(ftx_model* m);

/* KV cache [n_layer][cap][n_head_kv*head_dim] of kv_dtype elements. */
int ftx_kv_create(ftx_ctx* ctx, const ftx_model* m, int64_t cap, int kv_dtype, ftx_kv** out);
int ftx_kv_free(ftx_kv* kv);
/* Raw device buffers: K is [n_layer][cap_alloc][n_head_kv*head_dim], V is
 * stored transposed as [n_layer][n_head_kv][head_dim][cap_alloc], cap_alloc =
 * cap rounded up to a multiple of 128 (for fills that ignore the layout). */
int ftx_kv_pointers(ftx_kv* kv, void** k, void** v, int64_t* npast);
/* Copy the whole cache from / to host arrays in the reference layout
 * [n_layer][cap][n_head_kv*head_dim] (include/ft/kv_cache.h:10-47). */
int ftx_kv_write(ftx_kv* kv, const void* k, const void* v);
int ftx_kv_read(ftx_kv* kv, void* k, void* v);
/* Set the number of committed positions (rollback after acceptance). */
int ftx_kv_truncate(ftx_kv* kv, int64_t npast);
/* Commit an accepted draft path after a verify step that did not advance:
 * the K / V rows of draft nodes nodes[0..n-1] (strictly increasing, nodes[i]
 * >= i, n <= 256; a root-to-node path of the draft tree) move to slots
 * npast + i, then npast += n.  A chain (nodes[i] == i) moves nothing and is
 * Engine::truncate_to(npast + n) (src/engine.cpp:423-428, KvCache::set_npast
 * include/ft/kv_cache.h:31); trees extend it.  Enqueued on the context's
 * stream, ordered before later verify steps. */
int ftx_kv_commit(ftx_kv* kv, const int32_t* nodes, int64_t n);

typedef struct {
    int64_t M;               /* tokens verified in this step */
    const int32_t* tokens;   /* host [M] */
    const int32_t* parents;  /* host [M], parents[i] in {-1, 0..i-1}; NULL = chain */
    float* logits;           /* device [M][vocab]; NULL skips the LM head (prefill chunks) */
    int32_t advance;         /* 1: npast += M afterwards (chain extend_verify) */
    int32_t pad_;
} ftx_verify_args;
/* Forward of M draft tokens against the committed context: node i sits at
 * position npast + depth(i), is written to KV slot npast + i, attends to the
 * context plus its ancestors and itself.  Engine::step (src/engine.cpp:650-
 * 658) is M = 1 with advance = 1; Engine::prefill (598-648, without its
 * prefix cache) is a sequence of advancing chains, the last with logits. */
int ftx_verify_step(ftx_ctx* ctx, ftx_model* m, ftx_kv* kv, const ftx_verify_args* a);

/* Several sequences in one step (no counterpart in the reference, whose
 * Engine holds one KvCache, include/ft/kv_cache.h:10-47): sequence s
 * verifies its own draft (a chain or a tree) against its own cache, as
 * ftx_verify_step would, while every projection streams the weights once
 * for the tokens of all sequences.  At most FTX_MAX_SEQ sequences and
 * max_tokens tokens in total; every cache must be made for this model and
 * distinct; the logits pointers are all NULL (no LM head) or all set. */
enum { FTX_MAX_SEQ = 16 };
typedef struct {
    ftx_kv* kv;
    int64_t M;               /* tokens of this sequence (>= 1) */
    const int32_t* tokens;   /* host [M] */
    const int32_t* parents;  /* host [M], in this sequence's node ids, or NULL */
    float* logits;           /* device [M][vocab] or NULL */
    int32_t advance;         /* npast += M afterwards */
    int32_t pad_;
} ftx_seq_args;
int ftx_verify_batch(ftx_ctx* ctx, ftx_model* m, const ftx_seq_args* seqs, int64_t nseq);

typedef struct {
    const float* base_row;  /* device [V]: target logits before the draft */
    const float* rows;      /* device [M][V]: target logits of the M nodes */
    const float* q;         /* device [M][V] draft distributions (RESIDUAL) or NULL */
    int64_t M, V;
    const int32_t* props;   /* host [M] draft tokens */
    const int32_t* parents; /* host [M] or NULL (chain) */
    const float* pd;        /* host [M] draft prob of own token (RATIO) or NULL */
    int32_t mode;
    float temp;
    uint64_t* rng;          /* host, SplitMix64 state, in/out */
    int32_t* accepted;      /* host out [M]: accepted node ids in path order */
    int32_t* n_acc;         /* host out */
    int32_t* bonus;         /* host out: next token */
    float* margin;          /* host out: min |u - ratio| over decisions, or NULL */
    /* RATIO bonus token: Sampler::sample (include/ft/sampler.h:30-94) at
     * temp with top_k (1..64; <= 0 or >= V: off) and top_p (>= 1: off) from
     * the sampler's own SplitMix64 state (host, in/out; the reference starts
     * it at 0x9E3779B97F4A7C15 and carries it over between draws) */
    uint64_t* sampler_rng;
    int32_t top_k;
    float top_p;
} ftx_accept_args;
/* Acceptance of a verified draft (GREEDY: argmax tests, chain or tree, bonus
 * = argmax; RATIO: accept_chain_sampling's test from the rng stream, bonus by
 * the sampler; RESIDUAL: multi-candidate speculative sampling, bonus from the
 * residual distribution with one more uniform of the rng stream). */
int ftx_accept(ftx_ctx* ctx, const ftx_accept_args* a);
/* No counterpart in the reference, which runs one Engine per sequence and
 * so one acceptance per sequence: the acceptances of n (1..FTX_MAX_SEQ)
 * sequences verified in one step (ftx_verify_batch), each exactly as
 * ftx_accept would do it with its own arguments and streams, with one host
 * synchronisation and one copy each way for all of them; the GREEDY and
 * RATIO ones share one launch.  On an error the outputs of every sequence
 * are unspecified. */
int ftx_accept_batch(ftx_ctx* ctx, const ftx_accept_args* args, int n);

/* Greedy draft pick of one device row [V]: the first maximum
 * (Sampler::argmax, include/ft/sampler.h:21-28) and its probability under
 * softmax_prob at T = 1 (src/spec.cpp:89-95) -- what
 * DraftModelDrafter::draft takes per draft token (src/spec.cpp:100-119).
 * Synchronous (the host needs the token for the next step); prob may be
 * NULL. */
int ftx_argmax_prob(ftx_ctx* ctx, const float* row, int64_t V, int32_t* token, float* prob);

/* ---- kernel trace (the reference keeps wall-clock RunStats only,
 * include/ft/engine.h:25-39) ---- */
typedef struct {
    char name[24];
    int64_t launches;
    double ms;     /* summed device time between HIP events around each launch */
    double bytes;  /* summed algorithmic bytes (weights at stored size, KV, rows) */
    /* the class's main kernel timed on its own dispatch (events carried by
     * the launch itself: kernel start to end, no bracket time) */
    int64_t kernel_launches;
    double kernel_ms;
} ftx_trace_entry;
/* enable != 0 starts recording (and clears earlier records, then records
 * 32 empty event brackets as the entry "event_pair": the time a bracket adds
 * by itself); 0 stops. */
int ftx_trace(ftx_ctx* ctx, int enable);
/* Waits for the stream, then returns one entry per kernel class seen. */
int ftx_trace_read(ftx_ctx* ctx, ftx_trace_entry* out, int max, int* n);
/* Measurement hook with no counterpart in the reference: while tracing,
 * each launch of class `kind` (a trace entry name) whose outputs do not
 * depend on its own earlier results is issued `times` times back to back
 * between its events (counted as `times` launches), so that a class's
 * average launch time is not dominated by the events' own overhead.
 * times = 1 switches it off. */
int ftx_trace_replay(ftx_ctx* ctx, const char* kind, int times);

#ifdef __cplusplus
}
#endif
#endif
