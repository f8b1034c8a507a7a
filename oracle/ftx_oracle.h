/*
 * ftx_oracle.h -- CPU oracle for the speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  Nothing in the product
 * (xwfes_amd/) links or calls it.
 *
 * Every function restates the reference algorithm in plain C and cites the
 * reference file:line it follows (paths relative to ft-igpu-src/).  Where the
 * reference has no code (Q4_K/Q6_K, tree attention, tree acceptance, residual
 * resampling, fp16 KV) the restatement follows the public algorithm named at
 * the function and is pinned by the closed-form / invariant tests in tests/.
 *
 * Reference bugs fixed here (each is flagged at the function):
 *   - CpuBackend::matmul sums the M rows into y[r] (src/cpu_backend.cpp:95-103);
 *     orc_matmul writes y[m*N + r].
 *   - forward() embeds with HostTensor::slice(t), a plane index
 *     (src/engine.cpp:494-495, include/ft/types.h:134-137); orc_forward looks
 *     up row t.
 *   - generate() samples the bonus token from rows[min(acc,k-1)]
 *     (src/spec.cpp:309-311); orc_verify_accept samples it from the row that
 *     follows the last accepted node.
 *   - Sampler::sample re-seeds on every call when its seed is non-zero
 *     (include/ft/sampler.h:31); orc_sampler_sample carries the state over.
 */
#ifndef FTX_ORACLE_H
#define FTX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype ids: the reference's DType values (include/ft/types.h:20-27) plus the
 * ggml ids for the K-quants the reference lacks. */
enum {
    ORC_F32 = 0,
    ORC_F16 = 1,
    ORC_Q4_0 = 2,
    ORC_Q4_1 = 3,
    ORC_Q8_0 = 8,
    ORC_Q4_K = 12,
    ORC_Q6_K = 14,
    ORC_BF16 = 30
};

/* ---- scalar formats (include/ft/types.h:60-117) ---- */
float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
float orc_bf16_to_float(uint16_t b);

/* ---- block formats ---- */
int64_t orc_block_elems(int dtype);
int64_t orc_block_bytes(int dtype);
int64_t orc_row_bytes(int dtype, int64_t ncols);
/* returns 0 on success, -1 for an unsupported dtype */
int orc_dequant_row(float* dst, const uint8_t* src, int dtype, int64_t n);
float orc_dot_row_f32(const float* x, const uint8_t* w, int dtype, int64_t n);
/* test-data quantisers (no reference counterpart is needed for parity: the
 * dequant of whatever bytes they emit is what is checked) */
int orc_quantize_row(uint8_t* dst, const float* src, int dtype, int64_t n);

/* ---- linear algebra, host ops ---- */
void orc_set_threads(int n);
int orc_get_threads(void);
/* y[m*N + r] = sum_k x[m*K + k] * W[r, k]; W is N rows of K cols. */
void orc_matmul(const float* x, int64_t M, int64_t K, const uint8_t* W,
                int dtype, int64_t N, float* y);
/* y[m*N + j] += sum_i x[m*n_in + i] * W[i, j]; W is n_in rows of N cols. */
void orc_down_axpy(const float* x, int64_t M, int64_t n_in, const uint8_t* W,
                   int dtype, int64_t N, float* y);
void orc_rms_norm(float* out, const float* x, const float* w, int64_t n,
                  float eps);
void orc_rope_vec(float* v, int64_t hd, int64_t pos, double theta, int neox);
void orc_softmax_inplace(float* p, int64_t n);

/* ---- model ---- */
typedef struct {
    const uint8_t* data; /* GGUF bytes, rows of ne0 elements */
    int32_t dtype;
    int32_t pad_;
    int64_t ne0; /* cols (contiguous) */
    int64_t ne1; /* rows */
} orc_tensor;

/* per-layer tensor order in orc_model.layers[l*ORC_LAYER_TENSORS + i] */
enum {
    ORC_T_ATTN_NORM = 0,
    ORC_T_Q = 1,
    ORC_T_K = 2,
    ORC_T_V = 3,
    ORC_T_O = 4,
    ORC_T_FFN_NORM = 5,
    ORC_T_GATE = 6,
    ORC_T_UP = 7,
    ORC_T_DOWN = 8,  /* reference orientation: n_ff rows x n_embd cols */
    ORC_LAYER_TENSORS = 9
};

/* optional per-layer tensors (data == NULL: absent), in
 * orc_model.ext[l*ORC_LAYER_EXT + i]:
 *   attention bias added after the q / k / v projections and per-head
 *   RMSNorm of q and k (src/engine.cpp:519-542, loaded at 325-332);
 *   the MoE FFN (src/engine.cpp:179-258, loaded at 348-369): the router
 *   (n_expert rows of n_embd), its optional bias, the experts' gate / up /
 *   down planes (n_expert planes of n_ff rows x n_embd cols, down in the
 *   reference orientation) and an optional shared expert */
enum {
    ORC_X_Q_BIAS = 0,
    ORC_X_K_BIAS = 1,
    ORC_X_V_BIAS = 2,
    ORC_X_Q_NORM = 3,
    ORC_X_K_NORM = 4,
    ORC_X_GATE_INP = 5,
    ORC_X_GATE_EXPS = 6,
    ORC_X_UP_EXPS = 7,
    ORC_X_DOWN_EXPS = 8,
    ORC_X_ROUTER_BIAS = 9,
    ORC_X_GATE_SH = 10,
    ORC_X_UP_SH = 11,
    ORC_X_DOWN_SH = 12,
    ORC_LAYER_EXT = 13
};

typedef struct {
    int64_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, vocab;
    float rms_eps;
    int32_t rope_neox;
    double rope_theta;
    orc_tensor tok_embd;
    orc_tensor out_norm;
    orc_tensor output; /* data == NULL -> tied to tok_embd */
    const orc_tensor* layers;
    const orc_tensor* ext;  /* NULL or n_layer * ORC_LAYER_EXT */
    int64_t n_expert, n_expert_used;  /* a layer with a router runs the MoE FFN */
} orc_model;

/* one expert's SwiGLU FFN, out[S][K] += ...; h1 / h2 scratch of S*F floats
 * or NULL (src/cpu_backend.cpp:106-149 over all F neurons) */
void orc_expert_ffn(const float* x, int64_t S, int64_t K, const uint8_t* gate, const uint8_t* up,
                    int gu_dt, const uint8_t* down, int down_dt, int64_t F, float* out,
                    float* h1, float* h2);

/* MoE routing of M router rows [M][E] (src/engine.cpp:197-217): the row
 * plus the optional bias, softmax_inplace, the top U by value (ties: lower
 * expert index), weights renormalised by their float sum; experts listed in
 * first-use order over (token, rank).  out_e / out_w [M*U]: expert and
 * weight of (token m, rank u); used [E], n_used: the first-use order.
 * router is modified in place (the probabilities). */
void orc_moe_route(float* router, int64_t M, int64_t E, int64_t U, const float* bias,
                   int32_t* out_e, float* out_w, int32_t* used, int32_t* n_used);

/* KV cache element type for orc_forward */
enum { ORC_KV_F32 = 0, ORC_KV_F16 = 1 };

/*
 * Forward of M tokens (src/engine.cpp:461-596) with a draft-tree extension.
 *   kcache/vcache: [n_layer][cap][n_head_kv*head_dim], kv_dtype elements.
 *   parents: NULL for a chain (reference causal attention); else parents[i]
 *     in {-1, 0..i-1}; node i sits at position npast + depth(i), is written
 *     to KV slot npast + i and attends to the context plus its ancestors.
 *   logits: [M][vocab].
 *   layer_limit <= 0: all layers.
 * Returns 0, or -1 on invalid input.
 */
int orc_forward(const orc_model* mdl, void* kcache, void* vcache, int kv_dtype,
                int64_t cap, int64_t npast, const int32_t* toks, int64_t M,
                const int32_t* parents, int layer_limit, float* logits);

/* ---- sampling / acceptance (src/spec.cpp, include/ft/sampler.h) ---- */
uint64_t orc_rng_next(uint64_t* s);
float orc_rng_float(uint64_t* s);
int32_t orc_argmax(const float* row, int64_t n);
float orc_softmax_prob(const float* logits, int64_t V, int32_t t, float temp);
int orc_accept_chain_greedy(const float* base_row, const float* rows,
                            int64_t V, const int32_t* props, int64_t k);
int orc_accept_chain_sampling(const float* base_row, const float* rows,
                              const float* pd, int64_t V, const int32_t* props,
                              int64_t k, float temp, uint64_t* rng);

enum {
    ORC_ACCEPT_GREEDY = 0,   /* argmax match, chain or tree */
    ORC_ACCEPT_RATIO = 1,    /* reference ratio test with scalar pd, chain */
    ORC_ACCEPT_RESIDUAL = 2  /* multi-candidate speculative sampling, full q */
};

/* index of the first w_i whose running double sum exceeds u * sum(w) */
int32_t orc_sample_weights(const double* w, int64_t V, float u);

/*
 * Full verify-step acceptance (chain or tree) plus the bonus token.
 *   rows: [M][V] target logits of the M nodes; base_row: logits before them.
 *   parents: NULL = chain.  pd: [M] draft prob of each node's own token
 *   (RATIO).  q: [M][V] draft distribution each node's token was drawn
 *   from (RESIDUAL).  accepted: out, node ids along the accepted path (<= M);
 *   *n_acc: out count; *bonus: out next token; *margin: min |u - ratio| seen.
 * Returns 0 or -1.
 */
int orc_verify_accept(const float* base_row, const float* rows, int64_t M,
                      int64_t V, const int32_t* props, const int32_t* parents,
                      const float* pd, const float* q, int mode, float temp,
                      uint64_t* rng, uint64_t* sampler_state, int32_t top_k, float top_p,
                      int32_t* accepted, int32_t* n_acc, int32_t* bonus, float* margin);

/* Sampler::sample (include/ft/sampler.h:30-94) with its state carried over
 * between calls; top_k <= 0 or >= n and top_p >= 1 switch the filters off. */
int32_t orc_sampler_sample(const float* lg, int64_t n, float temp, int32_t top_k, float top_p,
                           uint64_t* state);

#ifdef __cplusplus
}
#endif
#endif
