/*
 * model.c -- host ops and the M-token forward of the CPU oracle (test
 * infrastructure; see ftx_oracle.h).  Loop nests and accumulation orders
 * follow the reference so the oracle doubles as the "reference loop nest"
 * CPU baseline; OpenMP only splits independent outputs, never a sum.
 */
#include "ftx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void orc_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int orc_get_threads(void) { return g_threads; }

/*
 * y[m*N + r] = x_m . W_r.  Loop nest of CpuBackend::matmul
 * (src/cpu_backend.cpp:90-104: rows split over threads, dot_row_f32 per
 * (row, m)) with the M-sum bug fixed: the reference writes
 * y[r] = sum_m x_m . W_r (cpu_backend.cpp:98-101).
 */
void orc_matmul(const float* x, int64_t M, int64_t K, const uint8_t* W,
                int dt, int64_t N, float* y) {
    const int64_t stride = orc_row_bytes(dt, K);
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t r = 0; r < N; ++r) {
        const uint8_t* wr = W + stride * r;
        for (int64_t m = 0; m < M; ++m) y[m * N + r] = orc_dot_row_f32(x + m * K, wr, dt, K);
    }
}

/*
 * y[m, :] += x[m, i] * W[i, :] for i < n_in, skipping x == 0; W is n_in rows
 * of N columns (reference down orientation).  src/cpu_backend.cpp:60-75.
 * The reference runs this on one thread; here columns are split over
 * threads, which leaves every output's summation order (ascending i)
 * unchanged.
 */
void orc_down_axpy(const float* x, int64_t M, int64_t n_in, const uint8_t* W,
                   int dt, int64_t N, float* y) {
    const int64_t stride = orc_row_bytes(dt, N);
    int nt = g_threads;
    if (nt > 1 && N % 256 == 0) {
        int64_t nchunk = N / 256;
#pragma omp parallel for schedule(static) num_threads(nt)
        for (int64_t c = 0; c < nchunk; ++c) {
            float row[256];
            const int64_t j0 = c * 256;
            /* a 256-column window starts on a block boundary for every
             * supported block size (1, 32, 256) */
            const int64_t off = orc_row_bytes(dt, j0);
            for (int64_t i = 0; i < n_in; ++i) {
                orc_dequant_row(row, W + stride * i + off, dt, 256);
                for (int64_t m = 0; m < M; ++m) {
                    const float v = x[m * n_in + i];
                    if (v == 0.f) continue;
                    float* ym = y + m * N + j0;
                    for (int64_t j = 0; j < 256; ++j) ym[j] += v * row[j];
                }
            }
        }
        return;
    }
    float* row = (float*)malloc((size_t)N * sizeof(float));
    for (int64_t i = 0; i < n_in; ++i) {
        orc_dequant_row(row, W + stride * i, dt, N);
        for (int64_t m = 0; m < M; ++m) {
            const float v = x[m * n_in + i];
            if (v == 0.f) continue;
            float* ym = y + m * N;
            for (int64_t j = 0; j < N; ++j) ym[j] += v * row[j];
        }
    }
    free(row);
}

/* src/engine.cpp:23-41: float sequential sum of squares,
 * inv = 1/sqrt(ss/n + eps), out = (x * inv) * w */
void orc_rms_norm(float* out, const float* x, const float* w, int64_t n, float eps) {
    float ss = 0.f;
    for (int64_t i = 0; i < n; ++i) ss += x[i] * x[i];
    const float inv = 1.f / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; ++i) out[i] = w ? x[i] * inv * w[i] : x[i] * inv;
}

/* src/engine.cpp:43-60: frequencies and angles in double, cos/sin rounded
 * to float; neox pairs (i, i+hd/2), otherwise interleaved (2i, 2i+1) */
void orc_rope_vec(float* v, int64_t hd, int64_t pos, double theta, int neox) {
    for (int64_t i = 0; i < hd / 2; ++i) {
        const double f = pow(theta, -2.0 * (double)i / (double)hd);
        const double ang = (double)pos * f;
        const float c = (float)cos(ang), s = (float)sin(ang);
        const int64_t ia = neox ? i : 2 * i, ib = neox ? i + hd / 2 : 2 * i + 1;
        const float a = v[ia], b = v[ib];
        v[ia] = a * c - b * s;
        v[ib] = a * s + b * c;
    }
}

/* src/engine.cpp:62-72: float max, float exp, double sum, float scale */
void orc_softmax_inplace(float* p, int64_t n) {
    float mx = p[0];
    for (int64_t i = 1; i < n; ++i) mx = fmaxf(mx, p[i]);
    double sum = 0;
    for (int64_t i = 0; i < n; ++i) {
        p[i] = expf(p[i] - mx);
        sum += p[i];
    }
    const float inv = (float)(1.0 / sum);
    for (int64_t i = 0; i < n; ++i) p[i] *= inv;
}

static float kv_get(const void* c, int kv_dt, int64_t idx) {
    return kv_dt == ORC_KV_F16 ? orc_half_to_float(((const uint16_t*)c)[idx])
                               : ((const float*)c)[idx];
}

static void kv_put(void* c, int kv_dt, int64_t idx, float v) {
    if (kv_dt == ORC_KV_F16) ((uint16_t*)c)[idx] = orc_float_to_half(v);
    else ((float*)c)[idx] = v;
}

/* dequantise one vector-shaped tensor (norm weights) */
static float* vec_f32(const orc_tensor* t, int64_t n) {
    float* v = (float*)malloc((size_t)n * sizeof(float));
    orc_dequant_row(v, t->data, t->dtype, n);
    return v;
}

static const orc_tensor* ext_of(const orc_model* md, int64_t l, int i) {
    if (!md->ext) return NULL;
    const orc_tensor* t = md->ext + l * ORC_LAYER_EXT + i;
    return t->data ? t : NULL;
}

/* src/engine.cpp:197-217 */
void orc_moe_route(float* router, int64_t M, int64_t E, int64_t U, const float* bias,
                   int32_t* out_e, float* out_w, int32_t* used, int32_t* n_used) {
    int32_t* first = (int32_t*)malloc((size_t)E * sizeof(int32_t));
    for (int64_t e = 0; e < E; ++e) first[e] = 0;
    *n_used = 0;
    for (int64_t m = 0; m < M; ++m) {
        float* r = router + m * E;
        if (bias)
            for (int64_t j = 0; j < E; ++j) r[j] += bias[j];
        orc_softmax_inplace(r, E);
        /* the U largest in descending order, a tie to the lower index: the
         * order std::partial_sort gives for distinct values */
        int32_t* top = out_e + m * U;
        for (int64_t u = 0; u < U; ++u) {
            int32_t best = -1;
            for (int64_t j = 0; j < E; ++j) {
                int taken = 0;
                for (int64_t v = 0; v < u; ++v) taken |= top[v] == j;
                if (taken) continue;
                if (best < 0 || r[j] > r[best]) best = (int32_t)j;
            }
            top[u] = best;
        }
        float wsum = 0.f;
        for (int64_t u = 0; u < U; ++u) wsum += r[top[u]];
        const float inv = wsum > 0 ? 1.f / wsum : 0.f;
        for (int64_t u = 0; u < U; ++u) {
            out_w[m * U + u] = r[top[u]] * inv;
            if (!first[top[u]]) {
                first[top[u]] = 1;
                used[(*n_used)++] = top[u];
            }
        }
    }
    free(first);
}

/* one expert's SwiGLU FFN over S rows: out[S][K] += down^T (silu(x gate^T)
 * * (x up^T)); gate / up are F rows of K, down F rows of K (reference
 * orientation).  The reference runs it in windows of neurons
 * (include/ft/chunker.h:32-77, src/cpu_backend.cpp:106-149) whose down rows
 * add in ascending order, so one pass over all F gives the same sums.
 * h1 / h2: scratch of S*F floats each (NULL: allocated here). */
void orc_expert_ffn(const float* x, int64_t S, int64_t K, const uint8_t* gate, const uint8_t* up,
                    int gu_dt, const uint8_t* down, int down_dt, int64_t F, float* out,
                    float* h1, float* h2) {
    float* a = h1 ? h1 : (float*)malloc((size_t)(S * F) * sizeof(float));
    float* b = h2 ? h2 : (float*)malloc((size_t)(S * F) * sizeof(float));
    orc_matmul(x, S, K, gate, gu_dt, F, a);
    orc_matmul(x, S, K, up, gu_dt, F, b);
    for (int64_t i = 0; i < S * F; ++i) {
        float g = a[i];
        g = g / (1.f + expf(-g));
        a[i] = g * b[i];
    }
    orc_down_axpy(a, S, F, down, down_dt, K, out);
    if (!h1) free(a);
    if (!h2) free(b);
}

/* src/engine.cpp:179-258: router, per-expert SwiGLU FFN over the expert's
 * rows (ExpertStreamer windows add the down rows in ascending order, which a
 * single pass reproduces, include/ft/chunker.h:32-89 and
 * src/cpu_backend.cpp:106-149), the weighted sum into tmpo in first-use
 * order, then the optional shared expert */
static void moe_ffn(const orc_model* md, int64_t l, const float* xn, int64_t M, float* tmpo) {
    const int64_t K = md->n_embd, E = md->n_expert;
    const int64_t U = md->n_expert_used < E ? md->n_expert_used : E;
    const orc_tensor* gi = ext_of(md, l, ORC_X_GATE_INP);
    const orc_tensor* ge = ext_of(md, l, ORC_X_GATE_EXPS);
    const orc_tensor* ue = ext_of(md, l, ORC_X_UP_EXPS);
    const orc_tensor* de = ext_of(md, l, ORC_X_DOWN_EXPS);
    const orc_tensor* rb = ext_of(md, l, ORC_X_ROUTER_BIAS);
    const int64_t F = ge->ne1 / E;  /* rows per expert plane */
    float* router = (float*)malloc((size_t)(M * E) * sizeof(float));
    orc_matmul(xn, M, K, gi->data, gi->dtype, E, router);
    float* bias = rb ? vec_f32(rb, E) : NULL;
    int32_t* te = (int32_t*)malloc((size_t)(M * U) * sizeof(int32_t));
    float* tw = (float*)malloc((size_t)(M * U) * sizeof(float));
    int32_t* used = (int32_t*)malloc((size_t)E * sizeof(int32_t));
    int32_t n_used = 0;
    orc_moe_route(router, M, E, U, bias, te, tw, used, &n_used);
    float* xe = (float*)malloc((size_t)(M * K) * sizeof(float));
    float* acb = (float*)malloc((size_t)(M * K) * sizeof(float));
    float* h1 = (float*)malloc((size_t)(M * F) * sizeof(float));
    float* h2 = (float*)malloc((size_t)(M * F) * sizeof(float));
    int64_t* rows_m = (int64_t*)malloc((size_t)M * sizeof(int64_t));
    float* rows_w = (float*)malloc((size_t)M * sizeof(float));
    const int64_t gstride = orc_row_bytes(ge->dtype, K) * F;
    const int64_t ustride = orc_row_bytes(ue->dtype, K) * F;
    const int64_t dstride = orc_row_bytes(de->dtype, K) * F;
    for (int32_t ui = 0; ui < n_used; ++ui) {
        const int32_t e = used[ui];
        int64_t S = 0;
        for (int64_t m = 0; m < M; ++m)
            for (int64_t u = 0; u < U; ++u)
                if (te[m * U + u] == e) {
                    rows_m[S] = m;
                    rows_w[S] = tw[m * U + u];
                    memcpy(xe + S * K, xn + m * K, (size_t)K * sizeof(float));
                    ++S;
                }
        memset(acb, 0, (size_t)(S * K) * sizeof(float));
        orc_expert_ffn(xe, S, K, ge->data + gstride * e, ue->data + ustride * e, ge->dtype,
                       de->data + dstride * e, de->dtype, F, acb, h1, h2);
        for (int64_t si = 0; si < S; ++si) {
            float* trow = tmpo + rows_m[si] * K;
            const float* arow = acb + si * K;
            for (int64_t j = 0; j < K; ++j) trow[j] += rows_w[si] * arow[j];
        }
    }
    const orc_tensor* sg = ext_of(md, l, ORC_X_GATE_SH);
    const orc_tensor* su = ext_of(md, l, ORC_X_UP_SH);
    const orc_tensor* sd = ext_of(md, l, ORC_X_DOWN_SH);
    if (sg && su && sd)
        orc_expert_ffn(xn, M, K, sg->data, su->data, sg->dtype, sd->data, sd->dtype, sg->ne1,
                       tmpo, NULL, NULL);
    free(router); free(bias); free(te); free(tw); free(used); free(xe); free(acb);
    free(h1); free(h2); free(rows_m); free(rows_w);
}

/* src/engine.cpp:519-542: bias on q / k / v, then RMSNorm of every head of q
 * and of k with the norm vector of head_dim */
static void attn_extras(const orc_model* md, int64_t l, int64_t M, float* q, float* kb, float* vb) {
    const int64_t hd = md->head_dim, nh = md->n_head, dk = md->n_head_kv * hd;
    const orc_tensor* bq = ext_of(md, l, ORC_X_Q_BIAS);
    const orc_tensor* bk = ext_of(md, l, ORC_X_K_BIAS);
    const orc_tensor* bv = ext_of(md, l, ORC_X_V_BIAS);
    const orc_tensor* nq = ext_of(md, l, ORC_X_Q_NORM);
    const orc_tensor* nk = ext_of(md, l, ORC_X_K_NORM);
    float* buf[3] = {q, kb, vb};
    const orc_tensor* bias[3] = {bq, bk, bv};
    const int64_t dim[3] = {nh * hd, dk, dk};
    for (int b = 0; b < 3; ++b) {
        if (!bias[b]) continue;
        float* bv32 = vec_f32(bias[b], dim[b]);
        for (int64_t m = 0; m < M; ++m)
            for (int64_t j = 0; j < dim[b]; ++j) buf[b][m * dim[b] + j] += bv32[j];
        free(bv32);
    }
    const orc_tensor* nrm[2] = {nq, nk};
    const int64_t heads[2] = {nh, md->n_head_kv};
    for (int b = 0; b < 2; ++b) {
        if (!nrm[b]) continue;
        float* w = vec_f32(nrm[b], hd);
        for (int64_t m = 0; m < M; ++m)
            for (int64_t h = 0; h < heads[b]; ++h) {
                float* v = buf[b] + (m * heads[b] + h) * hd;
                orc_rms_norm(v, v, w, hd, md->rms_eps);
            }
        free(w);
    }
}

int orc_forward(const orc_model* md, void* kc, void* vc, int kv_dt, int64_t cap,
                int64_t npast, const int32_t* toks, int64_t M,
                const int32_t* parents, int layer_limit, float* logits) {
    if (!md || M <= 0) return -1;
    const int64_t K = md->n_embd, hd = md->head_dim, nh = md->n_head;
    const int64_t nkv = md->n_head_kv, dk = nkv * hd, V = md->vocab, F = md->n_ff;
    const int64_t gqa = nh / nkv;
    if (npast + M > cap) return -1;
    for (int64_t m = 0; m < M; ++m) {
        if (toks[m] < 0 || toks[m] >= V) return -1;
        if (parents && (parents[m] < -1 || parents[m] >= m)) return -1;
    }
    const int64_t nl = layer_limit > 0 && layer_limit < md->n_layer ? layer_limit : md->n_layer;

    /* tree geometry: depth, ancestor mask (chain == causal) */
    int64_t* depth = (int64_t*)malloc((size_t)M * sizeof(int64_t));
    uint8_t* anc = (uint8_t*)calloc((size_t)(M * M), 1);
    for (int64_t m = 0; m < M; ++m) {
        int64_t p = parents ? parents[m] : m - 1;
        depth[m] = p < 0 ? 0 : depth[p] + 1;
        anc[m * M + m] = 1;
        if (p >= 0)
            for (int64_t j = 0; j < M; ++j) anc[m * M + j] |= anc[p * M + j];
    }

    float* x = (float*)malloc((size_t)(M * K) * sizeof(float));
    float* xn = (float*)malloc((size_t)(M * K) * sizeof(float));
    float* q = (float*)malloc((size_t)(M * nh * hd) * sizeof(float));
    float* kb = (float*)malloc((size_t)(M * dk) * sizeof(float));
    float* vb = (float*)malloc((size_t)(M * dk) * sizeof(float));
    float* att = (float*)malloc((size_t)(M * nh * hd) * sizeof(float));
    float* tmpo = (float*)malloc((size_t)(M * K) * sizeof(float));
    float* h1 = (float*)malloc((size_t)(M * F) * sizeof(float));
    float* h2 = (float*)malloc((size_t)(M * F) * sizeof(float));

    /* embedding: row lookup of token t (fix of the plane-index bug at
     * src/engine.cpp:494-495); any dtype is dequantised */
    const int64_t erow = orc_row_bytes(md->tok_embd.dtype, K);
    for (int64_t m = 0; m < M; ++m)
        orc_dequant_row(x + m * K, md->tok_embd.data + erow * toks[m], md->tok_embd.dtype, K);

    const float scale = 1.f / sqrtf((float)hd);
    for (int64_t l = 0; l < nl; ++l) {
        const orc_tensor* T = md->layers + l * ORC_LAYER_TENSORS;
        float* an = vec_f32(&T[ORC_T_ATTN_NORM], K);
        for (int64_t m = 0; m < M; ++m) orc_rms_norm(xn + m * K, x + m * K, an, K, md->rms_eps);
        free(an);
        orc_matmul(xn, M, K, T[ORC_T_Q].data, T[ORC_T_Q].dtype, nh * hd, q);
        orc_matmul(xn, M, K, T[ORC_T_K].data, T[ORC_T_K].dtype, dk, kb);
        orc_matmul(xn, M, K, T[ORC_T_V].data, T[ORC_T_V].dtype, dk, vb);
        attn_extras(md, l, M, q, kb, vb);
        /* src/engine.cpp:544-551, position = npast + depth */
        for (int64_t m = 0; m < M; ++m) {
            for (int64_t h = 0; h < nh; ++h)
                orc_rope_vec(q + (m * nh + h) * hd, hd, npast + depth[m], md->rope_theta, md->rope_neox);
            for (int64_t h = 0; h < nkv; ++h)
                orc_rope_vec(kb + m * dk + h * hd, hd, npast + depth[m], md->rope_theta, md->rope_neox);
        }
        /* KV write at slots [npast, npast+M) (src/engine.cpp:555-561); the
         * block is then read back from the cache like the reference does */
        for (int64_t m = 0; m < M; ++m)
            for (int64_t j = 0; j < dk; ++j) {
                kv_put(kc, kv_dt, (l * cap + npast + m) * dk + j, kb[m * dk + j]);
                kv_put(vc, kv_dt, (l * cap + npast + m) * dk + j, vb[m * dk + j]);
            }
        /* attention, src/engine.cpp:137-177, with the ancestor mask */
#pragma omp parallel for schedule(static) num_threads(g_threads)
        for (int64_t idx = 0; idx < M * nh; ++idx) {
            const int64_t m = idx / nh, h = idx % nh, kvh = h / gqa;
            const float* qs = q + (m * nh + h) * hd;
            const int64_t len = npast + M;
            float* sc = (float*)malloc((size_t)len * sizeof(float));
            int64_t* slot = (int64_t*)malloc((size_t)len * sizeof(int64_t));
            int64_t n = 0;
            for (int64_t p = 0; p < npast; ++p) slot[n++] = p;
            for (int64_t j = 0; j < M; ++j)
                if (anc[m * M + j]) slot[n++] = npast + j;
            for (int64_t s = 0; s < n; ++s) {
                const int64_t base = (l * cap + slot[s]) * dk + kvh * hd;
                float d = 0.f;
                for (int64_t t = 0; t < hd; ++t) d += qs[t] * kv_get(kc, kv_dt, base + t);
                sc[s] = d * scale;
            }
            orc_softmax_inplace(sc, n);
            float* os = att + (m * nh + h) * hd;
            for (int64_t t = 0; t < hd; ++t) os[t] = 0.f;
            for (int64_t s = 0; s < n; ++s) {
                const float w = sc[s];
                if (w == 0.f) continue;
                const int64_t base = (l * cap + slot[s]) * dk + kvh * hd;
                for (int64_t t = 0; t < hd; ++t) os[t] += w * kv_get(vc, kv_dt, base + t);
            }
            free(sc);
            free(slot);
        }
        orc_matmul(att, M, nh * hd, T[ORC_T_O].data, T[ORC_T_O].dtype, K, tmpo);
        for (int64_t i = 0; i < M * K; ++i) x[i] += tmpo[i];
        float* fn = vec_f32(&T[ORC_T_FFN_NORM], K);
        for (int64_t m = 0; m < M; ++m) orc_rms_norm(xn + m * K, x + m * K, fn, K, md->rms_eps);
        free(fn);
        memset(tmpo, 0, (size_t)(M * K) * sizeof(float));
        if (ext_of(md, l, ORC_X_GATE_INP)) {
            moe_ffn(md, l, xn, M, tmpo);
        } else {
            /* dense FFN, src/engine.cpp:260-276 */
            orc_matmul(xn, M, K, T[ORC_T_GATE].data, T[ORC_T_GATE].dtype, F, h1);
            orc_matmul(xn, M, K, T[ORC_T_UP].data, T[ORC_T_UP].dtype, F, h2);
            for (int64_t i = 0; i < M * F; ++i) {
                float g = h1[i];
                g = g / (1.f + expf(-g));
                h1[i] = g * h2[i];
            }
            orc_down_axpy(h1, M, F, T[ORC_T_DOWN].data, T[ORC_T_DOWN].dtype, K, tmpo);
        }
        for (int64_t i = 0; i < M * K; ++i) x[i] += tmpo[i];
    }
    /* final norm and LM head (tied to tok_embd when output is absent),
     * src/engine.cpp:583-589 */
    float* on = vec_f32(&md->out_norm, K);
    for (int64_t m = 0; m < M; ++m) orc_rms_norm(xn + m * K, x + m * K, on, K, md->rms_eps);
    free(on);
    const orc_tensor* lm = md->output.data ? &md->output : &md->tok_embd;
    orc_matmul(xn, M, K, lm->data, lm->dtype, V, logits);

    free(depth); free(anc); free(x); free(xn); free(q); free(kb); free(vb);
    free(att); free(tmpo); free(h1); free(h2);
    return 0;
}
