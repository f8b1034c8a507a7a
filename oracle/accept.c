/*
 * accept.c -- acceptance sampling of the CPU oracle (test infrastructure;
 * see ftx_oracle.h).
 */
#include "ftx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* SplitMix64 (Steele, Lea, Flood 2014) as used by src/spec.cpp:10-16 */
uint64_t orc_rng_next(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* top 24 bits scaled by 2^-24, src/spec.cpp:17 */
float orc_rng_float(uint64_t* s) {
    return (float)(orc_rng_next(s) >> 40) * (1.f / 16777216.f);
}

/* first maximum wins (strict >), include/ft/sampler.h:21-28 */
int32_t orc_argmax(const float* row, int64_t n) {
    int32_t best = 0;
    float bv = row[0];
    for (int64_t i = 1; i < n; ++i)
        if (row[i] > bv) { bv = row[i]; best = (int32_t)i; }
    return best;
}

/*
 * p_T(t) = exp(z_t) / sum_i exp(z_i) with z_i = (l_i - max) / T computed in
 * float, exp and sum in double, result rounded to float.  With T == 1 this
 * is exactly prob_of / softmax_prob (src/spec.cpp:217-223, 89-95); the
 * reference ignores the temperature argument (spec.cpp:216), T != 1 is the
 * documented extension p = softmax(l / T).
 */
float orc_softmax_prob(const float* lg, int64_t V, int32_t t, float temp) {
    float mx = lg[0];
    for (int64_t i = 1; i < V; ++i) mx = fmaxf(mx, lg[i]);
    double sum = 0;
    for (int64_t i = 0; i < V; ++i) sum += exp((double)((lg[i] - mx) / temp));
    return (float)(exp((double)((lg[t] - mx) / temp)) / sum);
}

/* src/spec.cpp:203-212; row a-1 predicts position a, base_row predicts 0 */
int orc_accept_chain_greedy(const float* base_row, const float* rows, int64_t V,
                            const int32_t* props, int64_t k) {
    int a = 0;
    while (a < k) {
        const float* pred = a == 0 ? base_row : rows + (a - 1) * V;
        if (orc_argmax(pred, V) != props[a]) break;
        ++a;
    }
    return a;
}

/* src/spec.cpp:214-238: pd <= 0 -> greedy test; else reject iff
 * u > min(1, pt / max(pd, 1e-9)), one u per stochastic position evaluated */
int orc_accept_chain_sampling(const float* base_row, const float* rows,
                              const float* pd, int64_t V, const int32_t* props,
                              int64_t k, float temp, uint64_t* rng) {
    int a = 0;
    while (a < k) {
        const float* pred = a == 0 ? base_row : rows + (a - 1) * V;
        if (pd[a] <= 0.f) {
            if (orc_argmax(pred, V) != props[a]) break;
        } else {
            const float pt = orc_softmax_prob(pred, V, props[a], temp);
            const float ratio = fminf(1.f, pt / fmaxf(pd[a], 1e-9f));
            if (orc_rng_float(rng) > ratio) break;
        }
        ++a;
    }
    return a;
}

/* inverse CDF: first i whose running double sum exceeds u * total */
int32_t orc_sample_weights(const double* w, int64_t V, float u) {
    double tot = 0;
    for (int64_t i = 0; i < V; ++i) tot += w[i];
    const double target = (double)u * tot;
    double c = 0;
    int32_t last = 0;
    for (int64_t i = 0; i < V; ++i) {
        if (w[i] > 0) last = (int32_t)i;
        c += w[i];
        if (c > target) return (int32_t)i;
    }
    return last;
}

/* Sampler::sample (include/ft/sampler.h:30-94): temp <= 0 -> first-max
 * argmax; else p_i = expf((l_i - max) / T) in float, their double sum,
 * p_i = (float)(p_i / sum); top-k (0 < k < n): the k largest p (ties: lower
 * index first, the reference's partial_sort leaves tie order unspecified),
 * renormalised by their float sum taken in that order; top-p (p < 1): all p
 * in descending order (same ties), double cumulative sum cut at the first
 * cum >= top_p, the rest zeroed and its double sum `tail` divided out of the
 * kept (when tail > 0); then r = next_float() and the first i in index order
 * whose running double sum, as float, reaches r; none: argmax.  The state
 * carries over between calls (the reference re-seeds on every call when its
 * seed is non-zero, which makes every draw the same; with seed 0 its state
 * carries over in the same way).  next_float: SplitMix64 step, bits 24..47
 * of the output as a 24-bit fraction (sampler.h:84-92). */
static float sampler_next_float(uint64_t* st) {
    *st += 0x9E3779B97F4A7C15ull;
    uint64_t z = *st;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    const uint32_t u = (uint32_t)((z ^ (z >> 31)) >> 16);
    return (float)(u >> 8) * (1.f / 16777216.f);
}

static const float* g_sort_p;
static int by_prob_desc(const void* a, const void* b) {
    const int32_t i = *(const int32_t*)a, j = *(const int32_t*)b;
    const float pi = g_sort_p[i], pj = g_sort_p[j];
    if (pi > pj) return -1;
    if (pi < pj) return 1;
    return i < j ? -1 : (i > j);
}

int32_t orc_sampler_sample(const float* lg, int64_t n, float temp, int32_t top_k, float top_p,
                           uint64_t* state) {
    if (temp <= 0.f) return orc_argmax(lg, n);
    float* probs = (float*)malloc((size_t)n * sizeof(float));
    int32_t* idx = (int32_t*)malloc((size_t)n * sizeof(int32_t));
    float mx = lg[0];
    for (int64_t i = 1; i < n; ++i) mx = lg[i] > mx ? lg[i] : mx;
    double sum = 0;
    for (int64_t i = 0; i < n; ++i) {
        probs[i] = expf((lg[i] - mx) / temp);
        sum += probs[i];
    }
    for (int64_t i = 0; i < n; ++i) probs[i] = (float)(probs[i] / sum);
    if (top_k > 0 && top_k < n) {
        for (int64_t i = 0; i < n; ++i) idx[i] = (int32_t)i;
        g_sort_p = probs;
        qsort(idx, (size_t)n, sizeof(int32_t), by_prob_desc);
        float keep = 0;
        for (int32_t i = 0; i < top_k; ++i) keep += probs[idx[i]];
        float* filt = (float*)calloc((size_t)n, sizeof(float));
        for (int32_t i = 0; i < top_k; ++i) filt[idx[i]] = probs[idx[i]] / keep;
        memcpy(probs, filt, (size_t)n * sizeof(float));
        free(filt);
    }
    if (top_p < 1.f) {
        for (int64_t i = 0; i < n; ++i) idx[i] = (int32_t)i;
        g_sort_p = probs;
        qsort(idx, (size_t)n, sizeof(int32_t), by_prob_desc);
        double cum = 0;
        int64_t cut = n;
        for (int64_t i = 0; i < n; ++i) {
            cum += probs[idx[i]];
            if (cum >= top_p) {
                cut = i + 1;
                break;
            }
        }
        double tail = 0;
        for (int64_t i = cut; i < n; ++i) {
            tail += probs[idx[i]];
            probs[idx[i]] = 0;
        }
        if (tail > 0 && cut > 0)
            for (int64_t i = 0; i < cut; ++i) probs[idx[i]] = (float)(probs[idx[i]] / (1.0 - tail));
    }
    const float r = sampler_next_float(state);
    double c = 0;
    int32_t pick = -1;
    for (int64_t i = 0; i < n; ++i) {
        c += probs[i];
        if ((float)c >= r) {
            pick = (int32_t)i;
            break;
        }
    }
    free(probs);
    free(idx);
    return pick >= 0 ? pick : orc_argmax(lg, n);
}

/* normalised target distribution p_T of a logits row, in double */
static void target_dist(const float* lg, int64_t V, float temp, double* p) {
    float mx = lg[0];
    for (int64_t i = 1; i < V; ++i) mx = fmaxf(mx, lg[i]);
    double sum = 0;
    for (int64_t i = 0; i < V; ++i) {
        p[i] = exp((double)((lg[i] - mx) / temp));
        sum += p[i];
    }
    for (int64_t i = 0; i < V; ++i) p[i] /= sum;
}

/*
 * Verify-step acceptance over a chain or a draft tree, plus the bonus token.
 * GREEDY: accept the first child whose token is argmax of the parent's row
 *   (src/spec.cpp:203-212 generalised to trees); bonus = argmax of the row
 *   after the last accepted node.
 * RATIO: src/spec.cpp:214-238 exactly (chain only); the bonus is drawn from
 *   p_T of the row after the last accepted node with one more uniform (the
 *   reference uses rows[min(acc,k-1)], spec.cpp:309-311, which is the wrong
 *   row whenever a draft token is rejected).
 * RESIDUAL: multi-candidate speculative sampling (Leviathan et al. 2023,
 *   Alg. 1; Miao et al. 2023, SpecInfer): at node c with target p, children
 *   are tried in index order; child s is accepted iff
 *   u <= min(1, p(t_s) / q_s(t_s)); after a rejection p <- norm(max(0, p -
 *   q_s)).  If no child is accepted, or c has no children, the bonus is drawn
 *   from the current p.  One uniform per child tried, one for the bonus.  For
 *   the first child the ratio is computed with the same float arithmetic as
 *   RATIO, so a one-child-per-level tree reproduces RATIO decisions.
 */
int orc_verify_accept(const float* base_row, const float* rows, int64_t M,
                      int64_t V, const int32_t* props, const int32_t* parents,
                      const float* pd, const float* q, int mode, float temp,
                      uint64_t* rng, uint64_t* sampler_state, int32_t top_k, float top_p,
                      int32_t* accepted, int32_t* n_acc, int32_t* bonus, float* margin) {
    if (M < 0 || V <= 0) return -1;
    for (int64_t i = 0; i < M; ++i) {
        int32_t pa = parents ? parents[i] : (int32_t)i - 1;
        if (pa < -1 || pa >= i) return -1;
        if (props[i] < 0 || props[i] >= V) return -1;
        if (mode == ORC_ACCEPT_RATIO && pa != (int32_t)i - 1) return -1;
    }
    if (mode == ORC_ACCEPT_RATIO && !pd) return -1;
    if (mode == ORC_ACCEPT_RESIDUAL && !q) return -1;
    float mg = INFINITY;
    int32_t cur = -1, na = 0;
#define ROW(c) ((c) < 0 ? base_row : rows + (int64_t)(c) * V)
#define PARENT(i) (parents ? parents[i] : (int32_t)(i) - 1)
    if (mode == ORC_ACCEPT_GREEDY) {
        for (;;) {
            int32_t g = orc_argmax(ROW(cur), V), next = -2;
            for (int64_t i = 0; i < M; ++i)
                if (PARENT(i) == cur && props[i] == g) { next = (int32_t)i; break; }
            if (next < -1) { *bonus = g; break; }
            accepted[na++] = next;
            cur = next;
        }
    } else if (mode == ORC_ACCEPT_RATIO) {
        /* the loop of orc_accept_chain_sampling, recording |u - ratio| */
        int a = 0;
        while (a < M) {
            const float* pred = ROW(a - 1);
            if (pd[a] <= 0.f) {
                if (orc_argmax(pred, V) != props[a]) break;
            } else {
                const float pt = orc_softmax_prob(pred, V, props[a], temp);
                const float ratio = fminf(1.f, pt / fmaxf(pd[a], 1e-9f));
                const float u = orc_rng_float(rng);
                if (fabsf(u - ratio) < mg) mg = fabsf(u - ratio);
                if (u > ratio) break;
            }
            ++a;
        }
        for (int i = 0; i < a; ++i) accepted[na++] = i;
        cur = a - 1;
        /* the bonus: Sampler::sample of the row after the last accepted node
         * (generate, src/spec.cpp:309-311, with the row fixed) */
        *bonus = orc_sampler_sample(ROW(cur), V, temp, top_k, top_p, sampler_state);
    } else if (mode == ORC_ACCEPT_RESIDUAL) {
        double* p = (double*)malloc((size_t)V * sizeof(double));
        for (;;) {
            const float* lg = ROW(cur);
            float mx = lg[0];
            for (int64_t i = 1; i < V; ++i) mx = fmaxf(mx, lg[i]);
            double sum = 0;
            for (int64_t i = 0; i < V; ++i) {
                p[i] = exp((double)((lg[i] - mx) / temp));
                sum += p[i];
            }
            for (int64_t i = 0; i < V; ++i) p[i] /= sum;
            int32_t next = -2;
            for (int64_t c = 0; c < M; ++c) {
                if (PARENT(c) != cur) continue;
                const float* qc = q + c * V;
                const int32_t t = props[c];
                const float pt = (float)p[t];
                const float ratio = fminf(1.f, pt / fmaxf(qc[t], 1e-9f));
                const float u = orc_rng_float(rng);
                if (fabsf(u - ratio) < mg) mg = fabsf(u - ratio);
                if (u <= ratio) { next = (int32_t)c; break; }
                double tot = 0;
                for (int64_t i = 0; i < V; ++i) {
                    double r = p[i] - (double)qc[i];
                    p[i] = r > 0 ? r : 0;
                    tot += p[i];
                }
                if (tot > 0)
                    for (int64_t i = 0; i < V; ++i) p[i] /= tot;
                else
                    target_dist(lg, V, temp, p); /* p == q: keep p */
            }
            if (next < -1) {
                *bonus = orc_sample_weights(p, V, orc_rng_float(rng));
                break;
            }
            accepted[na++] = next;
            cur = next;
        }
        free(p);
    } else {
        return -1;
    }
#undef ROW
#undef PARENT
    *n_acc = na;
    if (margin) *margin = mg;
    return 0;
}
