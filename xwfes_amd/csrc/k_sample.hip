// k_sample.hip -- full-vocab row statistics and the acceptance sampler.
//
// Row statistics: first-max argmax (include/ft/sampler.h:21-28), float max,
// and sum_i exp((double)((l_i - max) / T)) in double (src/spec.cpp:89-95,
// 217-223).  Acceptance: accept_chain_greedy / accept_chain_sampling
// (src/spec.cpp:203-238) with the SplitMix64 stream of src/spec.cpp:10-17,
// the bonus token drawn from the row after the last accepted node, and the
// tree / residual-resampling extensions (Leviathan et al. 2023 Alg. 1;
// SpecInfer, Miao et al. 2023).
#include "ftx_internal.h"

namespace {

constexpr int NT = 1024;  // threads of the statistics and acceptance blocks

__device__ __forceinline__ uint64_t splitmix_next(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float splitmix_float(uint64_t& s) {
    return (float)(splitmix_next(s) >> 40) * (1.f / 16777216.f);
}

// block-wide argmax with first-index tie break; all threads get the result
__device__ void block_argmax(float& v, int32_t& i, float* sv, int32_t* si) {
    const int t = threadIdx.x;
    sv[t] = v;
    si[t] = i;
    __syncthreads();
    for (int o = NT / 2; o > 0; o >>= 1) {
        if (t < o) {
            const float a = sv[t], b = sv[t + o];
            const int32_t ia = si[t], ib = si[t + o];
            if (b > a || (b == a && ib < ia) || (a != a && b == b)) {
                sv[t] = b;
                si[t] = ib;
            }
        }
        __syncthreads();
    }
    v = sv[0];
    i = si[0];
    __syncthreads();
}

__device__ double block_sum(double v, double* sd) {
    const int t = threadIdx.x;
    sd[t] = v;
    __syncthreads();
    for (int o = NT / 2; o > 0; o >>= 1) {
        if (t < o) sd[t] += sd[t + o];
        __syncthreads();
    }
    const double r = sd[0];
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(NT) k_row_stats(const float* __restrict__ rows, int64_t V,
                                                  float temp, RowStats* __restrict__ out) {
#pragma clang fp contract(off)
    __shared__ float sv[NT];
    __shared__ int32_t si[NT];
    __shared__ double sd[NT];
    const float* r = rows + (int64_t)blockIdx.x * V;
    float best = -INFINITY;
    int32_t bi = 0x7FFFFFFF;
    for (int64_t i = threadIdx.x; i < V; i += NT) {
        const float v = r[i];
        if (v > best || bi == 0x7FFFFFFF) {
            best = v;
            bi = (int32_t)i;
        }
    }
    block_argmax(best, bi, sv, si);
    const float mx = best;
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < V; i += NT) s += exp((double)((r[i] - mx) / temp));
    s = block_sum(s, sd);
    if (threadIdx.x == 0) {
        out[blockIdx.x].mx = mx;
        out[blockIdx.x].amax = bi;
        out[blockIdx.x].sum = s;
    }
}

// ---- inverse-CDF sampling over p[0..V) (double weights) ----
// first i whose running sum exceeds u * sum(p); if rounding leaves none,
// the last positive weight (the restatement's sample_weights)
__device__ int32_t block_sample(const double* __restrict__ p, int64_t V, float u, double* sd,
                                int32_t* si) {
    const int t = threadIdx.x;
    const int64_t chunk = (V + NT - 1) / NT;
    const int64_t b = t * chunk, e = min(V, b + chunk);
    double cs = 0.0;
    int32_t lastpos = -1;
    for (int64_t i = b; i < e; ++i) {
        cs += p[i];
        if (p[i] > 0) lastpos = (int32_t)i;
    }
    // inclusive scan of chunk sums (sequential on thread 0: fixed order)
    sd[t] = cs;
    si[t] = lastpos;
    __syncthreads();
    __shared__ int32_t pick;
    if (t == 0) {
        double tot = 0.0;
        int32_t lp = 0;
        for (int k = 0; k < NT; ++k) {
            const double c = sd[k];
            sd[k] = tot;  // exclusive prefix
            tot += c;
            if (si[k] >= 0) lp = si[k];
        }
        const double target = (double)u * tot;
        int32_t res = lp;
        double c = 0.0;
        for (int k = 0; k < NT; ++k) {
            const int64_t kb = k * chunk, ke = min(V, kb + chunk);
            c = sd[k];
            const double cend = (k + 1 < NT) ? sd[k + 1] : tot;
            if (cend > target && kb < ke) {
                bool found = false;
                for (int64_t i = kb; i < ke; ++i) {
                    c += p[i];
                    if (c > target) {
                        res = (int32_t)i;
                        found = true;
                        break;
                    }
                }
                if (found) break;
            }
        }
        pick = res;
    }
    __syncthreads();
    const int32_t r = pick;
    __syncthreads();
    return r;
}

// p[i] = exp((double)((l_i - mx)/T)) / sum, the target distribution
__device__ void target_dist(const float* __restrict__ lg, int64_t V, float temp, float mx,
                            double* p, double* sd) {
#pragma clang fp contract(off)
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < V; i += NT) {
        const double e = exp((double)((lg[i] - mx) / temp));
        p[i] = e;
        s += e;
    }
    s = block_sum(s, sd);
    for (int64_t i = threadIdx.x; i < V; i += NT) p[i] /= s;
    __syncthreads();
}

__global__ void __launch_bounds__(NT) k_accept(AcceptDev a) {
#pragma clang fp contract(off)
    __shared__ double sd[NT];
    __shared__ int32_t si[NT];
    __shared__ uint64_t rng;
    __shared__ int32_t cur, nacc, bonus, next;
    __shared__ float mg;
    const int t = threadIdx.x;
    const int64_t V = a.V;
    if (t == 0) {
        rng = *a.rng;
        cur = -1;
        nacc = 0;
        bonus = 0;
        mg = INFINITY;
    }
    __syncthreads();
#define ROW(c) ((c) < 0 ? a.base_row : a.rows + (int64_t)(c) * V)
#define STAT(c) a.stats[(c) + 1]
    if (a.mode == FTX_ACCEPT_GREEDY) {
        if (t == 0) {
            for (;;) {
                const int32_t g = STAT(cur).amax;
                int32_t nx = -2;
                for (int64_t i = 0; i < a.M; ++i)
                    if (a.parents[i] == cur && a.props[i] == g) {
                        nx = (int32_t)i;
                        break;
                    }
                if (nx < -1) {
                    bonus = g;
                    break;
                }
                a.out[2 + nacc++] = nx;
                cur = nx;
            }
        }
        __syncthreads();
    } else if (a.mode == FTX_ACCEPT_RATIO) {
        if (t == 0) {
            uint64_t s = rng;
            int32_t k = 0;
            float m = INFINITY;
            while (k < a.M) {
                const RowStats st = STAT(k - 1);
                const float* lg = ROW(k - 1);
                const float pdk = a.pd[k];
                if (pdk <= 0.f) {
                    if (st.amax != a.props[k]) break;
                } else {
                    const float z = (lg[a.props[k]] - st.mx) / a.temp;
                    const float pt = (float)(exp((double)z) / st.sum);
                    const float ratio = fminf(1.f, pt / fmaxf(pdk, 1e-9f));
                    const float u = splitmix_float(s);
                    m = fminf(m, fabsf(u - ratio));
                    if (u > ratio) break;
                }
                ++k;
            }
            for (int32_t i = 0; i < k; ++i) a.out[2 + i] = i;
            nacc = k;
            cur = k - 1;
            rng = s;
            mg = m;
        }
        __syncthreads();
        const int32_t c = cur;
        target_dist(ROW(c), V, a.temp, STAT(c).mx, a.p, sd);
        __shared__ float ub;
        if (t == 0) {
            uint64_t s = rng;
            ub = splitmix_float(s);
            rng = s;
        }
        __syncthreads();
        const int32_t b = block_sample(a.p, V, ub, sd, si);
        if (t == 0) bonus = b;
        __syncthreads();
    } else {  // RESIDUAL
        for (;;) {
            const int32_t c = cur;
            target_dist(ROW(c), V, a.temp, STAT(c).mx, a.p, sd);
            if (t == 0) next = -2;
            __syncthreads();
            for (int64_t ch = 0; ch < a.M; ++ch) {
                if (a.parents[ch] != c) continue;
                __shared__ int32_t acc_flag;
                if (t == 0) {
                    const float* qc = a.q + ch * V;
                    const int32_t tok = a.props[ch];
                    const float pt = (float)a.p[tok];
                    const float ratio = fminf(1.f, pt / fmaxf(qc[tok], 1e-9f));
                    uint64_t s = rng;
                    const float u = splitmix_float(s);
                    rng = s;
                    mg = fminf(mg, fabsf(u - ratio));
                    acc_flag = u <= ratio;
                    if (acc_flag) next = (int32_t)ch;
                }
                __syncthreads();
                if (acc_flag) break;
                // p <- norm(max(0, p - q_ch))
                const float* qc = a.q + ch * V;
                double s = 0.0;
                for (int64_t i = t; i < V; i += NT) {
                    const double r = a.p[i] - (double)qc[i];
                    const double v = r > 0 ? r : 0;
                    a.p[i] = v;
                    s += v;
                }
                s = block_sum(s, sd);
                if (s > 0) {
                    for (int64_t i = t; i < V; i += NT) a.p[i] /= s;
                    __syncthreads();
                } else {
                    target_dist(ROW(c), V, a.temp, STAT(c).mx, a.p, sd);
                }
            }
            __syncthreads();
            if (next < -1) {
                __shared__ float ub2;
                if (t == 0) {
                    uint64_t s = rng;
                    ub2 = splitmix_float(s);
                    rng = s;
                }
                __syncthreads();
                const int32_t b = block_sample(a.p, V, ub2, sd, si);
                if (t == 0) bonus = b;
                __syncthreads();
                break;
            }
            if (t == 0) {
                a.out[2 + nacc++] = next;
                cur = next;
            }
            __syncthreads();
        }
    }
#undef ROW
#undef STAT
    if (t == 0) {
        a.out[0] = nacc;
        a.out[1] = bonus;
        *a.rng = rng;
        *a.margin = mg;
    }
}

}  // namespace

hipError_t launch_row_stats(hipStream_t st, const float* rows, int64_t nrows, int64_t V,
                            float temp, RowStats* out) {
    if (nrows == 0) return hipSuccess;
    hipLaunchKernelGGL(k_row_stats, dim3((unsigned)nrows), dim3(NT), 0, st, rows, V, temp, out);
    return hipGetLastError();
}

hipError_t launch_accept(hipStream_t st, const AcceptDev& a) {
    hipLaunchKernelGGL(k_accept, dim3(1), dim3(NT), 0, st, a);
    return hipGetLastError();
}
