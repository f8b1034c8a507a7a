// k_sample.hip -- full-vocab row statistics and the acceptance sampler.
//
// Row statistics: first-max argmax (include/ft/sampler.h:21-28), float max,
// and sum_i exp((double)((l_i - max) / T)) in double (src/spec.cpp:89-95,
// 217-223), each computed over 4096-element chunks in parallel and combined
// in chunk order.  Acceptance: accept_chain_greedy / accept_chain_sampling
// (src/spec.cpp:203-238) with the SplitMix64 stream of src/spec.cpp:10-17,
// the bonus token drawn from the row after the last accepted node, and the
// tree / residual-resampling extensions (Leviathan et al. 2023 Alg. 1;
// SpecInfer, Miao et al. 2023).  Inverse-CDF sampling takes the first index
// whose running double sum of the normalised target exceeds u * total.
#include "ftx_internal.h"

namespace {

constexpr int NT = 1024;  // threads of the single-block acceptance kernels
constexpr int SCH = 4096; // elements per statistics chunk

__device__ __forceinline__ uint64_t splitmix_next(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float splitmix_float(uint64_t& s) {
    return (float)(splitmix_next(s) >> 40) * (1.f / 16777216.f);
}

__device__ __forceinline__ bool better(float b, int32_t ib, float a, int32_t ia) {
    return b > a || (b == a && ib < ia) || (a != a && b == b);
}

// ---- statistics pass 1: per (row, chunk) first-max argmax
__global__ void __launch_bounds__(256) k_row_max(const float* __restrict__ rows, int64_t V,
                                                 int nch, float* __restrict__ cmax,
                                                 int32_t* __restrict__ carg) {
    __shared__ float sv[256];
    __shared__ int32_t si[256];
    const int64_t r = blockIdx.y;
    const int c = blockIdx.x, t = threadIdx.x;
    const float* row = rows + r * V;
    const int64_t b = (int64_t)c * SCH, e = min(V, b + SCH);
    float best = -INFINITY;
    int32_t bi = 0x7FFFFFFF;
#pragma unroll 8
    for (int64_t i = b + t; i < e; i += 256) {
        const float v = row[i];
        if (bi == 0x7FFFFFFF || better(v, (int32_t)i, best, bi)) {
            best = v;
            bi = (int32_t)i;
        }
    }
    sv[t] = best;
    si[t] = bi;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (t < o && si[t + o] != 0x7FFFFFFF &&
            (si[t] == 0x7FFFFFFF || better(sv[t + o], si[t + o], sv[t], si[t]))) {
            sv[t] = sv[t + o];
            si[t] = si[t + o];
        }
        __syncthreads();
    }
    if (t == 0) {
        cmax[r * nch + c] = sv[0];
        carg[r * nch + c] = si[0];
    }
}

// ---- statistics pass 2: per (row, chunk) sum of exp((l - max)/T), the row
// max being the max of the chunk maxima
__global__ void __launch_bounds__(256) k_row_sum(const float* __restrict__ rows, int64_t V,
                                                 int nch, float temp,
                                                 const float* __restrict__ cmax,
                                                 double* __restrict__ csum) {
#pragma clang fp contract(off)
    __shared__ double sd[256];
    const int64_t r = blockIdx.y;
    const int c = blockIdx.x, t = threadIdx.x;
    float mx = -INFINITY;
#pragma unroll 8
    for (int k = 0; k < nch; ++k) mx = fmaxf(mx, cmax[r * nch + k]);
    const float* row = rows + r * V;
    const int64_t b = (int64_t)c * SCH, e = min(V, b + SCH);
    double s = 0.0;
#pragma unroll 8
    for (int64_t i = b + t; i < e; i += 256) s += exp((double)((row[i] - mx) / temp));
    sd[t] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (t < o) sd[t] += sd[t + o];
        __syncthreads();
    }
    if (t == 0) csum[r * nch + c] = sd[0];
}

// ---- statistics pass 3: combine chunks in order
__global__ void k_row_final(int nch, const float* __restrict__ cmax,
                            const int32_t* __restrict__ carg, const double* __restrict__ csum,
                            int with_sum, RowStats* __restrict__ out) {
    if (threadIdx.x != 0) return;
    const int64_t r = blockIdx.x;
    float best = cmax[r * nch];
    int32_t bi = carg[r * nch];
    for (int k = 1; k < nch; ++k)
        if (better(cmax[r * nch + k], carg[r * nch + k], best, bi)) {
            best = cmax[r * nch + k];
            bi = carg[r * nch + k];
        }
    double s = 0.0;
    if (with_sum)
        for (int k = 0; k < nch; ++k) s += csum[r * nch + k];
    out[r].mx = best;
    out[r].amax = bi;
    out[r].sum = s;
}

// ---- inverse-CDF pick over p[0..V) (double weights) by one block: chunk
// sums, a block scan, then the crossing chunk scanned in order.  Falls back
// to the last positive weight when rounding leaves no crossing.
// Inverse-CDF pick over V probabilities: thread t owns the contiguous chunk
// [t * chunk, (t + 1) * chunk) and sums it in index order.  `tr` selects the
// chunk-transposed layout p[k * NT + t] = prob(t * chunk + k), whose loads
// are coalesced across threads; the arithmetic is the same in both layouts.
__device__ int32_t block_pick(const double* __restrict__ p, int64_t V, float u, bool tr) {
    __shared__ double incl[NT];
    __shared__ int32_t lastpos[NT];
    __shared__ int32_t pick;
    const int t = threadIdx.x;
    const int64_t chunk = (V + NT - 1) / NT;
    const int64_t b = t * chunk, e = min(V, b + chunk);
    // sums in index order; the loads of eight elements are issued together
    double cs = 0.0;
    int32_t lp = -1;
    auto at = [&](int64_t i) { return tr ? p[(i - b) * NT + t] : p[i]; };
    for (int64_t i0 = b; i0 < e; i0 += 8) {
        double v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = i0 + k < e ? at(i0 + k) : 0.0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (i0 + k >= e) break;
            cs += v[k];
            if (v[k] > 0) lp = (int32_t)(i0 + k);
        }
    }
    incl[t] = cs;
    lastpos[t] = lp;
    if (t == 0) pick = -1;
    __syncthreads();
    for (int o = 1; o < NT; o <<= 1) {
        const double add = t >= o ? incl[t - o] : 0.0;
        const int32_t lpo = t >= o ? lastpos[t - o] : -1;
        __syncthreads();
        incl[t] += add;
        if (lastpos[t] < 0) lastpos[t] = lpo;
        __syncthreads();
    }
    const double tot = incl[NT - 1];
    const double target = (double)u * tot;
    const double ex = t ? incl[t - 1] : 0.0;
    if (incl[t] > target && ex <= target && b < e) {
        double c = ex;
        bool found = false;
        for (int64_t i0 = b; i0 < e && !found; i0 += 8) {
            double v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = i0 + k < e ? at(i0 + k) : 0.0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (found || i0 + k >= e) break;
                c += v[k];
                if (c > target) {
                    pick = (int32_t)(i0 + k);
                    found = true;
                }
            }
        }
    }
    __syncthreads();
    int32_t r = pick;
    if (r < 0) r = lastpos[NT - 1] >= 0 ? lastpos[NT - 1] : 0;
    __syncthreads();
    return r;
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

// Decisions.  GREEDY and RESIDUAL finish here; RATIO records the row the
// bonus is drawn from and its uniform for the two bonus kernels.
__global__ void __launch_bounds__(NT) k_accept(AcceptDev a) {
#pragma clang fp contract(off)
    __shared__ double sd[NT];
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
            *a.bu = splitmix_float(s);  // the bonus token's uniform
            *a.brow = k - 1;
            rng = s;
            mg = m;
        }
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
                const int32_t b = block_pick(a.p, V, ub2, false);
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

// RATIO bonus, step 1: the normalised target of the recorded row, in
// parallel, stored chunk-transposed for the pick (see block_pick)
__global__ void __launch_bounds__(256) k_bonus_dist(AcceptDev a) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.V) return;
    const int32_t c = *a.brow;
    const float* lg = c < 0 ? a.base_row : a.rows + (int64_t)c * a.V;
    const RowStats st = a.stats[c + 1];
    const int64_t chunk = (a.V + NT - 1) / NT;
    a.p[(i % chunk) * NT + i / chunk] = exp((double)((lg[i] - st.mx) / a.temp)) / st.sum;
}

// RATIO bonus, step 2: the inverse-CDF pick
__global__ void __launch_bounds__(NT) k_bonus_pick(AcceptDev a) {
    const int32_t b = block_pick(a.p, a.V, *a.bu, true);
    if (threadIdx.x == 0) a.out[1] = b;
}

}  // namespace

size_t row_stats_scratch_bytes(int64_t nrows, int64_t V) {
    const int64_t nch = (V + SCH - 1) / SCH;
    return (size_t)(nrows * nch) * (4 + 4 + 8) + 64;
}

hipError_t launch_row_stats(hipStream_t st, const float* rows, int64_t nrows, int64_t V,
                            float temp, int with_sum, void* scratch, RowStats* out) {
    if (nrows == 0) return hipSuccess;
    const int nch = (int)((V + SCH - 1) / SCH);
    double* csum = (double*)scratch;
    float* cmax = (float*)(csum + nrows * nch);
    int32_t* carg = (int32_t*)(cmax + nrows * nch);
    hipLaunchKernelGGL(k_row_max, dim3((unsigned)nch, (unsigned)nrows), dim3(256), 0, st, rows, V,
                       nch, cmax, carg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (with_sum) {
        hipLaunchKernelGGL(k_row_sum, dim3((unsigned)nch, (unsigned)nrows), dim3(256), 0, st, rows,
                           V, nch, temp, cmax, csum);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_row_final, dim3((unsigned)nrows), dim3(64), 0, st, nch, cmax, carg, csum,
                       with_sum, out);
    return hipGetLastError();
}

hipError_t launch_accept(hipStream_t st, const AcceptDev& a) {
    hipLaunchKernelGGL(k_accept, dim3(1), dim3(NT), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.mode != FTX_ACCEPT_RATIO) return e;
    hipLaunchKernelGGL(k_bonus_dist, dim3((unsigned)((a.V + 255) / 256)), dim3(256), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_bonus_pick, dim3(1), dim3(NT), 0, st, a);
    return hipGetLastError();
}
