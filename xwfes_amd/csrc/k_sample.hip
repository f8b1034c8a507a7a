// k_sample.hip -- full-vocab row statistics and the acceptance sampler.
//
// Row statistics: first-max argmax (include/ft/sampler.h:21-28), float max,
// and sum_i exp((double)((l_i - max) / T)) in double (src/spec.cpp:89-95,
// 217-223).  Two launches cover the base row and every draft row: per
// 4096-element chunk the first-max argmax, then per 128-element sub-chunk
// the double sum of the exponentials with the row max.  The acceptance
// kernel combines them: accept_chain_greedy / accept_chain_sampling
// (src/spec.cpp:203-238) with the SplitMix64 stream of src/spec.cpp:10-17,
// the bonus token drawn from the row after the last accepted node, and the
// tree / residual-resampling extensions (Leviathan et al. 2023 Alg. 1;
// SpecInfer, Miao et al. 2023).  Inverse-CDF sampling takes the first index
// whose running double sum of the target exceeds u * total; the ratio-mode
// bonus finds the crossing 128-element sub-chunk by a scan of the sub-chunk
// sums and sums only that sub-chunk element by element.
#include "ftx_internal.h"

namespace {

constexpr int NT = 1024;  // threads of the single-block acceptance kernel
constexpr int SCH = 4096; // elements per statistics chunk
constexpr int SUB = 128;  // elements per exp-sum sub-chunk (SCH / SUB per chunk)

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

__device__ __forceinline__ const float* stat_row(const float* base_row, const float* rows,
                                                 int64_t r, int64_t V) {
    return r == 0 ? base_row : rows + (r - 1) * V;
}

// exp((double)((l - mx) / T)): the one expression every sum and pick uses
__device__ __forceinline__ double texp(float l, float mx, float temp) {
#pragma clang fp contract(off)
    return exp((double)((l - mx) / temp));
}

// ---- statistics pass 1: per (row, chunk) first-max argmax; the 16 loads
// of a thread are issued together (clamped index, masked)
__global__ void __launch_bounds__(256) k_row_max(const float* __restrict__ base_row,
                                                 const float* __restrict__ rows, int64_t V,
                                                 RowChunks rc) {
    __shared__ float sv[256];
    __shared__ int32_t si[256];
    const int64_t r = blockIdx.y;
    const int c = blockIdx.x, t = threadIdx.x;
    const float* row = stat_row(base_row, rows, r, V);
    const int64_t b = (int64_t)c * SCH;
    float v[SCH / 256];
#pragma unroll
    for (int k = 0; k < SCH / 256; ++k) v[k] = row[min(b + t + 256 * k, V - 1)];
    float best = -INFINITY;
    int32_t bi = 0x7FFFFFFF;
#pragma unroll
    for (int k = 0; k < SCH / 256; ++k) {
        const int64_t i = b + t + 256 * k;
        if (i < V && (bi == 0x7FFFFFFF || better(v[k], (int32_t)i, best, bi))) {
            best = v[k];
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
        rc.cmax[r * rc.nch + c] = sv[0];
        rc.carg[r * rc.nch + c] = si[0];
    }
}

// ---- statistics pass 2: per (row, 128-element sub-chunk) sum of
// exp((l - max)/T), the row max being the max of the chunk maxima.  Thread
// t takes elements 16t .. 16t + 15 of the chunk (vector loads when rows are
// 16-byte aligned), eight threads one sub-chunk: sums in index order per
// thread, then over the eight threads in a fixed tree.
template <bool VEC>
__global__ void __launch_bounds__(256) k_row_sum(const float* __restrict__ base_row,
                                                 const float* __restrict__ rows, int64_t V,
                                                 float temp, RowChunks rc) {
#pragma clang fp contract(off)
    const int64_t r = blockIdx.y;
    const int c = blockIdx.x, t = threadIdx.x;
    const float* row = stat_row(base_row, rows, r, V);
    const int64_t i0 = (int64_t)c * SCH + 16 * t;
    float v[16];
    if (VEC && i0 + 16 <= V) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 q = *(const float4*)(row + i0 + 4 * k);
            v[4 * k] = q.x;
            v[4 * k + 1] = q.y;
            v[4 * k + 2] = q.z;
            v[4 * k + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = row[min(i0 + k, V - 1)];
    }
    float mx = -INFINITY;
    for (int k = 0; k < rc.nch; ++k) mx = fmaxf(mx, rc.cmax[r * rc.nch + k]);
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < 16; ++k)
        if (i0 + k < V) s += texp(v[k], mx, temp);
    s += __shfl_xor(s, 4, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 1, 64);
    const int64_t j = (int64_t)c * (SCH / SUB) + t / 8;
    if ((t & 7) == 0 && j < rc.nsub) rc.csub[r * rc.nsub + j] = s;
}

// Inverse-CDF pick over p[0..V) (double weights) by one block: thread t sums
// the contiguous chunk [t * chunk, (t + 1) * chunk) in index order (eight
// loads issued together), a block scan, then the crossing chunk scanned in
// order.  Falls back to the last positive weight when rounding leaves no
// crossing.
__device__ int32_t block_pick(const double* __restrict__ p, int64_t V, float u) {
    __shared__ double incl[NT];
    __shared__ int32_t lastpos[NT];
    __shared__ int32_t pick;
    const int t = threadIdx.x;
    const int64_t chunk = (V + NT - 1) / NT;
    const int64_t b = t * chunk, e = min(V, b + chunk);
    double cs = 0.0;
    int32_t lp = -1;
    for (int64_t i0 = b; i0 < e; i0 += 8) {
        double v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = i0 + k < e ? p[i0 + k] : 0.0;
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
            for (int k = 0; k < 8; ++k) v[k] = i0 + k < e ? p[i0 + k] : 0.0;
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

// Inclusive block scan of one double per thread (wave scans, then the wave
// totals); returns the thread's inclusive prefix, *tot the block total.
__device__ double block_scan(double v, double* tot) {
    __shared__ double wsum[NT / 64];
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double n = __shfl_up(v, o, 64);
        if (l >= o) v += n;
    }
    if (l == 63) wsum[w] = v;
    __syncthreads();
    if (w == 0) {
        double x = l < NT / 64 ? wsum[l] : 0.0;
#pragma unroll
        for (int o = 1; o < NT / 64; o <<= 1) {
            const double n = __shfl_up(x, o, 64);
            if (l >= o) x += n;
        }
        if (l < NT / 64) wsum[l] = x;
    }
    __syncthreads();
    const double r = v + (w ? wsum[w - 1] : 0.0);
    *tot = wsum[NT / 64 - 1];
    __syncthreads();
    return r;
}

// Ratio-mode bonus: inverse CDF over exp((l - mx)/T) of row `lg` from its
// sub-chunk sums `sub` (nsub of them): thread t owns sub-chunks [t spt, (t +
// 1) spt); the crossing thread finds the crossing sub-chunk, whose 128
// exponentials are formed again by one wave and summed in index order by its
// first lane.  Rounding that leaves no crossing inside the sub-chunk picks
// its last positive element.
__device__ int32_t pick_from_subs(const float* __restrict__ lg, int64_t V, float mx, float temp,
                                  const double* __restrict__ sub, int nsub, float u) {
#pragma clang fp contract(off)
    __shared__ int jsel, first;
    __shared__ double exsel;
    __shared__ double ev[SUB];
    __shared__ double incl[NT];
    __shared__ int32_t pick;
    const int t = threadIdx.x;
    const int spt = (nsub + NT - 1) / NT;
    const int j0 = t * spt, j1 = min(nsub, j0 + spt);
    double cs = 0.0;
    for (int j = j0; j < j1; ++j) cs += sub[j];
    if (t == 0) {
        jsel = -1;
        pick = -1;
        first = NT;
    }
    double tot;
    const double inc = block_scan(cs, &tot);
    incl[t] = inc;
    const double target = (double)u * tot;
    if (inc > target) atomicMin(&first, t);
    __syncthreads();
    if (t == first) {
        // the first thread whose inclusive prefix passes the target: its
        // sub-chunks in order from the previous thread's prefix
        double c = t ? incl[t - 1] : 0.0;
        int js = -1;
        double es = c;
        for (int j = j0; j < j1; ++j) {
            const double nc = c + sub[j];
            if (sub[j] > 0) {
                js = j;
                es = c;
            }
            if (nc > target) break;
            c = nc;
        }
        jsel = js;
        exsel = es;
    }
    __syncthreads();
    const int js = jsel;
    if (t < 64 && js >= 0) {
#pragma unroll
        for (int k = 0; k < SUB / 64; ++k) {
            const int64_t i = (int64_t)js * SUB + t + 64 * k;
            ev[t + 64 * k] = i < V ? texp(lg[i], mx, temp) : 0.0;
        }
    }
    __syncthreads();
    if (t == 0 && js >= 0) {
        double c = exsel;
        int32_t last = -1, pk = -1;
        for (int k = 0; k < SUB; ++k) {
            if (ev[k] > 0) last = js * SUB + k;
            c += ev[k];
            if (c > target) {
                pk = js * SUB + k;
                break;
            }
        }
        pick = pk >= 0 ? pk : last;
    }
    __syncthreads();
    const int32_t r = pick >= 0 ? pick : 0;
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
    __shared__ float mg, bu;
    const int t = threadIdx.x;
    const int64_t V = a.V;
    if (t == 0) {
        rng = *a.rng;
        cur = -1;
        nacc = 0;
        bonus = 0;
        mg = INFINITY;
    }
    // row statistics from the chunk results, one wave per row: first-max
    // argmax over the chunks, the exp sum over the sub-chunks (lane-strided
    // sums in index order, then a fixed tree)
    {
        const int w = t >> 6, l = t & 63;
        const RowChunks& rc = a.rc;
        for (int64_t r = w; r <= a.M; r += NT / 64) {
            float best = -INFINITY;
            int32_t bi = 0x7FFFFFFF;
            for (int c = l; c < rc.nch; c += 64) {
                const float v = rc.cmax[r * rc.nch + c];
                const int32_t iv = rc.carg[r * rc.nch + c];
                if (iv != 0x7FFFFFFF && (bi == 0x7FFFFFFF || better(v, iv, best, bi))) {
                    best = v;
                    bi = iv;
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(best, o, 64);
                const int32_t oi = __shfl_xor(bi, o, 64);
                if (oi != 0x7FFFFFFF && (bi == 0x7FFFFFFF || better(ov, oi, best, bi))) {
                    best = ov;
                    bi = oi;
                }
            }
            double sum = 0.0;
            if (a.with_sum) {
                for (int j = l; j < rc.nsub; j += 64) sum += rc.csub[r * rc.nsub + j];
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
            }
            if (l == 0) a.stats[r] = RowStats{best, bi, sum};
        }
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
            bu = splitmix_float(s);  // the bonus token's uniform
            rng = s;
            mg = m;
        }
        __syncthreads();
        // the bonus from the row after the last accepted node
        const int32_t c = cur;
        const int32_t b = pick_from_subs(ROW(c), V, STAT(c).mx, a.temp,
                                         a.rc.csub + (int64_t)(c + 1) * a.rc.nsub, a.rc.nsub, bu);
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
                const int32_t b = block_pick(a.p, V, ub2);
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

size_t row_stats_scratch_bytes(int64_t nrows, int64_t V) {
    const int64_t nch = (V + SCH - 1) / SCH, nsub = (V + SUB - 1) / SUB;
    return (size_t)(nrows * nsub) * 8 + (size_t)(nrows * nch) * 8 + 64;
}

RowChunks row_chunks(void* scratch, int64_t nrows, int64_t V) {
    RowChunks rc{};
    rc.nch = (int)((V + SCH - 1) / SCH);
    rc.nsub = (int)((V + SUB - 1) / SUB);
    rc.csub = (double*)scratch;
    rc.cmax = (float*)(rc.csub + nrows * rc.nsub);
    rc.carg = (int32_t*)(rc.cmax + nrows * rc.nch);
    return rc;
}

hipError_t launch_row_stats(hipStream_t st, const float* base_row, const float* rows,
                            int64_t nrows, int64_t V, float temp, int with_sum,
                            const RowChunks& rc) {
    if (nrows == 0) return hipSuccess;
    const dim3 grid((unsigned)rc.nch, (unsigned)nrows);
    hipLaunchKernelGGL(k_row_max, grid, dim3(256), 0, st, base_row, rows, V, rc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !with_sum) return e;
    const bool vec = V % 4 == 0 && ((uintptr_t)base_row % 16) == 0 &&
                     (nrows == 1 || ((uintptr_t)rows % 16) == 0);
    if (vec)
        hipLaunchKernelGGL(k_row_sum<true>, grid, dim3(256), 0, st, base_row, rows, V, temp, rc);
    else
        hipLaunchKernelGGL(k_row_sum<false>, grid, dim3(256), 0, st, base_row, rows, V, temp, rc);
    return hipGetLastError();
}

hipError_t launch_accept(hipStream_t st, const AcceptDev& a) {
    hipLaunchKernelGGL(k_accept, dim3(1), dim3(NT), 0, st, a);
    return hipGetLastError();
}
