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

#include <climits>

namespace {

constexpr int NT = 1024;  // threads of the single-block acceptance kernel
constexpr int ACC_RES_WG = 32;  // workgroups of the residual acceptance kernel (<= 64)
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

// exp((double)((l - mx) / T)): the acceptance test's exponential
__device__ __forceinline__ double texp(float l, float mx, float temp) {
#pragma clang fp contract(off)
    return exp((double)((l - mx) / temp));
}

// expf((l - mx) / T) in float: the sampler's exponential (sampler.h:40)
__device__ __forceinline__ float sexp(float l, float mx, float temp) {
#pragma clang fp contract(off)
    return expf((l - mx) / temp);
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
    double s = 0.0, sf = 0.0;
    float smx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 16; ++k)
        if (i0 + k < V) {
            s += texp(v[k], mx, temp);
            sf += (double)sexp(v[k], mx, temp);
            smx = fmaxf(smx, v[k]);
        }
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) {
        s += __shfl_xor(s, o, 64);
        sf += __shfl_xor(sf, o, 64);
        smx = fmaxf(smx, __shfl_xor(smx, o, 64));
    }
    const int64_t j = (int64_t)c * (SCH / SUB) + t / 8;
    if ((t & 7) == 0 && j < rc.nsub) {
        rc.csub[r * rc.nsub + j] = s;
        rc.csubf[r * rc.nsub + j] = sf;
        rc.submax[r * rc.nsub + j] = smx;
    }
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

constexpr int SMAXK = 64;     // largest top-k of the device sampler
constexpr int SMAXSUB = 4096; // largest sub-chunk count it takes (V <= 524288)
constexpr int SMAXEQ = 1024;  // probabilities equal to the k-th kept for the tie break

// The sampler's SplitMix64 draw: bits 24..47 of the output as a 24-bit
// fraction (include/ft/sampler.h:84-92)
__device__ __forceinline__ float sampler_next_float(uint64_t& st) {
    st += 0x9E3779B97F4A7C15ull;
    uint64_t z = st;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    const uint32_t u = (uint32_t)((z ^ (z >> 31)) >> 16);
    return (float)(u >> 8) * (1.f / 16777216.f);
}

// order-preserving unsigned key of a float
__device__ __forceinline__ uint32_t fkey(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Block-wide radix select: the `need`-th largest key among n entries (key_of
// (e, &k) returns false for an entry without a value), 8 bits a pass;
// returns the key and *take: how many entries equal to it are among the
// `need` largest.  Wave 0 finds each pass's bin by a suffix scan over the
// 256 bins (four per lane).
template <typename KeyOf>
__device__ uint32_t block_radix_kth(int n, uint32_t need, KeyOf key_of, uint32_t* take) {
    // one histogram per wave, rows 257 words apart so that the waves' copies
    // of a bin sit in different banks; summed into row 0 before the scan
    constexpr int HS = 257;
    __shared__ uint32_t whist[NT / 64][HS];
    __shared__ uint32_t s_pre, s_msk, s_need;
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    uint32_t* hist = whist[0];
    if (t == 0) {
        s_pre = 0;
        s_msk = 0;
        s_need = need;
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = t; i < (NT / 64) * HS; i += NT) (&whist[0][0])[i] = 0;
        __syncthreads();
        const uint32_t pre = s_pre, msk = s_msk;
        for (int e = t; e < n; e += NT) {
            uint32_t k;
            if (key_of(e, &k) && (k & msk) == pre) atomicAdd(&whist[w][(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (t < 256) {
            uint32_t v = 0;
#pragma unroll
            for (int q = 0; q < NT / 64; ++q) v += whist[q][t];
            hist[t] = v;  // row 0 is read only by thread t before this write
        }
        __syncthreads();
        if (t < 64) {
            const uint32_t h0 = hist[4 * l], h1 = hist[4 * l + 1], h2 = hist[4 * l + 2],
                           h3 = hist[4 * l + 3];
            const uint32_t loc = h0 + h1 + h2 + h3;
            uint32_t inc = loc;  // sum over this lane and the lanes above it
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t v = __shfl_down(inc, o, 64);
                if (l + o < 64) inc += v;
            }
            const uint32_t nd = s_need;
            uint32_t cum = inc - loc;  // entries in higher bins
            const uint32_t hb[4] = {h0, h1, h2, h3};
#pragma unroll
            for (int q = 3; q >= 0; --q) {
                if (cum < nd && cum + hb[q] >= nd) {
                    s_pre = pre | ((uint32_t)(4 * l + q) << shift);
                    s_msk = msk | (255u << shift);
                    s_need = nd - cum;
                }
                cum += hb[q];
            }
        }
        __syncthreads();
    }
    const uint32_t r = s_pre;
    *take = s_need;
    __syncthreads();
    return r;
}

// Sampler::sample (include/ft/sampler.h:30-94) of row lg (max mx, double sum
// S of the float exponentials) at temperature T > 0: top-k (1 <= K <= 64, K <
// V) or, without it, all V <= 64 elements; top-p (< 1) or none; one draw from
// *state.  The K largest probabilities lie in the K sub-chunks of largest
// maxima (the probability is monotone in the logit), so those K * 128
// elements are the candidates; radix selects find the K-th largest sub-chunk
// maximum and then the K-th largest candidate probability, ties at either
// going to the lower index (the reference's partial_sort leaves their order
// unspecified).  The kept values then go through the reference's arithmetic
// in order.
__device__ int32_t sampler_pick(const float* __restrict__ lg, int64_t V, float mx, float temp,
                                int topk, float top_p, const double* __restrict__ csubf,
                                const float* __restrict__ submax, int nsub, int32_t amax,
                                uint64_t* state) {
#pragma clang fp contract(off)
    __shared__ float cp[SMAXK * SUB];  // candidate probabilities (-1: no element)
    __shared__ float smx[SMAXSUB];
    __shared__ int32_t sel[SMAXK];
    __shared__ uint32_t nsel_gt, neq;
    __shared__ int32_t eqi[SMAXEQ];
    __shared__ float kp[SMAXK];
    __shared__ int32_t ki[SMAXK];
    __shared__ int32_t kx[SMAXK];
    __shared__ double ssum;
    __shared__ int32_t pick;
    const int t = threadIdx.x, l = t & 63;
    const bool use_k = topk > 0 && topk < V;
    const int K = use_k ? topk : (int)V;
    const int nsel = use_k ? min(K, nsub) : nsub;
    // the normaliser and the sub-chunk maxima
    if (t < 64) {
        double sv = 0.0;
        // lane-strided in index order, 16 loads in flight per lane
        for (int j0 = t; j0 < nsub; j0 += 64 * 16) {
            double v[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = csubf[min(j0 + 64 * k, nsub - 1)];
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (j0 + 64 * k < nsub) sv += v[k];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) sv += __shfl_xor(sv, o, 64);
        if (t == 0) {
            ssum = sv;
            nsel_gt = 0;
            neq = 0;
            pick = -1;
        }
    }
    for (int j = t; j < nsub; j += NT) smx[j] = submax[j];
    __syncthreads();
    // the nsel sub-chunks of largest maxima (ties: lower index)
    float thr = -INFINITY;  // the top K all lie at or above the K-th largest maximum
    if (use_k && nsel < nsub) {
        uint32_t take;
        const uint32_t kk = block_radix_kth(nsub, (uint32_t)nsel,
                                            [&](int e, uint32_t* k) {
                                                *k = fkey(smx[e]);
                                                return true;
                                            },
                                            &take);
        for (int j = t; j < nsub; j += NT) {
            const uint32_t k = fkey(smx[j]);
            if (k > kk) {
                sel[atomicAdd(&nsel_gt, 1u)] = j;
            } else if (k == kk) {
                const uint32_t s2 = atomicAdd(&neq, 1u);
                if (s2 < SMAXEQ) eqi[s2] = j;
            }
        }
        __syncthreads();
        const int ne = (int)min(neq, (uint32_t)SMAXEQ), g = (int)nsel_gt;
        for (int s2 = t; s2 < ne; s2 += NT) {
            int r = 0;
            for (int u = 0; u < ne; ++u) r += eqi[u] < eqi[s2];
            if (r < (int)take) sel[g + r] = eqi[s2];
        }
        __syncthreads();
        if (t == 0) {
            nsel_gt = 0;
            neq = 0;
        }
        // the K-th largest maximum: K sub-chunks hold an element at least
        // this large, so the K-th largest element is too
        const uint32_t u = (kk & 0x80000000u) ? (kk & 0x7FFFFFFFu) : ~kk;
        thr = __uint_as_float(u);
    } else if (t < nsel) {
        sel[t] = t;
    }
    __syncthreads();
    const double S = ssum;
    const int nc = nsel * SUB;
    for (int e = t; e < nc; e += NT) {
        const int64_t i = (int64_t)sel[e / SUB] * SUB + e % SUB;
        const float x = i < V ? lg[i] : -INFINITY;
        cp[e] = i < V && x >= thr ? (float)((double)sexp(x, mx, temp) / S) : -1.f;
    }
    __syncthreads();
    // the K-th largest probability (bits of p >= 0 order as p)
    uint32_t take_eq;
    const uint32_t kth = block_radix_kth(nc, (uint32_t)K,
                                         [&](int e, uint32_t* k) {
                                             const float pv = cp[e];
                                             *k = __float_as_uint(pv);
                                             return pv >= 0.f;
                                         },
                                         &take_eq);
    for (int e = t; e < nc; e += NT) {
        const float pv = cp[e];
        if (pv < 0.f) continue;
        const uint32_t key = __float_as_uint(pv);
        const int32_t i = sel[e / SUB] * SUB + e % SUB;
        if (key > kth) {
            const uint32_t s2 = atomicAdd(&nsel_gt, 1u);
            kp[s2] = pv;
            ki[s2] = i;
        } else if (key == kth) {
            const uint32_t s2 = atomicAdd(&neq, 1u);
            if (s2 < SMAXEQ) eqi[s2] = i;
        }
    }
    __syncthreads();
    {
        const int ne = (int)min(neq, (uint32_t)SMAXEQ), g = (int)nsel_gt;
        const float kv = __uint_as_float(kth);
        for (int s2 = t; s2 < ne; s2 += NT) {
            int r = 0;
            for (int u = 0; u < ne; ++u) r += eqi[u] < eqi[s2];
            if (r < (int)take_eq) {
                kp[g + r] = kv;
                ki[g + r] = eqi[s2];
            }
        }
    }
    __syncthreads();
    // the reference's arithmetic over the K kept values, on wave 0 with
    // value l in lane l: the orders by rank (comparisons with every lane's
    // value, read by v_readlane, then one LDS scatter / gather), the
    // sequential sums as loops over the lanes that every lane runs alike
    // (the same operations in the same order as one thread's loop over the
    // sorted array)
    if (t < 64) {
        float pv = l < K ? kp[l] : 0.f;
        int32_t iv = l < K ? ki[l] : INT_MAX;
        int32_t xr = 0;  // the element's rank by index, carried along
        // lane r takes the element of rank r of (p, i): p descending, index
        // ascending (the comparisons combined bitwise: no branch per lane
        // read); with_index: the ranks by index too
        auto place = [&](int r) {
            __builtin_amdgcn_wave_barrier();
            if (l < K) {
                kp[r] = pv;
                ki[r] = iv;
                kx[r] = xr;
            }
            __builtin_amdgcn_wave_barrier();
            pv = l < K ? kp[l] : 0.f;
            iv = l < K ? ki[l] : INT_MAX;
            xr = l < K ? kx[l] : 0;
            __builtin_amdgcn_wave_barrier();
        };
        auto rank = [&](bool with_index) {
            int r = 0, ri = 0;
#pragma unroll 4
            for (int j = 0; j < K; ++j) {
                const float pj = lane_f(pv, j);
                const int32_t ij = lane_i(iv, j);
                r += (int)((pj > pv) | ((pj == pv) & (ij < iv)));
                ri += (int)(ij < iv);
            }
            if (with_index) xr = ri;
            return r;
        };
        place(rank(true));
        if (use_k) {
            float keep = 0.f;
            for (int i = 0; i < K; ++i) keep += lane_f(pv, i);
            if (l < K) pv = pv / keep;
        }
        if (top_p < 1.f) {
            // the filtered values in (p, i) order again: the division keeps
            // the order of unequal values but can make neighbours equal,
            // whose order is then by index -- sorted again only if some
            // neighbour pair is out of that order
            const float pn = __shfl_down(pv, 1, 64);
            const int32_t in = __shfl_down(iv, 1, 64);
            if (__ballot(l + 1 < K && pn == pv && in < iv)) place(rank(false));
            double cum = 0.0;
            int cut = K + 1;  // not reached among the kept: nothing cut
            for (int i = 0; i < K; ++i) {
                cum += lane_f(pv, i);
                if (cum >= (double)top_p) {
                    cut = i + 1;
                    break;
                }
            }
            if (cut <= K) {
                double tail = 0.0;
                for (int i = cut; i < K; ++i) tail += lane_f(pv, i);
                if (l >= cut) pv = 0.f;
                if (tail > 0.0 && l < cut) pv = (float)(pv / (1.0 - tail));
            }
        }
        // the draw: the first index whose running double sum, as float,
        // reaches r (the elements in index order by their carried ranks)
        place(xr);
        uint64_t st = *state;
        const float r = sampler_next_float(st);
        int32_t pk = -1;
        if (r <= 0.f) {
            pk = 0;  // the reference's loop stops at index 0
        } else {
            double c = 0.0;
            for (int i = 0; i < K; ++i) {
                c += lane_f(pv, i);
                if ((float)c >= r) {
                    pk = lane_i(iv, i);
                    break;
                }
            }
        }
        if (l == 0) {
            *state = st;
            pick = pk >= 0 ? pk : amax;
        }
    }
    __syncthreads();
    const int32_t r = pick;
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

// Row r's statistics from its chunk results, by one wave (lane l): first-max
// argmax over the chunks, the exp sum over the sub-chunks (lane-strided sums
// in index order, then a fixed tree).
__device__ void row_stat_wave(const AcceptDev& a, int64_t r, int l) {
    const RowChunks& rc = a.rc;
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
        // lane-strided in index order, 16 loads in flight per lane
        const double* cs = rc.csub + r * rc.nsub;
        for (int j0 = l; j0 < rc.nsub; j0 += 64 * 16) {
            double v[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = cs[min(j0 + 64 * k, rc.nsub - 1)];
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (j0 + 64 * k < rc.nsub) sum += v[k];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    }
    if (l == 0) a.stats[r] = RowStats{best, bi, sum};
}

// Decisions by one workgroup: GREEDY and RESIDUAL (one-block form) finish
// here; RATIO walks the chain and draws the bonus with the sampler.
__device__ void accept_wg(const AcceptDev& a) {
#pragma clang fp contract(off)
    __shared__ double sd[NT];
    __shared__ uint64_t rng;
    __shared__ int32_t cur, nacc, bonus, next;
    __shared__ float mg;
    __shared__ uint64_t srng;
    const int t = threadIdx.x;
    const int64_t V = a.V;
    if (t == 0) {
        rng = *a.rng;
        srng = a.sampler_rng ? *a.sampler_rng : 0;
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
        for (int64_t r = w; r <= a.M; r += NT / 64) row_stat_wave(a, r, l);
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
        // the bonus: Sampler::sample of the row after the last accepted node
        const int32_t c = cur;
        const int64_t ro = (int64_t)(c + 1) * a.rc.nsub;
        const int32_t b = sampler_pick(ROW(c), V, STAT(c).mx, a.temp, a.top_k, a.top_p,
                                       a.rc.csubf + ro, a.rc.submax + ro, a.rc.nsub,
                                       STAT(c).amax, &srng);
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
        if (a.sampler_rng) *a.sampler_rng = srng;
        *a.margin = mg;
    }
}

__global__ void __launch_bounds__(NT) k_accept(AcceptDev a) { accept_wg(a); }

// several sequences' acceptances at once, workgroup s taking arr[s] (each
// sequence its own rows, statistics, streams and outputs)
__global__ void __launch_bounds__(NT) k_accept_multi(const AcceptDev* __restrict__ arr) {
    const AcceptDev a = arr[blockIdx.x];
    accept_wg(a);
}

// ---- RESIDUAL acceptance over many workgroups.  The decisions are made
// by every workgroup alike (each runs the same sequential walk on the same
// data, so no decision is broadcast); the vocabulary-wide work -- the
// residual p <- norm(max(0, p - q)) of a rejected child and its sum -- is
// split into one contiguous slice per workgroup, followed by a reduction
// barrier after which every workgroup has the slices' partial sums in slice
// order.
// The residual is kept unnormalised (P with its sum T, p = P / T), in two
// buffers used in turn by successive passes (as are the partial sums), so
// that a pass never overwrites what a slower workgroup may still read of
// the previous one; a node's
// target p = exp((l - mx) / T) / sum is formed on the fly from the row
// statistics, so a node whose first child is accepted costs no pass at all.
// The bonus after an all-rejected node is the inverse-CDF pick of the
// residual (the crossing slice from the partial sums, then the crossing
// element by a block scan of the slice); after a node without children it is
// the pick of the target (the crossing 128-element sub-chunk from the
// statistics' sub-chunk sums, then the element).
//
// The grid barrier is a flag per workgroup: a workgroup publishes its
// barrier count (release: its stores written back first), and one wave polls
// every flag with one load per lane until all have reached that count
// (acquire).  Measured on the device: 1.5-3 us for 16-32 workgroups, against
// 2.7-4.1 us for one shared counter (its atomics serialise at the memory
// side).  The waits are bounded: a barrier that does not complete in about
// 0.3 s sets the error word and every workgroup returns.

constexpr int RT = 256;  // threads per workgroup of the residual kernel

struct GridBar {
    int err, pad_[63];
    unsigned flags[ACC_RES_WG];
};

__device__ bool grid_barrier(GridBar* gb, unsigned G, unsigned& gen) {
    __shared__ int ok;
    __syncthreads();
    ++gen;
    if (threadIdx.x == 0) {
        ok = 1;
        __threadfence();
        __hip_atomic_store(&gb->flags[blockIdx.x], gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x < 64) {
        unsigned n = 0;
        for (;;) {
            int mine = 1;
            for (unsigned w = threadIdx.x; w < G; w += 64)
                mine &= (int)(__hip_atomic_load(&gb->flags[w], __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT) -
                                  gen <
                              0x80000000u);
            if (__all(mine)) break;
            if (++n > (1u << 18) ||
                __hip_atomic_load(&gb->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                if (threadIdx.x == 0) {
                    __hip_atomic_store(&gb->err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = 0;
                }
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (threadIdx.x == 0) __threadfence();
    }
    __syncthreads();
    return ok != 0;
}

// The reduction barrier of a pass: the partial sums are the flags.  Pass k
// uses buffer k % 3 of G 64-bit words holding the bitwise complement of each
// workgroup's sum, zero meaning "not yet published" (a sum is never the
// all-ones NaN pattern: the residual entries are finite and non-negative);
// workgroup w first clears its word of buffer (k + 1) % 3 (last read in
// pass k - 2, which every workgroup has finished: each has already
// published its pass k - 1 sum), then publishes its sum (release: its
// residual slice written back first); one wave polls all G words with one
// 64-bit load per lane until none is zero (acquire), and forms the
// sequential sum in slice order from the lanes' values.  vals and incl (LDS
// [G]) receive the values and the running sums.
__device__ bool part_barrier(GridBar* gb, unsigned long long* cur, unsigned long long* nxt,
                             double loc, unsigned G,
                             double* vals, double* incl, double& tot) {
    __shared__ int ok;
    __shared__ double stot;
    __syncthreads();
    if (threadIdx.x == 0) {
        ok = 1;
        __hip_atomic_store(&nxt[blockIdx.x], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __threadfence();
        __hip_atomic_store(&cur[blockIdx.x], ~(unsigned long long)__double_as_longlong(loc),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        double v = 0.0;
        unsigned n = 0;
        for (;;) {
            int mine = 1;
            if (l < (int)G) {
                const unsigned long long bits =
                    __hip_atomic_load(&cur[l], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                mine = bits != 0ull;
                v = __longlong_as_double((long long)~bits);
            }
            if (__all(mine)) break;
            if (++n > (1u << 18) ||
                __hip_atomic_load(&gb->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                if (l == 0) {
                    __hip_atomic_store(&gb->err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = 0;
                }
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (l == 0) __threadfence();
        double sum = 0.0;
        for (unsigned w = 0; w < G; ++w) {
            sum += lane_d(v, (int)w);
            if (l == (int)w) {
                vals[w] = v;
                incl[w] = sum;
            }
        }
        if (l == 0) stot = sum;
    }
    __syncthreads();
    tot = stot;
    return ok != 0;
}

__device__ double rblock_sum(double v, double* sd) {
    const int t = threadIdx.x;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((t & 63) == 0) sd[t >> 6] = v;
    __syncthreads();
    const double r = ((sd[0] + sd[1]) + sd[2]) + sd[3];
    __syncthreads();
    return r;
}

// Inverse-CDF pick inside [b, e) for `target` (the weights' running sum
// from b is compared with it): thread t takes a contiguous run, a block scan
// finds the crossing run, its thread scans it.  w(i) gives the weight of
// element i.  Returns the crossing index or, when rounding leaves none, the
// last positive one (-1 if none); *before (if given) receives the running
// sum ahead of the crossing element (0 when there is none).
template <typename Wf>
__device__ int32_t range_pick(int64_t b, int64_t e, double target, Wf w,
                              double* before = nullptr) {
    constexpr int RB = 16;  // run elements per thread with their loads in flight together
    __shared__ double incl[RT];
    __shared__ int32_t lastpos[RT];
    __shared__ int32_t pick;
    __shared__ double pick_before;
    const int t = threadIdx.x;
    const int64_t run = (e - b + RT - 1) / RT;
    const int64_t rb = min(e, b + t * run), re = min(e, rb + run);
    double cs = 0.0;
    int32_t lp = -1;
    for (int64_t i0 = rb; i0 < re; i0 += RB) {
        double v[RB];
#pragma unroll
        for (int k = 0; k < RB; ++k) v[k] = w(min(i0 + k, re - 1));
#pragma unroll
        for (int k = 0; k < RB; ++k)
            if (i0 + k < re) {
                cs += v[k];
                if (v[k] > 0) lp = (int32_t)(i0 + k);
            }
    }
    incl[t] = cs;
    lastpos[t] = lp;
    if (t == 0) {
        pick = -1;
        pick_before = 0.0;
    }
    __syncthreads();
    for (int o = 1; o < RT; o <<= 1) {
        const double add = t >= o ? incl[t - o] : 0.0;
        const int32_t lpo = t >= o ? lastpos[t - o] : -1;
        __syncthreads();
        incl[t] += add;
        if (lastpos[t] < 0) lastpos[t] = lpo;
        __syncthreads();
    }
    const double ex = t ? incl[t - 1] : 0.0;
    if (incl[t] > target && ex <= target && rb < re) {
        double c = ex, cb = 0.0;
        int32_t found = -1;
        for (int64_t i0 = rb; i0 < re && found < 0; i0 += RB) {
            double v[RB];
#pragma unroll
            for (int k = 0; k < RB; ++k) v[k] = w(min(i0 + k, re - 1));
#pragma unroll
            for (int k = 0; k < RB; ++k)
                if (i0 + k < re && found < 0) {
                    cb = c;
                    c += v[k];
                    if (c > target) found = (int32_t)(i0 + k);
                }
        }
        if (found >= 0) {
            pick = found;
            pick_before = cb;
        }
    }
    __syncthreads();
    const int32_t r = pick >= 0 ? pick : lastpos[RT - 1];
    if (before) *before = pick_before;
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(RT) k_accept_res(AcceptDev a, GridBar* gb,
                                                   unsigned long long* part) {
#pragma clang fp contract(off)
    constexpr int PU = 16;  // residual elements per thread with their loads in flight together
    __shared__ double sd[RT / 64];
    __shared__ double pvals[ACC_RES_WG], pincl[ACC_RES_WG];
    const unsigned G = gridDim.x;
    const int wg = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const int64_t V = a.V, M = a.M;
    unsigned gen = 0;
    // row statistics: one wave per row, rows spread over the workgroups
    for (int64_t r = (int64_t)wg * (RT / 64) + (t >> 6); r <= M; r += (int64_t)G * (RT / 64))
        row_stat_wave(a, r, lane);
    if (!grid_barrier(gb, G, gen)) return;
    const int64_t slice = (V + G - 1) / G;
    const int64_t s0 = min(V, (int64_t)wg * slice), s1 = min(V, s0 + slice);
    uint64_t rng = *a.rng;
    float mg = INFINITY;
    int32_t cur = -1, nacc = 0;
    int64_t pass = 0;  // residual passes so far: buffer pass % 2 holds the latest
    const double* Pc = a.p;  // the latest residual
#define ROW(c) ((c) < 0 ? a.base_row : a.rows + (int64_t)(c) * V)
    for (int64_t step = 0; step <= M; ++step) {
        const RowStats st = a.stats[cur + 1];
        const float* lg = ROW(cur);
        double T = st.sum;
        bool have_res = false;
        int32_t next = -2;
        // the children of cur in index order: 64 parents per load, the
        // matches taken from the ballot (uniform over the workgroup)
        for (int64_t c0 = 0; c0 < M && next < -1; c0 += 64) {
            const int32_t par = c0 + lane < M ? a.parents[c0 + lane] : INT_MIN;
            const int32_t ptok = c0 + lane < M ? a.props[c0 + lane] : 0;
            uint64_t kids = __ballot(par == cur);
            while (kids) {
                const int j = __builtin_ctzll(kids);
                const int64_t ch = c0 + j;
                kids &= kids - 1;
                const float* qc = a.q + ch * V;
                const int32_t tok = lane_i(ptok, j);
                const double pv = have_res ? Pc[tok] / T : texp(lg[tok], st.mx, a.temp) / T;
                const float pt = (float)pv;
                const float ratio = fminf(1.f, pt / fmaxf(qc[tok], 1e-9f));
                const float u = splitmix_float(rng);
                mg = fminf(mg, fabsf(u - ratio));
                if (u <= ratio) {
                    next = (int32_t)ch;
                    break;
                }
                // p <- max(0, p - q_ch) over this workgroup's slice, its sum
                // (element order per thread as a plain strided loop)
                double* Pn = a.p + (pass & 1) * V;
                unsigned long long* partn = part + (pass % 3) * G;
                unsigned long long* partx = part + ((pass + 1) % 3) * G;
                double loc = 0.0;
                for (int64_t i0 = s0 + t; i0 < s1; i0 += (int64_t)RT * PU) {
                    double bv[PU];
                    float qv[PU];
                    if (have_res) {
#pragma unroll
                        for (int k = 0; k < PU; ++k) bv[k] = Pc[min(i0 + (int64_t)k * RT, s1 - 1)];
                    } else {
                        float lv[PU];
#pragma unroll
                        for (int k = 0; k < PU; ++k) lv[k] = lg[min(i0 + (int64_t)k * RT, s1 - 1)];
#pragma unroll
                        for (int k = 0; k < PU; ++k) bv[k] = texp(lv[k], st.mx, a.temp);
                    }
#pragma unroll
                    for (int k = 0; k < PU; ++k) qv[k] = qc[min(i0 + (int64_t)k * RT, s1 - 1)];
#pragma unroll
                    for (int k = 0; k < PU; ++k) {
                        const int64_t i = i0 + (int64_t)k * RT;
                        const double r = bv[k] / T - (double)qv[k];
                        const double v = r > 0 ? r : 0.0;
                        if (i < s1) {
                            Pn[i] = v;
                            loc += v;
                        }
                    }
                }
                loc = rblock_sum(loc, sd);
                ++pass;
                Pc = Pn;
                double tot;
                if (!part_barrier(gb, partn, partx, loc, G, pvals, pincl, tot)) return;
                if (tot > 0) {
                    T = tot;
                    have_res = true;
                } else {  // p == q: back to the target (p untouched by the oracle)
                    T = st.sum;
                    have_res = false;
                }
            }
        }
        if (next >= -1) {
            if (wg == 0 && t == 0) a.out[2 + nacc] = next;
            ++nacc;
            cur = next;
            continue;
        }
        // the bonus
        const float ub = splitmix_float(rng);
        int32_t bonus = -1;
        if (have_res) {
            const double target = (double)ub * T;
            double cum = 0.0;
            unsigned ws = G;
            for (unsigned w = 0; w < G; ++w) {
                if (pincl[w] > target) {
                    ws = w;
                    break;
                }
                cum = pincl[w];
            }
            if (ws == G) {  // rounding: the last slice with weight
                for (unsigned w = G; w-- > 0;)
                    if (pvals[w] > 0) {
                        ws = w;
                        break;
                    }
                cum = -1.0;  // take that slice's last positive element
            }
            if ((unsigned)wg == ws) {
                const int64_t b = min(V, (int64_t)ws * slice), e = min(V, b + slice);
                const double* P = Pc;
                const int32_t r = range_pick(b, e, cum < 0 ? INFINITY : target - cum,
                                             [&](int64_t i) { return P[i]; });
                bonus = r >= 0 ? r : (int32_t)b;
            }
        } else if (wg == 0) {
            // the target: crossing sub-chunk by the sub-chunk sums, then its
            // elements
            const RowChunks& rc = a.rc;
            const double* cs = rc.csub + (int64_t)(cur + 1) * rc.nsub;
            const double target = (double)ub * st.sum;
            double before;
            const int32_t sc =
                range_pick(0, rc.nsub, target, [&](int64_t j) { return cs[j]; }, &before);
            if (sc >= 0) {
                const int64_t b = (int64_t)sc * SUB, e = min(V, b + SUB);
                const float mx = st.mx, tp = a.temp;
                const int32_t r = range_pick(b, e, target - before,
                                             [&](int64_t i) { return texp(lg[i], mx, tp); });
                bonus = r >= 0 ? r : (int32_t)b;
            } else {
                bonus = st.amax;
            }
        }
        if (bonus >= 0 && t == 0) a.out[1] = bonus;
        break;
    }
#undef ROW
    if (wg == 0 && t == 0) {
        a.out[0] = nacc;
        *a.rng = rng;
        *a.margin = mg;
    }
}

// Sampler::argmax and softmax_prob of that token (src/spec.cpp:89-95, as
// DraftModelDrafter::draft uses them, 100-119) from one row's chunk
// statistics at T = 1: the first maximum and 1 / sum_i exp((double)(l_i -
// max)) as float.  One wave; out = {token, prob bits}.
__global__ void __launch_bounds__(64) k_argmax_prob(RowChunks rc, int32_t* out) {
    const int l = threadIdx.x;
    float best = -INFINITY;
    int32_t bi = 0x7FFFFFFF;
    for (int c = l; c < rc.nch; c += 64) {
        const float v = rc.cmax[c];
        const int32_t iv = rc.carg[c];
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
    for (int j = l; j < rc.nsub; j += 64) sum += rc.csub[j];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (l == 0) {
        out[0] = bi;
        out[1] = __float_as_int((float)(exp(0.0) / sum));  // the maximum's exp((double)0)
    }
}

}  // namespace

hipError_t launch_argmax_prob(hipStream_t st, const float* row, int64_t V, void* scratch,
                              int32_t* out) {
    const RowChunks rc = row_chunks(scratch, 1, V);
    hipError_t e = launch_row_stats(st, row, nullptr, 1, V, 1.f, 1, rc);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_prob, dim3(1), dim3(64), 0, st, rc, out);
    return hipGetLastError();
}

size_t row_stats_scratch_bytes(int64_t nrows, int64_t V) {
    const int64_t nch = (V + SCH - 1) / SCH, nsub = (V + SUB - 1) / SUB;
    return (size_t)(nrows * nsub) * (8 + 8 + 4) + (size_t)(nrows * nch) * 8 + 64;
}

RowChunks row_chunks(void* scratch, int64_t nrows, int64_t V) {
    RowChunks rc{};
    rc.nch = (int)((V + SCH - 1) / SCH);
    rc.nsub = (int)((V + SUB - 1) / SUB);
    rc.csub = (double*)scratch;
    rc.csubf = rc.csub + nrows * rc.nsub;
    rc.cmax = (float*)(rc.csubf + nrows * rc.nsub);
    rc.carg = (int32_t*)(rc.cmax + nrows * rc.nch);
    rc.submax = (float*)(rc.carg + nrows * rc.nch);
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

hipError_t launch_accept_multi(hipStream_t st, const AcceptDev* d_arr, int n) {
    if (n < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_accept_multi, dim3((unsigned)n), dim3(NT), 0, st, d_arr);
    return hipGetLastError();
}

constexpr size_t ACC_RES_BAR = (sizeof(GridBar) + 255) & ~(size_t)255;
size_t accept_residual_scratch_bytes() { return ACC_RES_BAR + 3 * ACC_RES_WG * sizeof(double); }

// RESIDUAL acceptance over ACC_RES_WG workgroups, launched cooperatively so
// that all of them are resident for the grid barriers.  scratch: the
// barrier flags and error word and the slices' partial-sum words (three
// sets), all zeroed here; a.p holds two residual buffers of V doubles.
hipError_t launch_accept_residual(hipStream_t st, const AcceptDev& a, void* scratch) {
    GridBar* gb = (GridBar*)scratch;
    unsigned long long* part = (unsigned long long*)((uint8_t*)scratch + ACC_RES_BAR);
    // flags, error word and partial-sum words: zero
    hipError_t e = hipMemsetAsync(gb, 0, accept_residual_scratch_bytes(), st);
    if (e != hipSuccess) return e;
    AcceptDev ac = a;
    void* args[] = {(void*)&ac, (void*)&gb, (void*)&part};
    return hipLaunchCooperativeKernel((const void*)k_accept_res, dim3(ACC_RES_WG), dim3(RT), args,
                                      0, st);
}

int accept_residual_error(const void* scratch, hipStream_t st, int* err) {
    return hipMemcpyAsync(err, (const uint8_t*)scratch + offsetof(GridBar, err), sizeof(int),
                          hipMemcpyDeviceToHost, st) == hipSuccess
               ? 0
               : -1;
}
