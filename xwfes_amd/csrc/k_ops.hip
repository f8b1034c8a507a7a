// k_ops.hip -- per-layer host ops of Engine::forward moved to the device:
// embedding lookup, RMSNorm, RoPE + KV append, and tree-masked GQA attention.
#include "ftx_internal.h"
#include "quant_dev.h"

// ---------------------------------------------------------------- embedding
// x[m, :] = dequant(E row toks[m]): a row lookup (the reference indexes a
// plane with HostTensor::slice(t), src/engine.cpp:494-495, which is only
// right for t == 0; the row is what forward() means).
__global__ void __launch_bounds__(256) k_embed(const uint8_t* __restrict__ E, int dt,
                                               int64_t row_bytes, int64_t d,
                                               const int32_t* __restrict__ toks,
                                               float* __restrict__ x) {
    const int64_t m = blockIdx.y;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g * 8 >= d) return;
    float v[8];
    dq8(E + (int64_t)toks[m] * row_bytes, dt, g * 8, d, v);
    float* o = x + m * d + g * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (g * 8 + i < d) o[i] = v[i];
}

hipError_t launch_embed(hipStream_t st, const uint8_t* E, int dt, int64_t row_bytes, int64_t d,
                        const int32_t* toks, int64_t M, float* x) {
    if (M == 0) return hipSuccess;
    const int64_t groups = (d + 7) / 8;
    hipLaunchKernelGGL(k_embed, dim3((unsigned)((groups + 255) / 256), (unsigned)M), dim3(256), 0,
                       st, E, dt, row_bytes, d, toks, x);
    return hipGetLastError();
}

// ---------------------------------------------------------------- RMSNorm
// src/engine.cpp:23-41: ss = sum x^2; inv = 1/sqrt(ss/n + eps); (x*inv)*w
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x,
                                                 const float* __restrict__ w, int64_t d,
                                                 float eps, float* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t m = blockIdx.x;
    const float* xr = x + m * d;
    float ss = 0.f;
    for (int64_t i = threadIdx.x; i < d; i += 256) ss += xr[i] * xr[i];
    // wave sums by shuffles, then the four waves' sums in wave order
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv = 1.f / sqrtf(tot / (float)d + eps);
    float* orow = out + m * d;
    for (int64_t i = threadIdx.x; i < d; i += 256) orow[i] = xr[i] * inv * w[i];
}

hipError_t launch_rmsnorm(hipStream_t st, const float* x, const float* w, int64_t d, int64_t M,
                          float eps, float* out) {
    if (M == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)M), dim3(256), 0, st, x, w, d, eps, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------- RoPE + KV
// src/engine.cpp:43-60 (frequencies and angles in double, cos/sin rounded
// to float; neox pairs (i, i+hd/2), else interleaved (2i, 2i+1)) applied to
// q and k at position npast + depth[m]; k and v are then written to KV slot
// npast + m (src/engine.cpp:555-561).  Before RoPE, when given: the bias of
// q / k / v and the per-head RMSNorm of q and k (src/engine.cpp:519-542;
// the head's sum of squares as a wave sum).  One wave per (token, head).
__device__ __forceinline__ void rope_kv_row(const RopeArgs& a, int64_t m, int64_t h) {
#pragma clang fp contract(off)
    // h: 0..n_head-1 q heads, then kv heads
    const int64_t half = a.hd / 2;
    const int64_t npast = *a.npast;
    const int64_t pos = npast + a.depth[m];
    const int64_t qdim = a.n_head * a.hd, kdim = a.n_kv * a.hd;
    float* row = a.qkv + m * a.ldq;
    float* v;
    const bool is_q = h < a.n_head;
    const int64_t off = is_q ? h * a.hd : qdim + (h - a.n_head) * a.hd;
    v = row + off;
    const float* nw = is_q ? a.qnorm : a.knorm;
    if (a.part) {
        // the head's q (or k and v) elements from the GEMM's split partials
        // (eight splits' loads in flight at a time)
        const float* p = a.part + m * a.ldp;
        auto sum = [&](int64_t col) {
            float g = 0.f;
            for (int s0 = 0; s0 < a.S; s0 += 8) {
                float pv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) pv[i] = s0 + i < a.S ? p[(s0 + i) * a.split_stride + col] : 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) g += pv[i];
            }
            return g;
        };
        for (int64_t t = threadIdx.x; t < a.hd; t += blockDim.x) {
            v[t] = sum(off + t);
            if (!is_q) row[off + kdim + t] = sum(off + kdim + t);
        }
        __syncthreads();
    }
    if (a.bias || nw) {
        float ss = 0.f;
        for (int64_t t = threadIdx.x; t < a.hd; t += blockDim.x) {
            float x = v[t];
            if (a.bias) {
                x = x + a.bias[off + t];
                v[t] = x;
                if (!is_q) row[off + kdim + t] += a.bias[off + kdim + t];  // v of this kv head
            }
            ss += x * x;
        }
        if (nw) {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            const float inv = 1.f / sqrtf(ss / (float)a.hd + a.eps);
            for (int64_t t = threadIdx.x; t < a.hd; t += blockDim.x) v[t] = v[t] * inv * nw[t];
        }
        __syncthreads();  // RoPE pairs cross the threads' elements
    }
    for (int64_t i = threadIdx.x; i < half; i += blockDim.x) {
        float c, s;
        if (a.cs) {
            c = a.cs[(m * half + i) * 2];
            s = a.cs[(m * half + i) * 2 + 1];
        } else {
            const double f = pow(a.theta, -2.0 * (double)i / (double)a.hd);
            const double ang = (double)pos * f;
            c = (float)cos(ang);
            s = (float)sin(ang);
        }
        const int64_t ia = a.neox ? i : 2 * i, ib = a.neox ? i + half : 2 * i + 1;
        const float x0 = v[ia], x1 = v[ib];
        const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
        v[ia] = y0;
        v[ib] = y1;
        if (h < a.n_head && a.qh16) {
            const int64_t o = (m * a.n_head + h) * a.hd;
            const _Float16 h0 = (_Float16)y0, h1 = (_Float16)y1;
            a.qh16[o + ia] = h0;
            a.qh16[o + ib] = h1;
            a.ql16[o + ia] = (_Float16)(y0 - (float)h0);
            a.ql16[o + ib] = (_Float16)(y1 - (float)h1);
        }
    }
    if (h < a.n_head) return;
    __syncthreads();
    const int64_t kh = h - a.n_head;
    const int64_t slot = npast + m;
    const float* kr = row + qdim + kh * a.hd;
    const float* vr = row + qdim + kdim + kh * a.hd;
    for (int64_t t = threadIdx.x; t < a.hd; t += blockDim.x) {
        const int64_t idx = slot * kdim + kh * a.hd + t;
        const int64_t vidx = v_index(slot, kh, t, a.hd, a.cap);
        if (a.kv_f16) {
            ((_Float16*)a.kc)[idx] = (_Float16)kr[t];
            ((_Float16*)a.vc)[vidx] = (_Float16)vr[t];
        } else {
            ((float*)a.kc)[idx] = kr[t];
            ((float*)a.vc)[vidx] = vr[t];
        }
    }
}

__global__ void k_rope_kv(RopeArgs a) { rope_kv_row(a, blockIdx.x, blockIdx.y); }

// The same for head sizes up to 256, one wave per (token, head) and four
// heads per workgroup: lane l takes the head's rotation pairs l and l + 64,
// and every value stays in registers from the split partials (or the row)
// to the row, query and cache writes (the one-wave form above passes each
// element through memory between its stages).  The arithmetic per element
// is the one-wave form's: partials in split order, bias, (x * inv) * w, the
// rotation without contraction; the head's sum of squares is a wave sum.
constexpr int ROPE_HPW = 4;  // heads per workgroup
__device__ __forceinline__ void rope_kv_head(const RopeArgs& a, int64_t m, int64_t h, int lane) {
#pragma clang fp contract(off)
    const int64_t half = a.hd / 2;
    const int64_t npast = *a.npast;
    const int64_t pos = npast + a.depth[m];
    const int64_t qdim = a.n_head * a.hd, kdim = a.n_kv * a.hd;
    float* row = a.qkv + m * a.ldq;
    const bool is_q = h < a.n_head;
    const int64_t off = is_q ? h * a.hd : qdim + (h - a.n_head) * a.hd;
    const float* nw = is_q ? a.qnorm : a.knorm;
    const float* prow = a.part ? a.part + m * a.ldp : nullptr;
    // pair j of the lane: index i = lane + 64 j, elements ia, ib of the head
    float x[2][2], v[2][2];
    int64_t el[2][2];
    bool ok[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int64_t i = lane + 64 * j;
        ok[j] = i < half;
        const int64_t ic = ok[j] ? i : 0;
        el[j][0] = a.neox ? ic : 2 * ic;
        el[j][1] = a.neox ? ic + half : 2 * ic + 1;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            x[j][e] = 0.f;
            v[j][e] = 0.f;
        }
    }
    if (prow) {
        // eight splits' loads of every element at once (clamped split index,
        // masked), then each element summed in split order
        for (int s0 = 0; s0 < a.S; s0 += 8) {
            float px[8][2][2], pv[8][2][2];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float* ps = prow + min(s0 + q, a.S - 1) * a.split_stride + off;
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        px[q][j][e] = ps[el[j][e]];
                        pv[q][j][e] = is_q ? 0.f : ps[kdim + el[j][e]];
                    }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const bool in = s0 + q < a.S;
                        x[j][e] += in ? px[q][j][e] : 0.f;
                        v[j][e] += in ? pv[q][j][e] : 0.f;
                    }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                x[j][e] = row[off + el[j][e]];
                if (!is_q) v[j][e] = row[off + kdim + el[j][e]];
            }
    }
    if (a.bias) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                x[j][e] = x[j][e] + a.bias[off + el[j][e]];
                if (!is_q) v[j][e] = v[j][e] + a.bias[off + kdim + el[j][e]];
            }
    }
    if (nw) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (ok[j]) {
                ss += x[j][0] * x[j][0];
                ss += x[j][1] * x[j][1];
            }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        const float inv = 1.f / sqrtf(ss / (float)a.hd + a.eps);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 2; ++e) x[j][e] = x[j][e] * inv * nw[el[j][e]];
    }
    const int64_t slot = npast + m;
    const int64_t kh = h - a.n_head;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if (!ok[j]) continue;
        const int64_t i = lane + 64 * j;
        float c, sn;
        if (a.cs) {
            c = a.cs[(m * half + i) * 2];
            sn = a.cs[(m * half + i) * 2 + 1];
        } else {
            const double f = pow(a.theta, -2.0 * (double)i / (double)a.hd);
            const double ang = (double)pos * f;
            c = (float)cos(ang);
            sn = (float)sin(ang);
        }
        const float x0 = x[j][0], x1 = x[j][1];
        const float y[2] = {x0 * c - x1 * sn, x0 * sn + x1 * c};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int64_t t = el[j][e];
            row[off + t] = y[e];
            if (is_q) {
                if (a.qh16) {
                    const int64_t o = (m * a.n_head + h) * a.hd + t;
                    const _Float16 hv = (_Float16)y[e];
                    a.qh16[o] = hv;
                    a.ql16[o] = (_Float16)(y[e] - (float)hv);
                }
            } else {
                if (prow || a.bias) row[off + kdim + t] = v[j][e];
                const int64_t idx = slot * kdim + kh * a.hd + t;
                const int64_t vidx = v_index(slot, kh, t, a.hd, a.cap);
                if (a.kv_f16) {
                    ((_Float16*)a.kc)[idx] = (_Float16)y[e];
                    ((_Float16*)a.vc)[vidx] = (_Float16)v[j][e];
                } else {
                    ((float*)a.kc)[idx] = y[e];
                    ((float*)a.vc)[vidx] = v[j][e];
                }
            }
        }
    }
}

__global__ void __launch_bounds__(64 * ROPE_HPW) k_rope_kv4(RopeBatch b) {
    int s = 0;
    while (s + 1 < b.nseq && (int)blockIdx.x >= b.row0[s + 1]) ++s;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t h = (int64_t)blockIdx.y * ROPE_HPW + w;
    if (h >= b.s[s].n_head + b.s[s].n_kv) return;  // wave-uniform; no barrier below
    rope_kv_head(b.s[s], (int64_t)blockIdx.x - b.row0[s], h, lane);
}

// several sequences: sequence s owns token rows row0[s] .. row0[s + 1] - 1
__global__ void k_rope_kv_batch(RopeBatch b) {
    int s = 0;
    while (s + 1 < b.nseq && (int)blockIdx.x >= b.row0[s + 1]) ++s;
    rope_kv_row(b.s[s], (int64_t)blockIdx.x - b.row0[s], blockIdx.y);
}

// V between the canonical per-layer [slot][n_kv*hd] layout and the device
// [n_kv][hd][slot] layout; one thread per element.
__global__ void __launch_bounds__(256) k_v_layout(const uint8_t* __restrict__ src,
                                                  uint8_t* __restrict__ dst, int64_t cap,
                                                  int64_t n_kv, int64_t hd, int eb,
                                                  int to_device, int64_t total) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int64_t per = cap * n_kv * hd;
    const int64_t l = t / per, r = t % per;
    const int64_t slot = r / (n_kv * hd), c = r % (n_kv * hd);
    const int64_t canon = l * per + r;
    const int64_t dev = l * per + v_index(slot, c / hd, c % hd, hd, cap);
    const int64_t s = to_device ? canon : dev, d = to_device ? dev : canon;
    if (eb == 2) ((uint16_t*)dst)[d] = ((const uint16_t*)src)[s];
    else ((uint32_t*)dst)[d] = ((const uint32_t*)src)[s];
}

hipError_t launch_v_layout(hipStream_t st, const void* src, void* dst, int64_t n_layer,
                           int64_t cap, int64_t n_kv, int64_t hd, int elem_bytes, int to_device) {
    const int64_t total = n_layer * cap * n_kv * hd;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_v_layout, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                       (const uint8_t*)src, (uint8_t*)dst, cap, n_kv, hd, elem_bytes, to_device,
                       total);
    return hipGetLastError();
}

hipError_t launch_rope_kv(hipStream_t st, const RopeArgs& a, int64_t M) {
    if (M == 0) return hipSuccess;
    if (a.hd % 2 == 0 && a.hd <= 256) return launch_rope_kv_batch(st, &a, &M, 1);
    hipLaunchKernelGGL(k_rope_kv, dim3((unsigned)M, (unsigned)(a.n_head + a.n_kv)), dim3(64), 0,
                       st, a);
    return hipGetLastError();
}

hipError_t launch_rope_kv_batch(hipStream_t st, const RopeArgs* as, const int64_t* M, int nseq) {
    if (nseq < 1 || nseq > FTX_MAX_SEQ) return hipErrorInvalidValue;
    RopeBatch b{};
    b.nseq = nseq;
    int rows = 0;
    for (int s = 0; s < nseq; ++s) {
        if (as[s].n_head != as[0].n_head || as[s].n_kv != as[0].n_kv) return hipErrorInvalidValue;
        b.s[s] = as[s];
        b.row0[s] = rows;
        rows += (int)M[s];
    }
    b.row0[nseq] = rows;
    if (rows == 0) return hipSuccess;
    bool regs = true;  // every sequence's head size fits the register form
    for (int s = 0; s < nseq; ++s) regs = regs && as[s].hd % 2 == 0 && as[s].hd <= 256;
    const int64_t nh = as[0].n_head + as[0].n_kv;
    if (regs)
        hipLaunchKernelGGL(k_rope_kv4, dim3((unsigned)rows, (unsigned)((nh + ROPE_HPW - 1) / ROPE_HPW)),
                           dim3(64 * ROPE_HPW), 0, st, b);
    else
        hipLaunchKernelGGL(k_rope_kv_batch, dim3((unsigned)rows, (unsigned)nh), dim3(64), 0, st, b);
    return hipGetLastError();
}

// ---------------------------------------------------------------- attention
// Impl::attn (src/engine.cpp:137-177) with an ancestor mask: query row m of
// head h attends to cache positions [0, npast) and to the tree slots
// npast + j of its ancestors j (itself included).  kv head = h / (n_head /
// n_kv); scores are float dots scaled by 1/sqrt(hd); softmax as
// softmax_inplace (float max, float exp, double sum, float scale).
__device__ __forceinline__ float kv_load(const void* base, int f16, int64_t idx) {
    return f16 ? (float)((const _Float16*)base)[idx] : ((const float*)base)[idx];
}

__global__ void __launch_bounds__(256) k_attention(AttnArgs a) {
#pragma clang fp contract(off)
    extern __shared__ float lds[];
    const int64_t m = blockIdx.x, h = blockIdx.y;
    const int64_t hd = a.hd, kdim = a.n_kv * hd;
    const int64_t kvh = h / (a.n_head / a.n_kv);
    const int64_t npast = *a.npast;
    float* qv = lds;                  // hd
    float* sc = lds + hd;             // slots
    __shared__ int32_t tslot[256];    // tree slots of this row
    __shared__ int ntree;
    __shared__ float red[256];
    __shared__ double redd[256];
    const int tid = threadIdx.x;
    for (int64_t t = tid; t < hd; t += 256) qv[t] = a.qkv[m * a.ldq + h * hd + t];
    if (tid == 0) {
        int c = 0;
        const uint32_t* an = a.anc + m * a.anc_words;
        for (int w = 0; w < a.anc_words; ++w) {
            uint32_t bits = an[w];
            while (bits) {
                const int b = __builtin_ctz(bits);
                bits &= bits - 1;
                tslot[c++] = w * 32 + b;
            }
        }
        ntree = c;
    }
    __syncthreads();
    const int64_t n = npast + ntree;
    const float scale = 1.f / sqrtf((float)hd);
    const int64_t koff = kvh * hd;
    for (int64_t s = tid; s < n; s += 256) {
        const int64_t slot = s < npast ? s : npast + tslot[s - npast];
        const int64_t base = slot * kdim + koff;
        float d = 0.f;
        for (int64_t t = 0; t < hd; ++t) d += qv[t] * kv_load(a.kc, a.kv_f16, base + t);
        sc[s] = d * scale;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int64_t s = tid; s < n; s += 256) mx = fmaxf(mx, sc[s]);
    red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    mx = red[0];
    double sum = 0.0;
    for (int64_t s = tid; s < n; s += 256) {
        const float e = expf(sc[s] - mx);
        sc[s] = e;
        sum += (double)e;
    }
    redd[tid] = sum;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) redd[tid] += redd[tid + o];
        __syncthreads();
    }
    const float inv = (float)(1.0 / redd[0]);
    // output: two threads per dimension, each over half the slots
    const int64_t dim = tid % 128, part = tid / 128;
    float* ored = red;  // reuse: [128] partials of part 1
    float acc = 0.f;
    if (dim < hd) {
        for (int64_t s = part; s < n; s += 2) {
            const float w = sc[s] * inv;
            if (w == 0.f) continue;
            const int64_t slot = s < npast ? s : npast + tslot[s - npast];
            acc += w * kv_load(a.vc, a.kv_f16, v_index(slot, kvh, dim, hd, a.cap));
        }
    }
    __syncthreads();
    if (part == 1 && dim < hd) ored[dim] = acc;
    __syncthreads();
    if (part == 0 && dim < hd) a.out[m * a.n_head * hd + h * hd + dim] = acc + ored[dim];
    // head_dim above 128 is handled by the loop below
    for (int64_t t = 128 + tid; t < hd; t += 256) {
        float o = 0.f;
        for (int64_t s = 0; s < n; ++s) {
            const float w = sc[s] * inv;
            if (w == 0.f) continue;
            const int64_t slot = s < npast ? s : npast + tslot[s - npast];
            o += w * kv_load(a.vc, a.kv_f16, v_index(slot, kvh, t, hd, a.cap));
        }
        a.out[m * a.n_head * hd + h * hd + t] = o;
    }
}

hipError_t launch_attention(hipStream_t st, const AttnArgs& a, int64_t M) {
    if (M == 0) return hipSuccess;
    const size_t lds = (size_t)(a.hd + a.max_ctx) * sizeof(float);
    if (lds > 160 * 1024 - 8 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_attention, dim3((unsigned)M, (unsigned)a.n_head), dim3(256), lds, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------- KV commit
// After a verify step over draft nodes at slots npast + j, keep the accepted
// path nodes[0..n-1] at slots npast + i (KvCache::set_npast / Engine::
// truncate_to, include/ft/kv_cache.h:31, src/engine.cpp:423-428, extended to
// trees).  Thread = one element of a K row or of a transposed V row of one
// layer; it walks the path in increasing i.  In place: nodes is strictly
// increasing with nodes[i] >= i, so a later source nodes[i'] > nodes[i] >= i
// is never a slot written before it.
template <typename T>
__global__ void __launch_bounds__(256) k_kv_commit(KvCommitArgs a, T* __restrict__ k,
                                                   T* __restrict__ v) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t l = blockIdx.y;
    const int64_t kdim = (int64_t)a.n_kv * a.hd;
    if (e >= kdim) return;
    T* kl = k + l * a.cap * kdim;
    // transposed V: [layer][n_kv][hd][cap]; element e = kv head e / hd, dim e % hd
    T* vr = v + (l * kdim + e) * a.cap;
    for (int i = 0; i < a.n; ++i) {
        const int64_t src = a.npast + a.nodes[i], dst = a.npast + i;
        if (src == dst) continue;
        kl[dst * kdim + e] = kl[src * kdim + e];
        vr[dst] = vr[src];
    }
}

hipError_t launch_kv_commit(hipStream_t st, const KvCommitArgs& a, void* k, void* v, int kv_f16) {
    if (a.n <= 0) return hipSuccess;
    const int64_t kdim = (int64_t)a.n_kv * a.hd;
    const dim3 grid((unsigned)((kdim + 255) / 256), (unsigned)a.n_layer);
    if (kv_f16)
        hipLaunchKernelGGL(k_kv_commit<_Float16>, grid, dim3(256), 0, st, a, (_Float16*)k,
                           (_Float16*)v);
    else
        hipLaunchKernelGGL(k_kv_commit<float>, grid, dim3(256), 0, st, a, (float*)k, (float*)v);
    return hipGetLastError();
}
