// k_attn.hip -- tree-masked GQA attention over the fp16 KV cache on MFMA,
// split over 64-slot chunks of the context (flash-decoding) and combined in
// a second pass.
//
// Semantics of Impl::attn (src/engine.cpp:137-177) with the draft-tree mask:
// query row m of head h attends to cache slots [0, npast) and to the tree
// slots npast + j of its ancestors j (itself included); kv head =
// h / (n_head / n_kv); scores are q.k / sqrt(hd); softmax; sum of p * v.
//
// One wave handles one kv head, one 64-slot chunk and up to 32 query rows
// (the GQA group of every draft token: row r -> token r / gqa, head
// kvh * gqa + r % gqa).  Scores are computed transposed, S^T = K . Q^T, with
// v_mfma_f32_32x32x16_f16: K is fp16 in the cache (exact operand), Q is
// split into fp16 hi + lo parts (two MFMAs) so the scores keep fp32
// accuracy.  In the S^T layout each lane holds 16 slots of one query row,
// so the row max / sum need one cross-lane step, and the probabilities are
// already laid out as the A operand of O = P . V (hi + lo again).  V is kept
// transposed in the cache ([kv head][dim][slot]) so the B operand of P . V
// is a contiguous load.
#include "ftx_internal.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int CH = 64;  // slots per chunk

__device__ __forceinline__ bool slot_visible(const AttnMArgs& a, int64_t npast, int m, int64_t p) {
    if (p < npast) return true;
    const int64_t j = p - npast;
    if (j >= a.M) return false;
    return (a.anc[(int64_t)m * a.anc_words + (j >> 5)] >> (j & 31)) & 1u;
}

template <int HD>
__global__ void __launch_bounds__(64) k_attn_mfma(AttnMArgs a) {
    constexpr int NDC = HD / 16;  // 16-dim chunks of the score contraction
    constexpr int NDT = HD / 32;  // 32-dim tiles of the output
    const int lane = threadIdx.x, col = lane & 31, g = lane >> 5;
    const int64_t npast = *a.npast;
    const int64_t total = npast + a.M;
    const int c = blockIdx.x;
    const int64_t slot0 = (int64_t)c * CH;
    if (slot0 >= total) return;
    const int kvh = blockIdx.y;
    const int gqa = a.n_head / a.n_kv;
    const int qrows = a.M * gqa;
    // this lane's query row (B operand column of S^T)
    const int rq = blockIdx.z * 32 + col;
    const bool qvalid = rq < qrows;
    const int mq = qvalid ? rq / gqa : 0;
    const int hq = kvh * gqa + (qvalid ? rq % gqa : 0);
    v8h qh[NDC], ql[NDC];
    {
        const float* qv = a.qkv + (int64_t)mq * a.ldq + (int64_t)hq * HD;
#pragma unroll
        for (int dc = 0; dc < NDC; ++dc) {
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const float x = qvalid ? qv[16 * dc + 8 * g + s] : 0.f;
                const _Float16 h = (_Float16)x;
                qh[dc][s] = h;
                ql[dc][s] = (_Float16)(x - (float)h);
            }
        }
    }
    const int64_t kdim = (int64_t)a.n_kv * HD;
    const _Float16* kbase = a.kc + (int64_t)kvh * HD;
    v16f st[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int64_t p = slot0 + 32 * t + col;  // K row of this lane (< padded cap)
        const _Float16* krow = kbase + p * kdim;
        v16f acc = {};
#pragma unroll
        for (int dc = 0; dc < NDC; ++dc) {
            const v8h kf = *(const v8h*)(krow + 16 * dc + 8 * g);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qh[dc], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, ql[dc], acc, 0, 0, 0);
        }
        st[t] = acc;
    }
    // lane (q = col, g) holds S^T[slot 8(r/4) + 4g + r%4][q] of tile t
    const float scale = 1.f / sqrtf((float)HD);
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t ps = slot0 + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
            const bool ok = qvalid && slot_visible(a, npast, mq, ps);
            const float s = ok ? st[t][r] * scale : -INFINITY;
            st[t][r] = s;
            mx = fmaxf(mx, s);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float e = st[t][r] == -INFINITY ? 0.f : expf(st[t][r] - mx);
            st[t][r] = e;
            sum += e;
        }
    sum += __shfl_xor(sum, 32, 64);
    // O = P . V: A = P (rows q, k-slot 8g+s <-> tile slot 16hf + 8(s/4) + 4g + s%4)
    const _Float16* vbase = a.vt + (int64_t)kvh * HD * a.cap;
    v16f o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = v16f{};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            v8h ph, pl;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const float pv = st[t][8 * hf + s];
                const _Float16 h = (_Float16)pv;
                ph[s] = h;
                pl[s] = (_Float16)(pv - (float)h);
            }
            const int64_t sbase = slot0 + 32 * t + 16 * hf + 4 * g;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const _Float16* vrow = vbase + (int64_t)(32 * dt + col) * a.cap + sbase;
                const v4h v0 = *(const v4h*)vrow;
                const v4h v1 = *(const v4h*)(vrow + 8);
                const v8h vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, vf, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl, vf, o[dt], 0, 0, 0);
            }
        }
    // partials: per query row max / sum, and O rows
    const int nch = (int)gridDim.x;
    if (qvalid && g == 0) {
        const int64_t qi = (int64_t)mq * a.n_head + hq;
        a.pmax[qi * nch + c] = mx;
        a.psum[qi * nch + c] = sum;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int q = 8 * (r >> 2) + 4 * g + (r & 3);
        const int rr = blockIdx.z * 32 + q;
        if (rr < qrows) {
            const int64_t qi = (int64_t)(rr / gqa) * a.n_head + kvh * gqa + rr % gqa;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                a.pout[(qi * nch + c) * HD + 32 * dt + col] = o[dt][r];
        }
    }
}

// out[m][h*hd + d] = sum_c e^(max_c - M) O_c[d] / sum_c e^(max_c - M) sum_c
// one block per query row; the chunk weights are formed once in LDS so the
// output loop is a stream of independent loads
__global__ void __launch_bounds__(128) k_attn_combine(AttnMArgs a, int nch) {
    __shared__ float wsh[1024];  // chunk weights (nch <= 1024)
    __shared__ float red[128];
    const int64_t qi = blockIdx.x;  // m * n_head + h
    const int d = threadIdx.x;
    const int64_t npast = *a.npast;
    const int nvalid = (int)((npast + a.M + CH - 1) / CH);
    float M = -INFINITY;
    for (int c = d; c < nvalid; c += 128) M = fmaxf(M, a.pmax[qi * nch + c]);
    red[d] = M;
    __syncthreads();
    for (int o = 64; o > 0; o >>= 1) {
        if (d < o) red[d] = fmaxf(red[d], red[d + o]);
        __syncthreads();
    }
    M = red[0];
    __syncthreads();
    float den = 0.f;
    for (int c = d; c < nvalid; c += 128) {
        const float mc = a.pmax[qi * nch + c];
        const float w = mc == -INFINITY ? 0.f : expf(mc - M);
        wsh[c] = w;
        den += w * a.psum[qi * nch + c];
    }
    red[d] = den;
    __syncthreads();
    for (int o = 64; o > 0; o >>= 1) {
        if (d < o) red[d] += red[d + o];
        __syncthreads();
    }
    den = red[0];
    if (d < a.hd) {
        float num = 0.f;
#pragma unroll 8
        for (int c = 0; c < nvalid; ++c) num += wsh[c] * a.pout[(qi * nch + c) * a.hd + d];
        a.out[qi * a.hd + d] = num / den;
    }
}

}  // namespace

bool attn_mfma_supported(int64_t hd, int kv_f16, int64_t M, int64_t n_head, int64_t n_kv) {
    return kv_f16 && (hd == 64 || hd == 128) && M >= 1 && (M * (n_head / n_kv)) <= 32 * 16;
}

size_t attn_part_floats(int64_t M, int64_t n_head, int64_t hd, int64_t cap_alloc) {
    const int64_t nch = cap_alloc / CH;
    return (size_t)(M * n_head * nch) * (size_t)(hd + 2);
}

hipError_t launch_attn_mfma(hipStream_t st, AttnMArgs a, float* part) {
    const int nch = (int)(a.cap / CH);
    if (nch > 1024) return hipErrorInvalidValue;  // combine weights live in LDS
    const int64_t qi = (int64_t)a.M * a.n_head;
    a.pmax = part;
    a.psum = part + qi * nch;
    a.pout = part + 2 * qi * nch;
    const int gqa = a.n_head / a.n_kv;
    const int qtiles = (a.M * gqa + 31) / 32;
    dim3 grid((unsigned)nch, (unsigned)a.n_kv, (unsigned)qtiles);
    if (a.hd == 128)
        hipLaunchKernelGGL(k_attn_mfma<128>, grid, dim3(64), 0, st, a);
    else if (a.hd == 64)
        hipLaunchKernelGGL(k_attn_mfma<64>, grid, dim3(64), 0, st, a);
    else
        return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)qi), dim3(128), 0, st, a, nch);
    return hipGetLastError();
}
