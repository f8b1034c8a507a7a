// k_gemv.hip -- generic quantised GEMV/GEMM kernels (any block dtype, any M).
//
// Row-dot form (y = x W^T, blocks along the contraction) follows
// CpuBackend::matmul (src/cpu_backend.cpp:90-104) with y[m*N + n] per row;
// column-axpy form (y += h W, blocks along the output) follows
// matmul_down_axpy (src/cpu_backend.cpp:60-75).  These are the general
// paths for every dtype; the MFMA kernels in k_mfma.hip take over the hot
// dtypes at small M.
#include "ftx_internal.h"
#include "quant_dev.h"

namespace {

constexpr int MT = 8;  // activation rows per pass

struct Segs {
    GemvSeg s[3];
    int64_t start[4];  // cumulative row starts
    int n;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// one wave per output row; lanes stride over groups of 8 elements
__global__ void __launch_bounds__(256) k_gemv_rows(Segs segs, const float* __restrict__ x,
                                                   int64_t ldx, int64_t K, int64_t M,
                                                   int epi) {
    const int lane = threadIdx.x & 63;
    const int64_t R = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (R >= segs.start[segs.n]) return;
    int si = 0;
    while (R >= segs.start[si + 1]) ++si;
    const GemvSeg sg = segs.s[si];
    const int64_t n = R - segs.start[si];
    const uint8_t* row = sg.W + n * sg.row_bytes;
    const int64_t ngroups = (K + 7) / 8;
    const int64_t m0 = (int64_t)blockIdx.y * MT;
    const int mc = (int)min((int64_t)MT, M - m0);
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.f;
    for (int64_t g = lane; g < ngroups; g += 64) {
        float w[8];
        dq8(row, sg.dt, g * 8, K, w);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < mc) {
                const float* xm = x + (m0 + m) * ldx + g * 8;
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (g * 8 + i < K) s += xm[i] * w[i];
                acc[m] += s;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = wave_sum(acc[m]);
    if (lane == 0) {
        for (int m = 0; m < mc; ++m) {
            float* yp = sg.y + (m0 + m) * sg.ldy + n;
            *yp = epi == EPI_ACCUM ? *yp + acc[m] : acc[m];
        }
    }
}

__global__ void __launch_bounds__(256) k_gemv_swiglu(const uint8_t* __restrict__ Wg,
                                                     const uint8_t* __restrict__ Wu, int dt,
                                                     int64_t row_bytes, int64_t N,
                                                     const float* __restrict__ x, int64_t ldx,
                                                     int64_t K, int64_t M,
                                                     float* __restrict__ h, int64_t ldh) {
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    const uint8_t* rg = Wg + n * row_bytes;
    const uint8_t* ru = Wu + n * row_bytes;
    const int64_t ngroups = (K + 7) / 8;
    const int64_t m0 = (int64_t)blockIdx.y * MT;
    const int mc = (int)min((int64_t)MT, M - m0);
    float ag[MT], au[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) ag[m] = au[m] = 0.f;
    for (int64_t g = lane; g < ngroups; g += 64) {
        float wg[8], wu[8];
        dq8(rg, dt, g * 8, K, wg);
        dq8(ru, dt, g * 8, K, wu);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < mc) {
                const float* xm = x + (m0 + m) * ldx + g * 8;
                float sg = 0.f, su = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (g * 8 + i < K) {
                        sg += xm[i] * wg[i];
                        su += xm[i] * wu[i];
                    }
                ag[m] += sg;
                au[m] += su;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        ag[m] = wave_sum(ag[m]);
        au[m] = wave_sum(au[m]);
    }
    if (lane == 0) {
        for (int m = 0; m < mc; ++m) {
            const float g = ag[m];
            // src/engine.cpp:271-273: g / (1 + exp(-g)) * u
            h[(m0 + m) * ldh + n] = g / (1.f + expf(-g)) * au[m];
        }
    }
}

// column-axpy partial sums: part[s][m][j] = sum_{i in split s} h[m,i] W[i,j]
__global__ void __launch_bounds__(256) k_down_part(const uint8_t* __restrict__ W, int dt,
                                                   int64_t row_bytes, int64_t n_in,
                                                   int64_t N, const float* __restrict__ h,
                                                   int64_t ldh, int64_t M, int64_t rows_per,
                                                   float* __restrict__ part) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // column group
    const int64_t ngroups = (N + 7) / 8;
    if (c >= ngroups) return;
    const int64_t s = blockIdx.y;
    const int64_t m0 = (int64_t)blockIdx.z * MT;
    const int mc = (int)min((int64_t)MT, M - m0);
    const int64_t i0 = s * rows_per, i1 = min(n_in, i0 + rows_per);
    float acc[MT][8];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[m][k] = 0.f;
    for (int64_t i = i0; i < i1; ++i) {
        float w[8];
        dq8(W + i * row_bytes, dt, c * 8, N, w);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < mc) {
                const float v = h[(m0 + m) * ldh + i];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[m][k] += v * w[k];
            }
        }
    }
    const int64_t S = gridDim.y;
    for (int m = 0; m < mc; ++m) {
        float* p = part + (s * M + m0 + m) * N + c * 8;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (c * 8 + k < N) p[k] = acc[m][k];
    }
    (void)S;
}

// y[m, j] += sum_s part[s][m][j] in split order
__global__ void __launch_bounds__(256) k_down_reduce(const float* __restrict__ part,
                                                     int64_t S, int64_t M, int64_t N,
                                                     float* __restrict__ y, int64_t ldy) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= M * N) return;
    const int64_t m = t / N, j = t % N;
    float s = 0.f;
    for (int64_t k = 0; k < S; ++k) s += part[(k * M + m) * N + j];
    y[m * ldy + j] += s;
}

int64_t down_splits(int64_t M, int64_t n_in, int64_t N) {
    const int64_t groups = (N + 7) / 8;
    const int64_t mch = (M + MT - 1) / MT;
    int64_t S = (65536 + groups * mch - 1) / (groups * mch);
    if (S > n_in) S = n_in;
    if (S > 256) S = 256;
    if (S < 1) S = 1;
    return S;
}

}  // namespace

hipError_t launch_gemv(hipStream_t st, const GemvSeg* segs, int nseg, const float* x,
                       int64_t ldx, int64_t K, int64_t M, int epi) {
    if (nseg < 1 || nseg > 3) return hipErrorInvalidValue;
    Segs s{};
    s.n = nseg;
    s.start[0] = 0;
    for (int i = 0; i < nseg; ++i) {
        s.s[i] = segs[i];
        s.start[i + 1] = s.start[i] + segs[i].N;
    }
    const int64_t rows = s.start[nseg];
    if (rows == 0 || M == 0) return hipSuccess;
    dim3 grid((unsigned)((rows + 3) / 4), (unsigned)((M + MT - 1) / MT));
    hipLaunchKernelGGL(k_gemv_rows, grid, dim3(256), 0, st, s, x, ldx, K, M, epi);
    return hipGetLastError();
}

hipError_t launch_gemv_swiglu(hipStream_t st, const uint8_t* Wg, const uint8_t* Wu, int dt,
                              int64_t row_bytes, int64_t N, const float* x, int64_t ldx,
                              int64_t K, int64_t M, float* h, int64_t ldh) {
    if (N == 0 || M == 0) return hipSuccess;
    dim3 grid((unsigned)((N + 3) / 4), (unsigned)((M + MT - 1) / MT));
    hipLaunchKernelGGL(k_gemv_swiglu, grid, dim3(256), 0, st, Wg, Wu, dt, row_bytes, N, x, ldx,
                       K, M, h, ldh);
    return hipGetLastError();
}

// floats of split-sum scratch that any M' <= M needs
size_t down_scratch_floats(int64_t M, int64_t n_in, int64_t N) {
    size_t best = 0;
    for (int64_t m = 1; m <= M; ++m) {
        const size_t need = (size_t)(down_splits(m, n_in, N) * m * N);
        if (need > best) best = need;
    }
    return best;
}

hipError_t launch_down(hipStream_t st, const uint8_t* W, int dt, int64_t row_bytes,
                       int64_t n_in, int64_t N, const float* h, int64_t ldh, int64_t M,
                       float* y, int64_t ldy, float* part) {
    if (M == 0 || N == 0 || n_in == 0) return hipSuccess;
    const int64_t S = down_splits(M, n_in, N);
    const int64_t rows_per = (n_in + S - 1) / S;
    const int64_t groups = (N + 7) / 8;
    dim3 grid((unsigned)((groups + 255) / 256), (unsigned)S, (unsigned)((M + MT - 1) / MT));
    hipLaunchKernelGGL(k_down_part, grid, dim3(256), 0, st, W, dt, row_bytes, n_in, N, h, ldh, M,
                       rows_per, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_down_reduce, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0, st,
                       part, S, M, N, y, ldy);
    return hipGetLastError();
}
