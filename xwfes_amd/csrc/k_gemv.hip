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
    // four rows a pass: every load of the pass is issued before its
    // arithmetic (rows past the range read the last row with a zero factor)
    constexpr int RU = 4;
    for (int64_t ib = i0; ib < i1; ib += RU) {
        float w[RU][8], hv[RU][MT];
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            const int64_t i = ib + u < i1 ? ib + u : i1 - 1;
            dq8(W + i * row_bytes, dt, c * 8, N, w[u]);
#pragma unroll
            for (int m = 0; m < MT; ++m)
                hv[u][m] = (m < mc && ib + u < i1) ? h[(m0 + m) * ldh + i] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < RU; ++u)
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[m][k] += hv[u][m] * w[u][k];
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
    // split order (the loads issued ahead of the adds)
    constexpr int RB = 16;
    int64_t k = 0;
    for (; k + RB <= S; k += RB) {
        float p[RB];
#pragma unroll
        for (int u = 0; u < RB; ++u) p[u] = part[((k + u) * M + m) * N + j];
#pragma unroll
        for (int u = 0; u < RB; ++u) s += p[u];
    }
    for (; k < S; ++k) s += part[(k * M + m) * N + j];
    y[m * ldy + j] += s;
}

// ---------------------------------------------------------------- MFMA form
//
// The same row-dot on v_mfma_f32_16x16x32_f16 for any block dtype and any M:
// A = activations (16 rows per m-tile), B = dequantised weights (16 output
// rows), both split into fp16 hi + lo parts; hi*hi + hi*lo + lo*hi in fp32
// accumulators keeps the sum at fp32 accuracy (the dropped lo*lo term is
// 2^-22 of a product).  Inputs must lie within the fp16 range (the
// normalised activations, attention outputs and weights of the verify step).
// Workgroup: 16 output rows (and the matching up rows of a SwiGLU pair), all
// MTI m-tiles; its 8 waves split the contraction into eighths, each reading
// its activation fragments straight from global memory (L2-resident), and
// the slices are added in LDS in wave order.

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int GQ = 8;   // contraction slices (waves)
constexpr int GU = 2;   // 32-column steps whose loads are issued together
constexpr int GK = GQ * GU * 32;  // K must be a multiple of this

__device__ __forceinline__ void split8(const float* w, v8h_t& hi, v8h_t& lo) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const _Float16 h = (_Float16)w[i];
        hi[i] = h;
        lo[i] = (_Float16)(w[i] - (float)h);
    }
}

template <int MTI, bool PAIR>
__global__ void __launch_bounds__(64 * GQ) k_gemm_rows(Segs segs, const float* __restrict__ x,
                                                   int64_t ldx, int64_t K, int64_t M, int epi) {
    constexpr int NT = PAIR ? 2 : 1;
    __shared__ v4f_t red[GQ - 1][NT][MTI][64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int col = lane & 15, g = lane >> 4;
    const int64_t m0 = (int64_t)blockIdx.y * (MTI * 16);
    const int64_t total = PAIR ? segs.s[0].N : segs.start[segs.n];
    const int64_t R = (int64_t)blockIdx.x * 16 + col;  // this lane's weight row
    const bool rvalid = R < total;
    const int64_t Rc = rvalid ? R : total - 1;  // loads clamped to a valid row
    const uint8_t* wrow[NT];
    int wdt[NT];
    int si = 0;
    if (PAIR) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            wrow[t] = segs.s[t].W + Rc * segs.s[t].row_bytes;
            wdt[t] = segs.s[t].dt;
        }
    } else {
        while (Rc >= segs.start[si + 1]) ++si;
        wrow[0] = segs.s[si].W + (Rc - segs.start[si]) * segs.s[si].row_bytes;
        wdt[0] = segs.s[si].dt;
    }
    // activation rows of this lane (clamped; rows past M contribute zeros)
    const float* xr[MTI];
    float xf[MTI];
#pragma unroll
    for (int mt = 0; mt < MTI; ++mt) {
        const int64_t m = m0 + mt * 16 + col;
        xr[mt] = x + (m < M ? m : M - 1) * ldx;
        xf[mt] = m < M ? 1.f : 0.f;
    }
    v4f_t acc[NT][MTI];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MTI; ++mt) acc[t][mt] = v4f_t{0.f, 0.f, 0.f, 0.f};
    const int64_t kq = K / GQ, ka = w * kq, kb = ka + kq;
    for (int64_t k0 = ka; k0 < kb; k0 += GU * 32) {
        // every load of the GU steps first, weights then activations
        float wv[NT][GU][8];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int h = 0; h < GU; ++h) dq8(wrow[t], wdt[t], k0 + 32 * h + 8 * g, K, wv[t][h]);
        float4 xv[MTI][GU][2];
#pragma unroll
        for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
            for (int h = 0; h < GU; ++h) {
                const float* p = xr[mt] + k0 + 32 * h + 8 * g;
                xv[mt][h][0] = *(const float4*)p;
                xv[mt][h][1] = *(const float4*)(p + 4);
            }
#pragma unroll
        for (int h = 0; h < GU; ++h) {
            v8h_t bh[NT], bl[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) split8(wv[t][h], bh[t], bl[t]);
#pragma unroll
            for (int mt = 0; mt < MTI; ++mt) {
                const float4 a0 = xv[mt][h][0], a1 = xv[mt][h][1];
                const float av[8] = {a0.x * xf[mt], a0.y * xf[mt], a0.z * xf[mt], a0.w * xf[mt],
                                     a1.x * xf[mt], a1.y * xf[mt], a1.z * xf[mt], a1.w * xf[mt]};
                v8h_t ah, al;
                split8(av, ah, al);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[t], acc[t][mt], 0, 0, 0);
                    acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[t], acc[t][mt], 0, 0, 0);
                    acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[t], acc[t][mt], 0, 0, 0);
                }
            }
        }
    }
    // the slices added in wave order: waves 1..7 hand theirs to wave 0
    if (w > 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int mt = 0; mt < MTI; ++mt) red[w - 1][t][mt][lane] = acc[t][mt];
    }
    __syncthreads();
    if (w > 0 || !rvalid) return;
#pragma unroll
    for (int q = 0; q < GQ - 1; ++q)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int mt = 0; mt < MTI; ++mt) acc[t][mt] += red[q][t][mt][lane];
    // lane (col, g) holds C[4 g + r][col] of each m-tile
    if (PAIR) {
        const GemvSeg& sg = segs.s[0];
#pragma unroll
        for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + mt * 16 + 4 * g + r;
                if (m >= M) continue;
                const float gv = acc[0][mt][r], uv = acc[NT - 1][mt][r];
                // src/engine.cpp:271-273: g / (1 + exp(-g)) * u
                sg.y[m * sg.ldy + R] = gv / (1.f + expf(-gv)) * uv;
            }
    } else {
        const GemvSeg& sg = segs.s[si];
        const int64_t n = R - segs.start[si];
#pragma unroll
        for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + mt * 16 + 4 * g + r;
                if (m >= M) continue;
                float* yp = sg.y + m * sg.ldy + n;
                const float v = acc[0][mt][r];
                *yp = epi == EPI_ACCUM ? *yp + v : v;
            }
    }
}

template <bool PAIR>
hipError_t launch_gemm_rows(hipStream_t st, const Segs& s, int64_t rows, const float* x,
                            int64_t ldx, int64_t K, int64_t M, int epi) {
    const int mti = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    const dim3 grid((unsigned)((rows + 15) / 16), (unsigned)((M + 16 * mti - 1) / (16 * mti)));
    if (mti == 1)
        hipLaunchKernelGGL((k_gemm_rows<1, PAIR>), grid, dim3(64 * GQ), 0, st, s, x, ldx, K, M, epi);
    else if (mti == 2)
        hipLaunchKernelGGL((k_gemm_rows<2, PAIR>), grid, dim3(64 * GQ), 0, st, s, x, ldx, K, M, epi);
    else
        hipLaunchKernelGGL((k_gemm_rows<4, PAIR>), grid, dim3(64 * GQ), 0, st, s, x, ldx, K, M, epi);
    return hipGetLastError();
}

int64_t down_splits(int64_t M, int64_t n_in, int64_t N) {
    const int64_t groups = (N + 7) / 8;
    const int64_t mch = (M + MT - 1) / MT;
    // about 16k threads over the splits, at most 64 partials per output
    int64_t S = (16384 + groups * mch - 1) / (groups * mch);
    if (S > n_in) S = n_in;
    if (S > 64) S = 64;
    if (S < 1) S = 1;
    return S;
}

// the MFMA form needs K a multiple of 512 (whole steps in every slice) and
// 16-byte aligned activation rows; it runs for more than 8 activation rows,
// or for at least 16384 output rows (below that the one-wave-per-row kernel
// fills the device better)
bool gemm_rows_ok(const float* x, int64_t ldx, int64_t K, int64_t M, int64_t rows) {
    return K % GK == 0 && ldx % 4 == 0 && ((uintptr_t)x & 15) == 0 &&
           (M > 8 || rows >= 16384);
}

// planar copy of Q8_0 / Q4_0 rows: thread per (row, block)
__global__ void __launch_bounds__(256) k_planar(const uint8_t* __restrict__ src, int64_t nrows,
                                                int64_t nb, int qb, uint8_t* __restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nrows * nb) return;
    const int64_t r = t / nb, b = t % nb;
    const int64_t rb = nb * (2 + qb);
    const uint8_t* s = src + r * rb + b * (2 + qb);
    uint8_t* d = dst + r * rb;
    d[2 * b] = s[0];
    d[2 * b + 1] = s[1];
    for (int i = 0; i < qb; ++i) d[2 * nb + b * qb + i] = s[2 + i];
}

}  // namespace

int planar_dtype(int dt, int64_t ncols) {
    if (ncols % 128) return -1;
    return dt == FTX_Q8_0 ? FTX_Q8_0_PLANAR : (dt == FTX_Q4_0 ? FTX_Q4_0_PLANAR : -1);
}

hipError_t launch_planar(hipStream_t st, const uint8_t* src, int dt, int64_t nrows, int64_t ncols,
                         uint8_t* dst) {
    if (planar_dtype(dt, ncols) < 0) return hipErrorInvalidValue;
    const int64_t nb = ncols / 32, total = nrows * nb;
    const int qb = dt == FTX_Q8_0 ? 32 : 16;
    hipLaunchKernelGGL(k_planar, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, src,
                       nrows, nb, qb, dst);
    return hipGetLastError();
}

hipError_t launch_gemv(hipStream_t st, const GemvSeg* segs, int nseg, const float* x,
                       int64_t ldx, int64_t K, int64_t M, int epi, bool fp16_range) {
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
    if (fp16_range && gemm_rows_ok(x, ldx, K, M, rows))
        return launch_gemm_rows<false>(st, s, rows, x, ldx, K, M, epi);
    dim3 grid((unsigned)((rows + 3) / 4), (unsigned)((M + MT - 1) / MT));
    hipLaunchKernelGGL(k_gemv_rows, grid, dim3(256), 0, st, s, x, ldx, K, M, epi);
    return hipGetLastError();
}

hipError_t launch_gemv_swiglu(hipStream_t st, const uint8_t* Wg, const uint8_t* Wu, int dt,
                              int64_t row_bytes, int64_t N, const float* x, int64_t ldx,
                              int64_t K, int64_t M, float* h, int64_t ldh, bool fp16_range) {
    if (N == 0 || M == 0) return hipSuccess;
    if (fp16_range && gemm_rows_ok(x, ldx, K, M, N)) {
        Segs s{};
        s.n = 2;
        s.s[0] = GemvSeg{Wg, dt, row_bytes, N, h, ldh};
        s.s[1] = GemvSeg{Wu, dt, row_bytes, N, nullptr, 0};
        s.start[1] = N;
        s.start[2] = 2 * N;
        return launch_gemm_rows<true>(st, s, N, x, ldx, K, M, EPI_SWIGLU);
    }
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
    // blocks no wider than the column groups (small widths leave no idle lanes)
    const int bs = groups >= 256 ? 256 : (int)((groups + 63) / 64 * 64);
    dim3 grid((unsigned)((groups + bs - 1) / bs), (unsigned)S, (unsigned)((M + MT - 1) / MT));
    hipLaunchKernelGGL(k_down_part, grid, dim3(bs), 0, st, W, dt, row_bytes, n_in, N, h, ldh, M,
                       rows_per, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_down_reduce, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0, st,
                       part, S, M, N, y, ldy);
    return hipGetLastError();
}
