// k_down.hip -- ffn_down on MFMA for small M (M <= 8): y[m, j] += sum_i
// h[m, i] * W[i, j], with W in the reference orientation (n_ff rows of n_embd
// columns, quantisation blocks along the output j; src/cpu_backend.cpp:60-75).
//
// Along the contraction i every row carries its own scales, so they cannot be
// applied to an MFMA result; they are folded into the activation operand:
//   Q4_K  W[i,j] = d_i*sc_{i,s}*q_{i,j} - dmin_i*m_{i,s}     (s = j/32)
//     y[m,j] = sum_i (h[m,i]*d_i*sc_{i,s}) * q_{i,j}  -  sum_i h[m,i]*dmin_i*m_{i,s}
//   Q6_K  W[i,j] = d_i*sc_{i,s}*(q_{i,j} - 32)               (s = j/16)
// For each 32-row slice a workgroup (one 256-column super-block) builds
// A_s[m][i] = h[m,i]*d_i*sc_{i,s} for all its sub-blocks s in LDS, split into
// fp16 hi + lo parts (two MFMAs, ~22-bit operand), and the second sum with
// plain VALU FMAs.  The weights enter v_mfma_f32_16x16x32_f16 as exact small
// integers (q, or q - 32) from a re-tiled copy of the tensor whose byte
// order puts each lane's eight contraction slots in one 32-bit word.
//
// Tiled layouts (n_in rows, N columns; I = i/32, C = j/64, g = (i%32)/8,
// t = i%8, ct = (j%64)/16, col = j%16):
//   Q4_K  QS  [I][C][g][col][ct] x 4 B : byte t%4, nibble t/4 (q)
//         HDR [N/256][n_in] x 16 B     : d, dmin, 12 scale bytes (GGUF order)
//   Q6_K  QL  as QS (low 4 bits of q)
//         QH  [I][C][g][col][ct/2] x 4 B : byte t%4 holds, for the even ct,
//             bits 4-5 = q>>4 of slot t%4 and bits 6-7 of slot 4+t%4; the odd
//             ct the same in bits 0-3
//         SC  [N/256][n_in] x 16 int8,  D [N/256][n_in] x fp16
#include "ftx_internal.h"
#include "quant_dev.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

struct DownArgs {
    const uint8_t* qs;   // QS / QL plane
    const uint8_t* qh;   // Q6_K QH plane
    const uint8_t* hdr;  // Q4_K headers / Q6_K scales
    const uint8_t* d6;   // Q6_K d plane
    const float* h;      // [M][ldh]
    int64_t ldh;
    int M;
    int64_t n_in, N;
    int slices_per_split;
    float* part;         // [S][8][N]
};

// 8 nibbles (slot t: byte t%4, nibble t/4) -> 8 fp16 values q + bias
__device__ __forceinline__ v8h nib8_to_h(uint32_t w, float bias) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    // 0x64 in the high byte: fp16 1024 + q, exact
    const uint32_t p0 = __builtin_amdgcn_perm(lo, 0x64646464u, 0x00050004u);
    const uint32_t p1 = __builtin_amdgcn_perm(lo, 0x64646464u, 0x00070006u);
    const uint32_t p2 = __builtin_amdgcn_perm(hi, 0x64646464u, 0x00050004u);
    const uint32_t p3 = __builtin_amdgcn_perm(hi, 0x64646464u, 0x00070006u);
    const v2h b = {(_Float16)(-1024.f - bias), (_Float16)(-1024.f - bias)};
    const v2h h0 = __builtin_bit_cast(v2h, p0) + b, h1 = __builtin_bit_cast(v2h, p1) + b;
    const v2h h2 = __builtin_bit_cast(v2h, p2) + b, h3 = __builtin_bit_cast(v2h, p3) + b;
    return v8h{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// One workgroup = one 256-column super-block (wave w: columns 64w..64w+63)
// over a contiguous range of 32-row slices, processed in batches of NB
// slices: stage the batch's h and row scales (prefetched into registers one
// batch ahead), build the scaled fp16 hi/lo activation tables in LDS, then
// the MFMAs over the batch's weights (also prefetched one batch ahead).
template <int DT>
struct DownCfg {
    static constexpr int NS = DT == FTX_Q4_K ? 8 : 16;  // sub-blocks per super-block
    static constexpr int NB = 4;                         // slices per batch
};

template <int DT>
__global__ void __launch_bounds__(256) k_down_mfma(DownArgs a) {
    constexpr int NS = DownCfg<DT>::NS, NB = DownCfg<DT>::NB;
    // h / scale rows padded so 16-byte reads of different rows fall in
    // different LDS banks; the activation tables are stored [octet of rows]
    // [token][8 rows] so that one MFMA operand read covers consecutive bytes
    constexpr int HP = NB * 32 + 4;
    __shared__ float hs[8][HP];
    __shared__ float dsc[NS][HP];  // [sub-block][row of the batch]
    __shared__ float dmn[DT == FTX_Q4_K ? 8 : 1][HP];
    __shared__ _Float16 ahi[NB][NS][4][8][8];
    __shared__ _Float16 alo[NB][NS][4][8][8];
    __shared__ float mpart[4][8][8];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t sbc = blockIdx.x, split = blockIdx.y;
    const int64_t nc64 = a.N / 64, nsl = a.n_in / 32;
    const int64_t I0 = split * a.slices_per_split;
    const int64_t I1 = min(I0 + a.slices_per_split, nsl);
    const int col = lane & 15, g = lane >> 4;
    const int64_t c64 = sbc * 4 + w;
    v4f acc[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
    float mt = 0.f;  // Q4_K min term of this thread's (s, m)
    // ---- per-batch register prefetch: h (thread: m = tid / 32, row tid % 32
    // of each slice), the row header (threads < NB * 32), the weights (lane)
    float hp[NB];
    v4i hdp = {0, 0, 0, 0};
    uint16_t d6p = 0;
    v4i wq[NB], wqn[NB];
    int2 wh[NB], whn[NB];
    auto slice_of = [&](int64_t I) { return I < I1 ? I : I1 - 1; };  // clamped for loads
    auto load_hs = [&](int64_t Ib) {
        const int m = tid >> 5, ii = tid & 31;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int64_t I = Ib + b;
            hp[b] = (m < a.M && I < I1) ? a.h[(int64_t)m * a.ldh + I * 32 + ii] : 0.f;
        }
        if (tid < NB * 32) {
            const int64_t i = slice_of(Ib + tid / 32) * 32 + tid % 32;
            hdp = *(const v4i*)(a.hdr + (sbc * a.n_in + i) * 16);
            if (DT == FTX_Q6_K) d6p = *(const uint16_t*)(a.d6 + (sbc * a.n_in + i) * 2);
        }
    };
    auto load_w = [&](int64_t Ib, v4i* q, int2* qh) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int64_t blk = (slice_of(Ib + b) * nc64 + c64) * 4 + g;
            q[b] = *(const v4i*)(a.qs + (blk * 16 + col) * 16);
            if (DT == FTX_Q6_K) qh[b] = *(const int2*)(a.qh + (blk * 16 + col) * 8);
        }
    };
    load_hs(I0);
    load_w(I0, wq, wh);
    for (int64_t Ib = I0; Ib < I1; Ib += NB) {
        __syncthreads();  // the previous batch is done with the LDS tables
        // ---- stage h and the per-row scales of this batch
        {
            const int m = tid >> 5, ii = tid & 31;
#pragma unroll
            for (int b = 0; b < NB; ++b) hs[m][b * 32 + ii] = hp[b];
        }
        if (tid < NB * 32) {
            if (DT == FTX_Q4_K) {
                const float d = h2f((uint16_t)((uint32_t)hdp.x & 0xFFFF));
                const float dm = h2f((uint16_t)((uint32_t)hdp.x >> 16));
                const uint32_t S0 = hdp.y, S1 = hdp.z, S2 = hdp.w;
                const uint32_t sc_lo = S0 & 0x3F3F3F3Fu, mn_lo = S1 & 0x3F3F3F3Fu;
                const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
                const uint32_t mn_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const uint32_t scw = s < 4 ? sc_lo : sc_hi, mnw = s < 4 ? mn_lo : mn_hi;
                    dsc[s][tid] = d * (float)((scw >> (8 * (s & 3))) & 0xFF);
                    dmn[s][tid] = dm * (float)((mnw >> (8 * (s & 3))) & 0xFF);
                }
            } else {
                const float d = h2f(d6p);
                const uint32_t* scw = (const uint32_t*)&hdp;
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    dsc[s][tid] = d * (float)(int8_t)((scw[s >> 2] >> (8 * (s & 3))) & 0xFF);
            }
        }
        // next batch's h and headers in flight from here
        if (Ib + NB < I1) load_hs(Ib + NB);
        __syncthreads();
        // ---- A_s[m][i] = h * d * sc as fp16 hi + lo, for every slice of the batch
        {
            const int oct = tid >> 6, m = tid & 7, sp = (tid >> 3) & 7;
#pragma unroll 1
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int rep = 0; rep < NS / 8; ++rep) {
                    const int s = sp * (NS / 8) + rep;
                    const int i0 = b * 32 + oct * 8;
                    // eight rows at once: two 16-byte LDS reads per table
                    const v4f h0 = *(const v4f*)&hs[m][i0], h1 = *(const v4f*)&hs[m][i0 + 4];
                    const v4f f0 = *(const v4f*)&dsc[s][i0], f1 = *(const v4f*)&dsc[s][i0 + 4];
                    const float hv[8] = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
                    const float fv[8] = {f0[0], f0[1], f0[2], f0[3], f1[0], f1[1], f1[2], f1[3]};
                    _Float16 ph[8], pl[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const float p = hv[k] * fv[k];
                        const _Float16 hi = (_Float16)p;
                        ph[k] = hi;
                        pl[k] = (_Float16)(p - (float)hi);
                    }
                    if (DT == FTX_Q4_K) {
                        const v4f n0 = *(const v4f*)&dmn[s][i0], n1 = *(const v4f*)&dmn[s][i0 + 4];
                        const float nv[8] = {n0[0], n0[1], n0[2], n0[3], n1[0], n1[1], n1[2], n1[3]};
#pragma unroll
                        for (int k = 0; k < 8; ++k) mt += hv[k] * nv[k];
                    }
                    *(v8h*)&ahi[b][s][oct][m][0] =
                        v8h{ph[0], ph[1], ph[2], ph[3], ph[4], ph[5], ph[6], ph[7]};
                    *(v8h*)&alo[b][s][oct][m][0] =
                        v8h{pl[0], pl[1], pl[2], pl[3], pl[4], pl[5], pl[6], pl[7]};
                }
            }
        }
        __syncthreads();
        // next batch's weights in flight during this batch's MFMAs
        if (Ib + NB < I1) load_w(Ib + NB, wqn, whn);
        // ---- MFMA: this wave's 64 columns (4 tiles of 16) over the batch's rows
        const int arow = lane & 15;  // A row (token m; rows 8..15 are zero)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const uint32_t* qw = (const uint32_t*)&wq[b];
            const uint32_t qhw[2] = {(uint32_t)wh[b].x, (uint32_t)wh[b].y};
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                v8h bv;
                if (DT == FTX_Q4_K) {
                    bv = nib8_to_h(qw[ct], 0.f);
                } else {
                    const uint32_t X = qhw[ct >> 1];
                    const uint32_t hl = (ct & 1) ? (X << 4) & 0x30303030u : X & 0x30303030u;
                    const uint32_t hh = (ct & 1) ? (X << 2) & 0x30303030u : (X >> 2) & 0x30303030u;
                    const uint32_t L = qw[ct];
                    const uint32_t vlo = (L & 0x0F0F0F0Fu) | hl;
                    const uint32_t vhi = ((L >> 4) & 0x0F0F0F0Fu) | hh;
                    // 6-bit values: place as (lo nibble word, hi nibble word)
                    const uint32_t p0 = __builtin_amdgcn_perm(vlo, 0x64646464u, 0x00050004u);
                    const uint32_t p1 = __builtin_amdgcn_perm(vlo, 0x64646464u, 0x00070006u);
                    const uint32_t p2 = __builtin_amdgcn_perm(vhi, 0x64646464u, 0x00050004u);
                    const uint32_t p3 = __builtin_amdgcn_perm(vhi, 0x64646464u, 0x00070006u);
                    const v2h bb = {(_Float16)(-1056.f), (_Float16)(-1056.f)};
                    const v2h h0 = __builtin_bit_cast(v2h, p0) + bb, h1 = __builtin_bit_cast(v2h, p1) + bb;
                    const v2h h2 = __builtin_bit_cast(v2h, p2) + bb, h3 = __builtin_bit_cast(v2h, p3) + bb;
                    bv = v8h{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
                }
                const int s = DT == FTX_Q4_K ? (w * 64 + ct * 16) / 32 : (w * 64 + ct * 16) / 16;
                v8h ah = {}, al = {};
                if (arow < 8) {
                    ah = *(const v8h*)&ahi[b][s][g][arow][0];
                    al = *(const v8h*)&alo[b][s][g][arow][0];
                }
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bv, acc[ct], 0, 0, 0);
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bv, acc[ct], 0, 0, 0);
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            wq[b] = wqn[b];
            if (DT == FTX_Q6_K) wh[b] = whn[b];
        }
    }
    // ---- min term per (s, m), summed over the four row octets
    if (DT == FTX_Q4_K) {
        mpart[tid >> 6][(tid >> 3) & 7][tid & 7] = mt;
        __syncthreads();
    }
    // lane (col, g) holds C[row 4g + r][col]; rows 0..7 are the tokens
    if (g < 2) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int64_t j = sbc * 256 + w * 64 + ct * 16 + col;
            const int s = (w * 64 + ct * 16) / 32;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * g + r;
                float v = acc[ct][r];
                if (DT == FTX_Q4_K)
                    v -= mpart[0][s][m] + mpart[1][s][m] + mpart[2][s][m] + mpart[3][s][m];
                a.part[(split * 8 + m) * a.N + j] = v;
            }
        }
    }
}

// ---- re-tiling from the resident row layout.  One thread per (8-row
// octet, super-block): the octet's eight rows are exactly the eight slots
// packed into each QS / QH byte, so every byte has a single writer.
__global__ void __launch_bounds__(256) k_down_tile(const uint8_t* __restrict__ src,
                                                   int64_t src_row_bytes, int dt, int64_t n_in,
                                                   int64_t N, uint8_t* __restrict__ qs,
                                                   uint8_t* __restrict__ qh,
                                                   uint8_t* __restrict__ hdr,
                                                   uint8_t* __restrict__ d6) {
    const int64_t nsb = N / 256;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (n_in / 8) * nsb) return;
    const int64_t oct = t / nsb, sb = t % nsb;
    const int64_t nc64 = N / 64;
    for (int64_t i = oct * 8; i < oct * 8 + 8; ++i) {
    const uint8_t* row = src + i * src_row_bytes;
    const int64_t I = i / 32;
    const int ii = (int)(i % 32), g = ii / 8, tt = ii % 8;
    // element (i, j) of this super-block -> its nibble / 2-bit slots
    for (int e = 0; e < 256; e += 8) {
        for (int k = 0; k < 8; ++k) {
            const int64_t j = sb * 256 + e + k;
            int q;  // 4-bit (Q4_K) or 6-bit (Q6_K) value
            if (dt == FTX_Q4_K) {
                const uint8_t* p = row + sb * 144;
                const int r = e + k, jj = r >> 5, l = r & 31;
                const uint8_t b = p[16 + 32 * (jj >> 1) + l];
                q = (jj & 1) ? (b >> 4) : (b & 0xF);
            } else {
                const int r = e + k, c = r >> 7, rr = r & 127, kk = rr >> 5, l = rr & 31;
                const uint8_t lb = row[sb * 128 + q6k_ql_dev(64 * c + 32 * (kk & 1) + l)];
                const uint8_t hb = row[nsb * 128 + sb * 64 + q6k_qh_dev(32 * c + l)];
                const int lo = (kk >> 1) ? (lb >> 4) : (lb & 0xF);
                const int hi = (hb >> (2 * kk)) & 3;
                q = lo | (hi << 4);
            }
            const int64_t C = j / 64;
            const int ct = (int)((j % 64) / 16), cl = (int)(j % 16);
            const int64_t blk = (I * nc64 + C) * 4 + g;
            const int64_t word = (blk * 16 + cl) * 4 + ct;
            uint8_t* qb = qs + word * 4 + (tt & 3);
            // each byte is written by exactly one thread (one row, one column pair)
            if (tt < 4) *qb = (uint8_t)((*qb & 0xF0) | (q & 0xF));
            else *qb = (uint8_t)((*qb & 0x0F) | ((q & 0xF) << 4));
            if (dt == FTX_Q6_K) {
                const int h2 = (q >> 4) & 3;
                uint8_t* hb = qh + ((blk * 16 + cl) * 2 + (ct >> 1)) * 4 + (tt & 3);
                const int sh = ((ct & 1) ? 0 : 4) + ((tt >= 4) ? 2 : 0);
                *hb = (uint8_t)((*hb & ~(3 << sh)) | (h2 << sh));
            }
        }
    }
    if (dt == FTX_Q4_K) {
        const uint8_t* p = row + sb * 144;
        for (int k = 0; k < 16; ++k) hdr[(sb * n_in + i) * 16 + k] = p[k];
    } else {
        for (int k = 0; k < 16; ++k) hdr[(sb * n_in + i) * 16 + k] = row[nsb * 192 + sb * 16 + k];
        d6[(sb * n_in + i) * 2] = row[nsb * 208 + sb * 2];
        d6[(sb * n_in + i) * 2 + 1] = row[nsb * 208 + sb * 2 + 1];
    }
    }
}

}  // namespace

bool down_mfma_supported(int dt, int64_t n_in, int64_t N, int64_t M) {
    return (dt == FTX_Q4_K || dt == FTX_Q6_K) && M >= 1 && M <= 8 && n_in % 32 == 0 &&
           N % 256 == 0;
}

size_t down_tiled_bytes(int dt, int64_t n_in, int64_t N) {
    const int64_t nsb = N / 256;
    if (dt == FTX_Q4_K) return (size_t)(n_in * N / 2 + n_in * nsb * 16);
    return (size_t)(n_in * N / 2 + n_in * N / 4 + n_in * nsb * 16 + n_in * nsb * 2);
}

// plane offsets inside a tiled buffer
static void down_planes(int dt, int64_t n_in, int64_t N, uint8_t* base, uint8_t** qs,
                        uint8_t** qh, uint8_t** hdr, uint8_t** d6) {
    const int64_t nsb = N / 256;
    *qs = base;
    if (dt == FTX_Q4_K) {
        *qh = nullptr;
        *hdr = base + n_in * N / 2;
        *d6 = nullptr;
    } else {
        *qh = base + n_in * N / 2;
        *hdr = *qh + n_in * N / 4;
        *d6 = *hdr + n_in * nsb * 16;
    }
}

hipError_t launch_down_tile(hipStream_t st, const uint8_t* src, int64_t src_row_bytes, int dt,
                            int64_t n_in, int64_t N, uint8_t* dst) {
    uint8_t *qs, *qh, *hdr, *d6;
    down_planes(dt, n_in, N, dst, &qs, &qh, &hdr, &d6);
    hipError_t e = hipMemsetAsync(dst, 0, down_tiled_bytes(dt, n_in, N), st);
    if (e != hipSuccess) return e;
    const int64_t total = (n_in / 8) * (N / 256);
    hipLaunchKernelGGL(k_down_tile, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, src,
                       src_row_bytes, dt, n_in, N, qs, qh, hdr, d6);
    return hipGetLastError();
}

size_t down_mfma_part_floats(int64_t n_in, int64_t N, int cu_count) {
    (void)cu_count;
    (void)n_in;
    return (size_t)64 * 8 * N;
}

hipError_t launch_down_mfma(hipStream_t st, int dt, const uint8_t* tiled, int64_t n_in, int64_t N,
                            const float* h, int64_t ldh, int64_t M, float* y, int64_t ldy,
                            float* part, int cu_count, int* splits) {
    DownArgs a{};
    uint8_t *qs, *qh, *hdr, *d6;
    down_planes(dt, n_in, N, (uint8_t*)tiled, &qs, &qh, &hdr, &d6);
    a.qs = qs;
    a.qh = qh;
    a.hdr = hdr;
    a.d6 = d6;
    a.h = h;
    a.ldh = ldh;
    a.M = (int)M;
    a.n_in = n_in;
    a.N = N;
    const int64_t nslices = n_in / 32, nsb = N / 256;
    // splits of the contraction: as many workgroups as fit the CUs at once
    // (LDS: three Q4_K or two Q6_K workgroups per CU), at most 64, each a
    // whole number of slice batches
    const int NB = dt == FTX_Q4_K ? DownCfg<FTX_Q4_K>::NB : DownCfg<FTX_Q6_K>::NB;
    const int64_t per_cu = dt == FTX_Q4_K ? 3 : 2;
    int64_t S = (per_cu * (int64_t)(cu_count > 0 ? cu_count : 256) + nsb - 1) / nsb;
    if (S > 64) S = 64;
    if (S > nslices) S = nslices;
    if (S < 1) S = 1;
    int64_t spp = (nslices + S - 1) / S;
    spp = (spp + NB - 1) / NB * NB;
    a.slices_per_split = (int)spp;
    S = (nslices + spp - 1) / spp;
    a.part = part;
    const dim3 grid((unsigned)nsb, (unsigned)S);
    if (dt == FTX_Q4_K)
        hipLaunchKernelGGL(k_down_mfma<FTX_Q4_K>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(k_down_mfma<FTX_Q6_K>, grid, dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (splits) {
        *splits = (int)S;
        return hipSuccess;
    }
    return launch_part_reduce(st, part, (int)S, N, M, y, ldy);
}
