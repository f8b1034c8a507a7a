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
#include "mm_dev.h"
#include "quant_dev.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
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

// fp16 pairs 1024 + q (p[i] = slots 2i, 2i + 1) -> x q per slot, exact: one
// fused multiply-add (1024 + q) x + (-1024 x) per pair
__device__ __forceinline__ v8h fma8(const v2h* p, const v8h& x, const v8h& nx) {
    v2h r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = __builtin_elementwise_fma(p[i], v2h{x[2 * i], x[2 * i + 1]}, v2h{nx[2 * i], nx[2 * i + 1]});
    return v8h{r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1], r[3][0], r[3][1]};
}

// 8 nibbles (slot t: byte t%4, nibble t/4) -> 8 fp16 values sc_t q_t, exact
__device__ __forceinline__ v8h nib8_fma(uint32_t w, const v8h& sc, const v8h& sn) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    v2h p[4];
    p[0] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(lo, 0x64646464u, 0x00050004u));
    p[1] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(lo, 0x64646464u, 0x00070006u));
    p[2] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(hi, 0x64646464u, 0x00050004u));
    p[3] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(hi, 0x64646464u, 0x00070006u));
    return fma8(p, sc, sn);
}

// One workgroup = one 256-column super-block over a contiguous range of
// 32-row slices, in batches of NB slices.  The
// row factors are split from the sub-block scales:
//   Q4_K  y[m,j] = sum_i (h d)[m,i] * (sc_{i,s} q_{i,j}) - sum_i (h dmin)[m,i] * m_{i,s}
//   Q6_K  y[m,j] = sum_i (16 h d)[m,i] * (sh_{i,s} q_{i,j}) + sum_i (h d)[m,i] * (sl_{i,s} q_{i,j})
//                  - 32 sum_i (h d)[m,i] * sc_{i,s}          (sc = 16 sh + sl, 0 <= sl < 16)
// so the activation operand (h d, and h dmin) is shared by every sub-block
// of the super-block and built once per slice per workgroup, as fp16 hi
// (A rows 0..7, the tokens) + lo (rows 8..15) parts; the weight operand is
// the integer sc * q (|.| <= 945, exact in fp16); the Q4_K min term and the
// Q6_K -32 sc term are one more MFMA per slice, with the sub-block scales as
// the B columns.  Per batch the workgroup builds the next batch's operands
// into a double-buffered LDS stage (threads 0..127 the activation tables,
// 128..255 the fp16 scale tables) while the waves run the current batch's
// MFMAs; one barrier per batch.  The weights of the next batches are in
// flight in a register ring (the loop is unrolled by the ring size so that
// no ring slot is copied).
template <int DT>
struct DownCfg {
    static constexpr int NS = DT == FTX_Q4_K ? 8 : 16;  // sub-blocks per super-block
    static constexpr int NB = 4;                         // slices per batch
    static constexpr int RP = NB * 32 + 8;               // padded scale-table row (halves)
    // weight register ring: batches of weights in flight ahead of the one
    // computed is RING - 1 (Q6_K's larger words take one slot less, which
    // keeps it within 128 VGPRs, four waves per SIMD)
    static constexpr int RING = DT == FTX_Q4_K ? 3 : 2;
};
// the activation operands are formed as (h d) * 2^10 so that their fp16 lo
// parts stay clear of the subnormal range (an exact power of two, undone on
// the outputs); |h d| < 64 keeps the hi parts finite, |h d| < 4 for Q6_K,
// whose sh term takes the operand times 16 (Q6_K d is at most max|w| / 4064)
constexpr float DOWN_ASCALE = 1024.f;

// 8 waves: wave w takes columns 64 (w % 4) .. + 63 and, of each batch, the
// slices 2 (w / 4) and 2 (w / 4) + 1; the two slice groups' outputs are added
// in LDS at the end (wave order)
constexpr int DOWN_WAVES = 8;
constexpr int DOWN_SPW = 2;  // slices of a batch per wave

template <int DT>
struct DownW {
    v4i q[DOWN_SPW];                        // QS / QL words of the lane
    int2 h[DT == FTX_Q6_K ? DOWN_SPW : 1];  // Q6_K QH words
};

// prefetched inputs of one batch's stage: thread t owns rows 2q, 2q+1 of the
// batch (q = t / 8) and index e = t % 8 (token for the activation tables,
// sub-block (and e + 8) for the scale tables); hv = h of token e on those
// rows, r[k] = the header of row 2q + k, dd = (Q6_K) their d words.  Every
// thread issues the same loads and runs the same straight-line code, so no
// divergent branch sits between a load and its use (the compiler's
// vector-memory waits stay exact and the weights in flight are not drained).
struct DownStageIn {
    int2 hv;
    v4i r[2];
    uint32_t dd;
};

template <int DT>
__global__ void __launch_bounds__(64 * DOWN_WAVES) __attribute__((amdgpu_waves_per_eu(4)))
k_down_mfma(DownArgs a) {
    constexpr int NS = DownCfg<DT>::NS, NB = DownCfg<DT>::NB, RP = DownCfg<DT>::RP;
    constexpr int NT = DT == FTX_Q4_K ? 2 : 1;  // activation tables: h d (, h dmin)
    // scale tables: sc, m, -1024 sc | sh, sl, sc, -1024 sh, -1024 sl (the
    // negated ones complete (1024 + q) x + (-1024 x) = q x in one fused
    // multiply-add per pair); TSUB = the sub-block term's B columns
    constexpr int NC = DT == FTX_Q4_K ? 3 : 5;
    constexpr int TSUB = DT == FTX_Q4_K ? 1 : 2;
    __shared__ _Float16 tab[2][NT][NB][4][16][8];  // [buf][table][slice][k octet][A row][8]
    __shared__ _Float16 sct[2][NC][NS][RP];        // [buf][table][sub-block][row]
    __shared__ float red[4][16][64];              // slice group 1's outputs
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
    const int cw = w & 3, sgp = w >> 2;  // column quarter, slice group
    const int64_t sbc = blockIdx.x, split = blockIdx.y;
    const int64_t nc64 = a.N / 64, nsl = a.n_in / 32;
    const int64_t I0 = split * a.slices_per_split;
    const int64_t I1 = min(I0 + a.slices_per_split, nsl);
    const int col = lane & 15, g = lane >> 4;
    const int64_t c64 = sbc * 4 + cw;
    v4f acc[4], accs;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
    accs = v4f{0.f, 0.f, 0.f, 0.f};
    auto slice_of = [&](int64_t I) { return I < I1 ? I : I1 - 1; };  // clamped for loads
    const int sq = tid >> 3, se = tid & 7;  // rows 2 sq, 2 sq + 1 of the batch
    const int hm = se < a.M ? se : 0;       // token row of h (masked in stage)
    DownStageIn si;
    auto load_stage = [&](int64_t Ib) {
        const int64_t i0 = slice_of(Ib + sq / 16) * 32 + (sq % 16) * 2;
        si.hv = *(const int2*)(a.h + (int64_t)hm * a.ldh + i0);
#pragma unroll
        for (int k = 0; k < 2; ++k) si.r[k] = *(const v4i*)(a.hdr + (sbc * a.n_in + i0 + k) * 16);
        if constexpr (DT == FTX_Q6_K) si.dd = *(const uint32_t*)(a.d6 + (sbc * a.n_in + i0) * 2);
    };
    auto stage = [&](int64_t Ib, int buf) {
        const int b = sq / 16, g8 = (sq / 4) % 4, k0 = (sq % 4) * 2;  // slice, k octet, first of 2
        // activation tables: token se, 2 rows; h of tokens past M or of
        // slices past the range is zero
        // (a 0 / 1 factor, not a select: keeps the block free of branches)
        const float lf = (float)((se < a.M) & (Ib + b < I1));
        const float2 h2 = __builtin_bit_cast(float2, si.hv);
        const float hv2[2] = {h2.x * lf, h2.y * lf};
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float p[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                uint32_t dw;
                if constexpr (DT == FTX_Q4_K)
                    dw = (uint32_t)si.r[k].x >> (16 * t);  // d | dmin << 16
                else
                    dw = si.dd >> (16 * k);
                p[k] = hv2[k] * h2f((uint16_t)(dw & 0xFFFF)) * DOWN_ASCALE;
            }
            v2h ph, pl;
            split_hl2(p[0], p[1], ph, pl);
            *(v2h*)&tab[buf][t][b][g8][se][k0] = ph;
            *(v2h*)&tab[buf][t][b][g8][8 + se][k0] = pl;
        }
        // scale tables: sub-block se (Q6_K also se + 8), 2 rows
        const int r0 = sq * 2;
        if constexpr (DT == FTX_Q4_K) {
            // 6-bit scale / min of sub-block se (GGUF K-quant packing)
            const int sh = 8 * (se & 3);
            v2h sc, mn;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t S0 = si.r[k].y, S1 = si.r[k].z, S2 = si.r[k].w;
                const uint32_t sc_lo = (S0 >> sh) & 0x3F, mn_lo = (S1 >> sh) & 0x3F;
                const uint32_t sc_hi = ((S2 >> sh) & 0x0F) | (((S0 >> sh) >> 2) & 0x30);
                const uint32_t mn_hi = ((S2 >> sh) >> 4 & 0x0F) | (((S1 >> sh) >> 2) & 0x30);
                sc[k] = (_Float16)(float)(se < 4 ? sc_lo : sc_hi);
                mn[k] = (_Float16)(float)(se < 4 ? mn_lo : mn_hi);
            }
            *(v2h*)&sct[buf][0][se][r0] = sc;
            *(v2h*)&sct[buf][1][se][r0] = mn;
            *(v2h*)&sct[buf][2][se][r0] = sc * v2h{(_Float16)(-1024.f), (_Float16)(-1024.f)};
        } else {
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int sb = se + 8 * h2;
                v2h vh, vl, vc;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int sc = (int)(int8_t)(((uint32_t)si.r[k][sb >> 2] >> (8 * (sb & 3))) & 0xFF);
                    vh[k] = (_Float16)(float)(sc >> 4);  // sc = 16 sh + sl
                    vl[k] = (_Float16)(float)(sc & 15);
                    vc[k] = (_Float16)(float)sc;
                }
                const v2h m1024 = {(_Float16)(-1024.f), (_Float16)(-1024.f)};
                *(v2h*)&sct[buf][0][sb][r0] = vh;
                *(v2h*)&sct[buf][1][sb][r0] = vl;
                *(v2h*)&sct[buf][2][sb][r0] = vc;
                *(v2h*)&sct[buf][3][sb][r0] = vh * m1024;
                *(v2h*)&sct[buf][4][sb][r0] = vl * m1024;
            }
        }
    };
    auto load_w = [&](int64_t Ib, DownW<DT>& o) {
#pragma unroll
        for (int bb = 0; bb < DOWN_SPW; ++bb) {
            const int64_t blk = (slice_of(Ib + sgp * DOWN_SPW + bb) * nc64 + c64) * 4 + g;
            o.q[bb] = *(const v4i*)(a.qs + (blk * 16 + col) * 16);
            if constexpr (DT == FTX_Q6_K) o.h[bb] = *(const int2*)(a.qh + (blk * 16 + col) * 8);
        }
    };
    // MFMAs of slice b = 2 sgp + bb of the staged batch in buf
    auto mfma = [&](int buf, const DownW<DT>& wt, int bb) {
        const int b = sgp * DOWN_SPW + bb;
        const uint32_t* qw = (const uint32_t*)&wt.q[bb];
        const int r0 = b * 32 + 8 * g;
        const v8h av = *(const v8h*)&tab[buf][0][b][g][col][0];
        // Q6_K: sc q = 16 sh q + sl q with both products exact in fp16; the
        // 16 goes on the activation operand (exact), one accumulator
        const v8h av16 = av * (_Float16)16.f;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            if constexpr (DT == FTX_Q4_K) {
                const int s = 2 * cw + (ct >> 1);
                const v8h sc = *(const v8h*)&sct[buf][0][s][r0];
                const v8h sn = *(const v8h*)&sct[buf][2][s][r0];
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, nib8_fma(qw[ct], sc, sn), acc[ct], 0,
                                                                 0, 0);
            } else {
                const uint32_t X = ct < 2 ? (uint32_t)wt.h[bb].x : (uint32_t)wt.h[bb].y;
                const uint32_t hl = (ct & 1) ? (X << 4) & 0x30303030u : X & 0x30303030u;
                const uint32_t hh = (ct & 1) ? (X << 2) & 0x30303030u : (X >> 2) & 0x30303030u;
                const uint32_t L = qw[ct];
                const uint32_t vlo = (L & 0x0F0F0F0Fu) | hl;
                const uint32_t vhi = ((L >> 4) & 0x0F0F0F0Fu) | hh;
                // 6-bit q as (lo nibble word, hi nibble word) -> fp16 1024 + q
                v2h p[4];
                p[0] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(vlo, 0x64646464u, 0x00050004u));
                p[1] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(vlo, 0x64646464u, 0x00070006u));
                p[2] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(vhi, 0x64646464u, 0x00050004u));
                p[3] = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(vhi, 0x64646464u, 0x00070006u));
                const int s = 4 * cw + ct;
                const v8h sh = *(const v8h*)&sct[buf][0][s][r0];
                const v8h sl = *(const v8h*)&sct[buf][1][s][r0];
                const v8h nh = *(const v8h*)&sct[buf][3][s][r0];
                const v8h nl = *(const v8h*)&sct[buf][4][s][r0];
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av16, fma8(p, sh, nh), acc[ct], 0, 0, 0);
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, fma8(p, sl, nl), acc[ct], 0, 0, 0);
            }
        }
        // sub-block term: B column col = sub-block (Q4_K: rows of m, with the
        // h dmin operand; Q6_K: sc, with the h d operand)
        const v8h as = DT == FTX_Q4_K ? *(const v8h*)&tab[buf][NT - 1][b][g][col][0] : av;
        v8h bsv = *(const v8h*)&sct[buf][TSUB][col % NS][r0];
        if (col >= NS) bsv = v8h{};
        accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(as, bsv, accs, 0, 0, 0);
    };
    // One batch: the next batch's stage into the other buffer, the stage
    // inputs two batches ahead and the weights RING - 1 ahead (stage inputs
    // first), then the MFMAs of the staged batch.  Vector-memory counters
    // retire in issue order, so each wait (stage inputs of the next batch,
    // weights of this one) covers only loads issued before it.  (Loads past
    // the range re-read its last slice, so that every batch issues the same
    // loads.)
    constexpr int RING = DownCfg<DT>::RING;
    auto batch = [&](int64_t Ib, int buf, DownW<DT>& cur, DownW<DT>& fill) {
        stage(Ib + NB, buf ^ 1);
        load_stage(Ib + 2 * NB);
        load_w(Ib + (RING - 1) * NB, fill);
#pragma unroll
        for (int bb = 0; bb < DOWN_SPW; ++bb) {
            if (Ib + sgp * DOWN_SPW + bb >= I1) break;
            mfma(buf, cur, bb);
        }
        __syncthreads();
    };
    DownW<DT> w0, w1, w2;
    load_w(I0, w0);
    load_stage(I0);
    stage(I0, 0);
    load_stage(I0 + NB);
    if constexpr (RING == 3) load_w(I0 + NB, w1);
    __syncthreads();
    int buf = 0;
    // unrolled by the ring size so that every slot is a fixed register set
    for (int64_t Ib = I0; Ib < I1; Ib += RING * NB) {
        if constexpr (RING == 3) {
            batch(Ib, buf, w0, w2);
            buf ^= 1;
            if (Ib + NB >= I1) break;
            batch(Ib + NB, buf, w1, w0);
            buf ^= 1;
            if (Ib + 2 * NB >= I1) break;
            batch(Ib + 2 * NB, buf, w2, w1);
            buf ^= 1;
        } else {
            batch(Ib, buf, w0, w1);
            buf ^= 1;
            if (Ib + NB >= I1) break;
            batch(Ib + NB, buf, w1, w0);
            buf ^= 1;
        }
    }
    // lane (col, g) holds C[4g + r][col]: rows 0..7 the hi parts, 8..15 the
    // lo parts of tokens 4(g % 2) + r; the sub-block term of (token, s) sits
    // in lane (s, g) of accs
#pragma unroll
    for (int r = 0; r < 4; ++r) accs[r] += __shfl_xor(accs[r], 32, 64);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
        v4f o = acc[ct];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] += __shfl_xor(o[r], 32, 64);
        const int s = DT == FTX_Q4_K ? 2 * cw + (ct >> 1) : 4 * cw + ct;
        v4f t;
#pragma unroll
        for (int r = 0; r < 4; ++r) t[r] = __shfl(accs[r], s + 16 * g, 64);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            o[r] = DT == FTX_Q4_K ? o[r] - t[r] : o[r] - 32.f * t[r];
            if (sgp) red[cw][ct * 4 + r][lane] = o[r];
        }
        acc[ct] = o;
    }
    __syncthreads();
    if (sgp == 0 && g < 2) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int64_t j = sbc * 256 + cw * 64 + ct * 16 + col;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * g + r;
                const float v = acc[ct][r] + red[cw][ct * 4 + r][lane];
                a.part[(split * 8 + m) * a.N + j] = v * (1.f / DOWN_ASCALE);
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

// split count of launch_down_mfma for a shape (the same for every M) and its
// slices per split (a whole number of batches)
static int64_t down_mfma_splits(int dt, int64_t n_in, int64_t N, int cu_count,
                                int64_t* slices_per_split = nullptr) {
    const int64_t nslices = n_in / 32, nsb = N / 256;
    const int NB = dt == FTX_Q4_K ? DownCfg<FTX_Q4_K>::NB : DownCfg<FTX_Q6_K>::NB;
    // one 8-wave workgroup per CU
    int64_t S = ((int64_t)(cu_count > 0 ? cu_count : 256) + nsb - 1) / nsb;
    if (S > 64) S = 64;
    if (S > nslices) S = nslices;
    if (S < 1) S = 1;
    int64_t spp = (nslices + S - 1) / S;
    spp = (spp + NB - 1) / NB * NB;
    if (slices_per_split) *slices_per_split = spp;
    return (nslices + spp - 1) / spp;
}

size_t down_mfma_part_floats(int dt, int64_t n_in, int64_t N, int64_t Mmax, int cu_count) {
    const int64_t S = down_mfma_splits(dt, n_in, N, cu_count);
    return (size_t)(((Mmax + 7) / 8) * S * 8 * N);
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
    const int64_t nsb = N / 256;
    // splits of the contraction: one 8-wave workgroup per CU (measured best
    // on the 8B shapes: more splits add partial traffic for the next prep to
    // fold and shorten each range), at most 64, each a whole number of slice
    // batches
    int64_t spp = 0;
    const int64_t S = down_mfma_splits(dt, n_in, N, cu_count, &spp);
    a.slices_per_split = (int)spp;
    a.part = part;
    const dim3 grid((unsigned)nsb, (unsigned)S);
    if (dt == FTX_Q4_K)
        ktimed_launch(k_down_mfma<FTX_Q4_K>, grid, dim3(64 * DOWN_WAVES), 0, st, a);
    else
        ktimed_launch(k_down_mfma<FTX_Q6_K>, grid, dim3(64 * DOWN_WAVES), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (splits) {
        *splits = (int)S;
        return hipSuccess;
    }
    return launch_part_reduce(st, part, (int)S, N, M, y, ldy);
}
