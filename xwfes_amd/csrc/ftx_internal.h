// ftx_internal.h -- shared declarations of the HIP library behind ftx.h.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ftx.h"

// ---------------------------------------------------------------- host side

// kernel classes recorded by the trace
enum TraceKind {
    TK_EMBED = 0,
    TK_RMSNORM,
    TK_GEMV_QKV,
    TK_ROPE_KV,
    TK_ATTENTION,
    TK_GEMV_O,
    TK_GEMV_SWIGLU,
    TK_DOWN,
    TK_HEAD,
    TK_ROW_STATS,
    TK_ACCEPT,
    TK_XQ_PREP,
    TK_MOE_ROUTE,
    TK_MOE_COMBINE,
    TK_EVENT_PAIR,  // empty event brackets: the brackets' own time
    TK_COUNT
};

struct TraceRec {
    int kind;
    int ev0, ev1;
    double bytes;
    int launches;
    bool kernel = false;  // ev0 / ev1 are the start / end of one kernel's dispatch
};

// The trace's kernel timer: while armed, the first launch that goes through
// ktimed_launch carries the timer's events on its own dispatch
// (hipExtLaunchKernelGGL: the kernel's start and end), so the trace can
// report kernel durations without the event brackets' own time.
struct KernelTimer {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    bool armed = false, fired = false;
};
extern thread_local KernelTimer* g_ktimer;

template <typename F, typename... Args>
inline void ktimed_launch(F kernel, const dim3& grid, const dim3& block, uint32_t shm,
                          hipStream_t st, Args... args) {
    KernelTimer* kt = g_ktimer;
    if (kt && kt->armed && !kt->fired) {
        kt->fired = true;
        hipExtLaunchKernelGGL(kernel, grid, block, shm, st, kt->e0, kt->e1, 0, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shm, st, args...);
    }
}

struct ftx_ctx {
    int device = 0;
    // trace: events around launches, resolved by ftx_trace_read
    bool trace = false;
    std::vector<hipEvent_t> events;
    int next_event = 0;
    std::vector<TraceRec> pending;
    int64_t tr_launches[TK_COUNT] = {};
    double tr_ms[TK_COUNT] = {};
    double tr_bytes[TK_COUNT] = {};
    int64_t tr_klaunches[TK_COUNT] = {};  // launches timed on their own dispatch
    double tr_kms[TK_COUNT] = {};
    KernelTimer kt;
    int kt_ev0 = -1, kt_ev1 = -1;
    // ftx_trace_replay: launches of class replay_kind at idempotent call
    // sites are issued replay_n times between their events
    int replay_kind = -1;
    int replay_n = 1;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    int cu_count = 0;
    // grow-only device workspace for staging host buffers and split sums
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // small pinned host buffer for step arguments
    void* pinned = nullptr;
    size_t pinned_bytes = 0;
    // device address of the no-allocation entry points' scratch array on
    // this context's device
    float* noalloc_scratch = nullptr;
};

struct ftx_tensor {
    ftx_ctx* ctx = nullptr;
    int dtype = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    int64_t row_bytes = 0;
    int64_t nrows = 0;  // ne1 * ne2 * ne3
    uint8_t* data = nullptr;
    bool owned = true;
};

int64_t ftx_block_elems(int dt);
int64_t ftx_block_bytes(int dt);
bool ftx_dtype_ok(int dt);
// bytes of one resident row: the GGUF row, except Q6_K's planar layout
int64_t dev_row_bytes(int dt, int64_t ncols);
hipError_t launch_q6k_repack(hipStream_t st, const uint8_t* src, int64_t src_row_bytes,
                             int64_t ncols, int64_t nrows, int64_t dst_row_bytes, uint8_t* dst);

int ftx_fail(ftx_ctx* ctx, int code, const std::string& msg);
#define FTX_HIP(ctx, call)                                                           \
    do {                                                                             \
        hipError_t e_ = (call);                                                      \
        if (e_ != hipSuccess)                                                        \
            return ftx_fail((ctx), FTX_E_DEVICE,                                     \
                            std::string(#call) + ": " + hipGetErrorString(e_));      \
    } while (0)

// device workspace of at least `bytes`, 256-B aligned
int ftx_workspace(ftx_ctx* ctx, size_t bytes, void** out);
// pinned host staging of at least `bytes`
int ftx_pinned(ftx_ctx* ctx, size_t bytes, void** out);
bool ftx_is_device_ptr(const void* p);

// trace brackets: tr_begin returns a token (-1 when tracing is off) that
// tr_end closes after the launch; tr_begin arms the calling thread's kernel
// timer with this context's events, which tr_end -- or tr_abort on an error
// path -- disarms
int tr_begin(ftx_ctx* ctx);
void tr_end(ftx_ctx* ctx, int token, int kind, double bytes, int launches = 1);
void tr_abort(ftx_ctx* ctx);
// A traced region: the timer is disarmed on every way out of the scope (a
// launch helper that fails returns through FTX_HIP before end() runs), so no
// later launch on this thread can reach this context's events.
struct TraceScope {
    ftx_ctx* ctx;
    int tok;
    bool open = true;
    explicit TraceScope(ftx_ctx* c) : ctx(c), tok(tr_begin(c)) {}
    void end(int kind, double bytes, int launches = 1) {
        open = false;
        tr_end(ctx, tok, kind, bytes, launches);
    }
    ~TraceScope() {
        if (open) tr_abort(ctx);
    }
    TraceScope(const TraceScope&) = delete;
    TraceScope& operator=(const TraceScope&) = delete;
};
// issues of one launch at an idempotent call site (1 unless replayed)
int tr_repeats(const ftx_ctx* ctx, int kind);

// ---------------------------------------------------------------- launchers
// All enqueue on `st` and return hipError_t of the launch.

// dequantise `nrows` rows of `ncols` elements (bit-exact export)
hipError_t launch_dequant(hipStream_t st, const uint8_t* W, int dt, int64_t row_bytes,
                          int64_t ncols, int64_t nrows, float* out);

// row-dot GEMV/GEMM segment: y[m*ldy + n] (=|+=) sum_k x[m*ldx + k] W[n,k];
// `tiled` marks W as an int8-MFMA tiled copy made with `rpt` rows per tile
struct GemvSeg {
    const uint8_t* W;
    int dt;
    int64_t row_bytes;
    int64_t N;
    float* y;
    int64_t ldy;
    int tiled = 0;
    int rpt = 0;
};
enum { EPI_STORE = 0, EPI_ACCUM = 1 };
// planar Q8_0 / Q4_0 copies (scales, then quants; the generic kernels read
// them through dq8): the internal dtype for a tensor of ncols columns, or -1
int planar_dtype(int dt, int64_t ncols);
hipError_t launch_planar(hipStream_t st, const uint8_t* src, int dt, int64_t nrows, int64_t ncols,
                         uint8_t* dst);
// fp16_range: the activations and dequantised weights lie within the fp16
// range, so the MFMA form (fp16 hi + lo operands) may run
hipError_t launch_gemv(hipStream_t st, const GemvSeg* segs, int nseg, const float* x,
                       int64_t ldx, int64_t K, int64_t M, int epi, bool fp16_range = false);
// gate/up pair with SwiGLU epilogue: h[m*ldh + n] = silu(x.g_n) * (x.u_n)
hipError_t launch_gemv_swiglu(hipStream_t st, const uint8_t* Wg, const uint8_t* Wu, int dt,
                              int64_t row_bytes, int64_t N, const float* x, int64_t ldx,
                              int64_t K, int64_t M, float* h, int64_t ldh,
                              bool fp16_range = false);
// y[m*ldy + j] += sum_i h[m*ldh + i] W[i, j] (W n_in rows x N cols)
// uses `part` scratch of down_scratch_floats(...) floats
size_t down_scratch_floats(int64_t M, int64_t n_in, int64_t N);
hipError_t launch_down(hipStream_t st, const uint8_t* W, int dt, int64_t row_bytes,
                       int64_t n_in, int64_t N, const float* h, int64_t ldh, int64_t M,
                       float* y, int64_t ldy, float* part);

// int8-MFMA GEMV (k_mfma.hip): activation operand prep + row-dot product.
// The prep optionally folds S split partials part[s][m][ldpart] into x
// (written back) and takes an RMSNorm weight; a normed operand is consumed
// with launch_mv(..., normed = 1, eps).
size_t xq_bytes(int64_t K);
// stride of the per-8-row-chunk operands when a prep covers more than 8 rows
size_t xq_chunk_bytes(int64_t K);
// layout16: the operand layout of the 16x16x32 row-dot GEMV (launch_rd)
// instead of launch_mv's
hipError_t launch_xq_prep(hipStream_t st, float* x, int64_t ldx, const float* normw,
                          const float* part, int S, int64_t ldpart, int64_t K, int64_t M,
                          int8_t* xq, int layout16 = 0);
bool mv_supported(int dt, int64_t K, int64_t M);
// the SwiGLU epilogue needs the whole contraction in one pass
bool mv_swiglu_supported(int64_t K);
enum { EPI_SWIGLU = 2, EPI_QKV = 3 };
// EPI_QKV: the q / k / v projection's epilogue does RoPE with interleaved
// pairs (src/engine.cpp:43-60; cos / sin of position npast + depth per token
// and pair, computed on the host in double precision as there), writes k and
// v into the KV cache slot npast + m (K [slot][kdim], V transposed), and q
// as fp16 hi + lo parts for the MFMA attention
struct QkvEpi {
    const float* cs;   // [M][hd / 2][cos, sin]
    _Float16* qh;      // [M][n_head][hd]
    _Float16* ql;
    void* kc;          // layer base of the K cache
    void* vc;          // layer base of the V cache
    int64_t slot0;     // npast
    int64_t cap;
    int hd, n_head, n_kv, kv_f16;
};



// tiled copies for the row-dot kernel: rows per tile for an N-row tensor,
// bytes of the copy, and the re-tiling launch (src in the resident row layout)
int mv_tile_rows(int64_t N, int cu_count);
size_t mv_tiled_bytes(int dt, int64_t N, int64_t K, int rpt);
hipError_t launch_mv_tile(hipStream_t st, const uint8_t* src, int64_t src_row_bytes, int dt,
                          int64_t N, int64_t K, int rpt, uint8_t* dst);
hipError_t launch_mv(hipStream_t st, const GemvSeg* segs, int nseg, const int8_t* xq, int64_t K,
                     int64_t M, int epi, int cu_count, int normed, float eps,
                     const QkvEpi* qkv = nullptr);
// The verify step's row-dot GEMV (k_rowdot.hip): up to 8 rows on
// v_mfma_i32_16x16x32_i8, weights as the B operand, from the tiled copies
// above (every segment tiled), the activation operand in the layout16 form;
// epilogues as launch_mv (EPI_STORE / ACCUM / SWIGLU / QKV)
bool rd_supported(int dt, int64_t K, int64_t M);
// whether launch_rd takes a projection of these segments (dtype, rows, tile
// rows of each): not the SwiGLU pairs, and only launches of one round of
// resident waves; otherwise launch_mv
bool rd_take(const int* dts, const int64_t* Ns, const int* rpts, int nseg, int64_t K, int64_t M,
             int epi, int cu_count);
hipError_t launch_rd(hipStream_t st, const GemvSeg* segs, int nseg, const int8_t* xq, int64_t K,
                     int64_t M, int epi, int normed, float eps, const QkvEpi* qkv = nullptr);

hipError_t launch_part_reduce(hipStream_t st, const float* part, int S, int64_t N, int64_t M,
                              float* y, int64_t ldy);

// Large-M GEMMs (k_gemm.hip): activations as fp16 hi / lo planes [Mp][K] and
// their 32-element sums [Mp][K / 32] (Mp = tokens padded to 64), weights as
// the tiled Q4_K copy or the planar Q8_0 / Q4_0 copy.
struct MmAct {
    _Float16 *xh, *xl, *sh, *sl;
    int64_t Mp, K;
};
struct MmSeg {
    const uint8_t* W;
    int dt;             // FTX_Q4_K (tiled), FTX_Q8_0_MMT or FTX_Q4_0_MMT (re-tiled copies)
    int64_t N;          // rows
    int rpt;            // Q4_K tile rows
    int64_t row_bytes;  // planar rows
};
// output rows of sequence s (row0[s] <= m < row0[s + 1]) go to base[s] +
// (m - row0[s]) * ld
struct MmOut {
    float* base[FTX_MAX_SEQ];
    int64_t row0[FTX_MAX_SEQ + 1];
    int nseq;
    int64_t ld;
    int accum;
};
int64_t mm_pad_tokens(int64_t M);
size_t mm_act_halves(int64_t Mp, int64_t K);
MmAct mm_act(void* buf, int64_t Mp, int64_t K);
// weight_dt: the consumer's operand (Q4_0 takes its octets reordered);
// gather: operand row m is x row gather[m] (< 0: zeros), for expert launches
hipError_t launch_mm_prep(hipStream_t st, const float* x, int64_t ldx, const float* normw,
                          float eps, int64_t M, const MmAct& act, int weight_dt,
                          const int32_t* gather = nullptr);
// Split partials of an accumulating GEMM (out += its result) not yet added
// into out: part + ks * split_stride + m * ldp + n, S splits, N columns
// (S = 0: nothing pending)
struct MmPend {
    const float* part = nullptr;
    int64_t split_stride = 0, ldp = 0, N = 0;
    int S = 0;
    int accum = 0;  // out += the sum (else out = the sum)
};
// the partials `fold` added into x (rows < M, written back), then the prep
// of launch_mm_prep without a gather (fold.S = 0: the plain prep)
hipError_t launch_mm_prep_fold(hipStream_t st, float* x, int64_t ldx, const float* normw,
                               float eps, int64_t M, const MmAct& act, int weight_dt,
                               const MmPend& fold);
// the partials `fold` added into y rows < M (a reduce launch)
hipError_t launch_mm_fold(hipStream_t st, const MmPend& fold, int64_t M, float* y, int64_t ldy);
bool mm_supported(int dt, int64_t K);
// the one-pass GEMM's copy of Q8_0 / Q4_0 weights (per 16-row tile and
// 256-element step, every lane's bytes contiguous): its internal dtype (or
// -1), size, and the re-tiling of nplanes planes of `rows` rows each
int mm_tiled_dtype(int dt, int64_t K);
size_t mm_tiled_bytes(int mdt, int64_t rows, int64_t K);
hipError_t launch_mm_tile(hipStream_t st, const uint8_t* src, int dt, int64_t rows,
                          int64_t nplanes, int64_t K, uint8_t* dst);
bool mm_down_supported(int dt, int64_t n_in, int64_t N);
// split-sum scratch of a launch over N output columns (`ntiles` 256-row
// workgroup columns, `steps` 256-element contraction steps)
size_t mm_part_floats(int64_t Mp, int64_t N, int64_t steps, int64_t ntiles, int cu_count);
size_t mm_down_part_floats(int64_t Mp, int64_t n_in, int64_t N, int cu_count);
// epi: EPI_STORE / EPI_ACCUM (out.accum) or EPI_SWIGLU (segments gate, up)
// pend (EPI_STORE / EPI_ACCUM into one output, split over the
// contraction): the partials are left in `part` for the caller to fold
// (launch_mm_prep_fold, launch_mm_fold, or RoPE's partial rows) instead of
// reduced here
hipError_t launch_mm(hipStream_t st, const MmSeg* segs, int nseg, const MmAct& act, int64_t M,
                     int epi, const MmOut& out, float* part, size_t part_floats, int cu_count,
                     MmPend* pend = nullptr);
hipError_t launch_mm_down(hipStream_t st, const uint8_t* tiled, int64_t n_in, int64_t N,
                          const float* h, int64_t ldh, int64_t M, const MmOut& out, float* part,
                          size_t part_floats, int cu_count, MmPend* pend = nullptr);
// SwiGLU output of an expert launch as the next GEMM's operand: fp16 hi / lo
// planes in k_mm_prep's fragment order (contraction K), values times scale
struct MmFragOut {
    _Float16 *h, *l;
    float scale;
    int64_t K;
};
// gate / up of the routed experts (segments gate, up with `plane` bytes per
// expert plane) over the gathered operand `act` (ntile_max * trows rows,
// trows 16 or 64), tile by tile of the routing's table xtab; SwiGLU into fo.
hipError_t launch_mm_experts(hipStream_t st, const MmSeg* segs, int nseg, const int64_t* plane,
                             const MmAct& act, const int32_t* xtab, int64_t ntile_max,
                             int64_t trows, const MmFragOut& fo, float* part, size_t part_floats,
                             int cu_count);

// MoE routing, expert ffn_down and the weighted sum (k_moe.hip)
struct MoeRoute {
    int32_t* tab;        // [1 + 2 * ntile_max]: tiles in use, (expert, rows) per tile
    int32_t* slot_tok;   // [ntile_max * tile rows]: token of each operand row, -1 for padding
    int32_t* comb_slot;  // [M][U]: operand rows of token m in first-use order of experts
    float* comb_w;       // [M][U]: their renormalised weights
    int32_t* te;         // [M][U]: token m's experts, descending probability
    float* tw;           // [M][U]: their renormalised weights
    uint32_t* done;      // router workgroups finished in the running launch (0 between
                         // launches; zero when the buffer is allocated)
};
// rows per routing tile (16 or 64) and the tile table bound of an M-token
// step; the largest operand row count of any step up to Mmax tokens
int64_t moe_tile_rows(int64_t M, int64_t E, int64_t U);
int64_t moe_tiles_max(int64_t M, int64_t E, int64_t U);
int64_t moe_rows_max(int64_t Mmax, int64_t E, int64_t U);
size_t moe_route_bytes(int64_t Mmax, int64_t E, int64_t U);
MoeRoute moe_route_view(void* buf, int64_t Mmax, int64_t E, int64_t U);
// ffn_norm of the residual rows x [M][K] into xn, the router (E rows of K,
// any stored dtype) on them plus rbias [E] or null, and the routing tables
hipError_t launch_moe_route(hipStream_t st, const float* x, const float* normw, float eps,
                            float* xn, int64_t K, const uint8_t* W, int dt, int64_t row_bytes,
                            const float* rbias, int64_t M, int64_t E, int64_t U,
                            const MoeRoute& r);
bool moe_down_supported(int dt, int64_t F, int64_t K);
size_t moe_down_tiled_bytes(int dt, int64_t F, int64_t K, int64_t E);
hipError_t launch_moe_down_tile(hipStream_t st, const uint8_t* src, int dt, int64_t F, int64_t K,
                                int64_t E, uint8_t* dst);
int moe_down_splits(int64_t F, int64_t K, int64_t ntile_max, int cu_count);
// part[S][ntile_max * trows][K] = the experts' down of the operand rows (fp16
// hi / lo planes of h in fragment order, contraction F), S splits of F
hipError_t launch_moe_down(hipStream_t st, const uint8_t* tiled, int dt, int64_t F, int64_t K,
                           const _Float16* ah, const _Float16* al, const int32_t* xtab,
                           int64_t ntile_max, int64_t trows, int S, float* part,
                           size_t part_floats);
// y[m][:] (+)= sum over token m's experts, in first-use order, of weight *
// (sum_s part[s][slot][:]) / 2^10; accum = 0 stores (the MoE FFN's tmpo)
hipError_t launch_moe_combine(hipStream_t st, const float* part, int S, int64_t rows, int64_t K,
                              const MoeRoute& r, int64_t M, int64_t U, float* y, int accum);
// y[i] += x[i], n elements
hipError_t launch_add(hipStream_t st, const float* x, float* y, int64_t n);

// MFMA ffn_down (k_down.hip) over a re-tiled copy of the weights
bool down_mfma_supported(int dt, int64_t n_in, int64_t N, int64_t M);
size_t down_tiled_bytes(int dt, int64_t n_in, int64_t N);
hipError_t launch_down_tile(hipStream_t st, const uint8_t* src, int64_t src_row_bytes, int dt,
                            int64_t n_in, int64_t N, uint8_t* dst);
// split partials of launch_down_mfma for up to Mmax rows in 8-row chunks
size_t down_mfma_part_floats(int dt, int64_t n_in, int64_t N, int64_t Mmax, int cu_count);
// splits == null: the split partials are added into y here; otherwise the
// partials are left in part[S][8][N] for the caller to fold and *splits = S
hipError_t launch_down_mfma(hipStream_t st, int dt, const uint8_t* tiled, int64_t n_in, int64_t N,
                            const float* h, int64_t ldh, int64_t M, float* y, int64_t ldy,
                            float* part, int cu_count, int* splits);

// quantise rows (synthetic model builder)
hipError_t launch_quantize(hipStream_t st, const float* src, int dt, int64_t ncols,
                           int64_t nrows, int64_t row_bytes, uint8_t* dst);

hipError_t launch_fill_normal(hipStream_t st, void* dst, int f16, int64_t n, uint64_t seed,
                              float std);

// layer ops
hipError_t launch_embed(hipStream_t st, const uint8_t* E, int dt, int64_t row_bytes,
                        int64_t d, const int32_t* toks, int64_t M, float* x);
hipError_t launch_rmsnorm(hipStream_t st, const float* x, const float* w, int64_t d,
                          int64_t M, float eps, float* out);
// KV cache layout per layer: K [cap][n_kv*hd] (the reference's
// [pos][n_kv*hd], include/ft/kv_cache.h:10-47); V transposed as
// [n_kv][hd][cap] so attention reads P.V operands contiguously.  `cap` here
// is the allocated slot count, a multiple of 128.
__host__ __device__ inline int64_t v_index(int64_t slot, int64_t kvh, int64_t dim, int64_t hd,
                                           int64_t cap) {
    return (kvh * hd + dim) * cap + slot;
}

// Lane j's value of v in the wave, j wave-uniform: v_readlane, a register
// read, where a shuffle (ds_bpermute) makes an LDS round trip -- the loops
// over the lanes of one wave (softmax sums, sampler ranks, running sums)
// run at VALU speed.
__device__ __forceinline__ float lane_f(float v, int j) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), j));
}
__device__ __forceinline__ int lane_i(int v, int j) { return __builtin_amdgcn_readlane(v, j); }
__device__ __forceinline__ double lane_d(double v, int j) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, j);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), j);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// The qkv epilogue of one output: RoPE on q / k rows (interleaved pairs:
// pv = the value of row n ^ 1; (c, s) = cos / sin of this row's angle), the
// fp16 hi / lo query for attention, the K / transposed-V cache write.
__device__ __forceinline__ void qkv_store(const QkvEpi& e, int si, int m, int64_t n, float v,
                                          float pv, float c, float s, float* yp) {
#pragma clang fp contract(off)
    const int64_t d = n % e.hd, h = n / e.hd;
    if (si < 2) {
        // x0' = x0 c - x1 s, x1' = x0 s + x1 c for the pair (x0, x1) = (2i, 2i + 1)
        v = (d & 1) ? pv * s + v * c : v * c - pv * s;
    }
    *yp = v;
    const int64_t slot = e.slot0 + m, kdim = (int64_t)e.n_kv * e.hd;
    if (si == 0) {
        const int64_t o = ((int64_t)m * e.n_head + h) * e.hd + d;
        const _Float16 hi = (_Float16)v;
        e.qh[o] = hi;
        e.ql[o] = (_Float16)(v - (float)hi);
    } else if (si == 1) {
        if (e.kv_f16) ((_Float16*)e.kc)[slot * kdim + n] = (_Float16)v;
        else ((float*)e.kc)[slot * kdim + n] = v;
    } else {
        const int64_t vi = v_index(slot, h, d, e.hd, e.cap);
        if (e.kv_f16) ((_Float16*)e.vc)[vi] = (_Float16)v;
        else ((float*)e.vc)[vi] = v;
    }
}

struct RopeArgs {
    float* qkv;        // [M][ldq]: q at 0, k at qdim, v at qdim + kdim
    int64_t ldq;
    int64_t n_head, n_kv, hd;
    const int32_t* depth;   // [M]
    const int64_t* npast;   // device scalar
    double theta;
    int neox;
    void* kc;          // layer base of K cache [cap][kdim]
    void* vc;          // layer base of V cache [n_kv][hd][cap]
    int kv_f16;
    int64_t cap;
    // optional: the rotated q also as fp16 hi + lo parts, [m][n_head][hd]
    _Float16* qh16 = nullptr;
    _Float16* ql16 = nullptr;
    // optional attention extras (src/engine.cpp:519-542), applied before
    // RoPE: bias [qdim + 2 kdim] added to q | k | v, RMSNorm weights [hd] of
    // every q head and every k head, with eps
    const float* bias = nullptr;
    const float* qnorm = nullptr;
    const float* knorm = nullptr;
    float eps = 0.f;
    // optional: the q | k | v row m is first formed from the split partials
    // of its GEMM, sum_s part[s * split_stride + m * ldp + col] in split order
    const float* part = nullptr;
    int64_t split_stride = 0, ldp = 0;
    int S = 0;
    // optional: the angles' cos / sin per row and pair, [M][hd / 2][2]
    // (computed on the host in double as rope_vec does), instead of forming
    // them on the device
    const float* cs = nullptr;
};
hipError_t launch_rope_kv(hipStream_t st, const RopeArgs& a, int64_t M);
// several sequences in one launch: sequence s's rows are M[s] tokens
struct RopeBatch {
    RopeArgs s[FTX_MAX_SEQ];
    int row0[FTX_MAX_SEQ + 1];  // first token row of each sequence
    int nseq;
};
hipError_t launch_rope_kv_batch(hipStream_t st, const RopeArgs* as, const int64_t* M, int nseq);
struct AttnArgs {
    const float* qkv;   // q rows, ldq stride
    int64_t ldq;
    const void* kc;     // layer base [cap][kdim]
    const void* vc;     // layer base [n_kv][hd][cap]
    int kv_f16;
    const int64_t* npast;      // device scalar
    const uint32_t* anc;       // [M][anc_words] ancestor bitmask (self included)
    int anc_words;
    int64_t n_head, n_kv, hd;
    int64_t max_ctx;           // upper bound of npast + M for LDS sizing
    float* out;                // [M][n_head*hd]
    int64_t cap;
};
hipError_t launch_attention(hipStream_t st, const AttnArgs& a, int64_t M);

// MFMA attention (k_attn.hip): fp16 KV, hd 64 or 128
// the one-pass GEMM's activation operand (fp16 hi / lo planes and
// 32-element sums in fragment order, as k_mm_prep writes them) as the
// destination of a producer: token row m of the producer is operand row
// row0 + m; contraction K; inter for Q4_0 weights
struct MmFragDst {
    _Float16 *xh = nullptr, *xl = nullptr, *sh = nullptr, *sl = nullptr;
    int64_t row0 = 0, K = 0;
    int inter = 0;
};
struct AttnMArgs {
    const float* qkv;
    int64_t ldq;
    const _Float16* qh16;  // rotated q split into fp16 hi + lo, [m][n_head][hd]
    const _Float16* ql16;
    const _Float16* kc;  // layer base [cap][kdim]
    const _Float16* vt;  // layer base [n_kv][hd][cap]
    int64_t cap;         // allocated slots, multiple of 128
    int64_t npast;       // committed slots before the draft
    const uint32_t* anc;
    int anc_words;
    int M, n_head, n_kv, hd;
    float* out;          // [M][n_head*hd]
    float *pmax, *psum, *pout;  // chunk partials
    int nc = 1;          // chunks per workgroup (and per partial)
    int pslots = 0;      // slots per partial (set by the launcher)
    MmFragDst frag;      // frag.xh set: the fp32 combine writes this operand instead of out
};
bool attn_mfma_supported(int64_t hd, int kv_f16, int64_t M, int64_t n_head, int64_t n_kv);
size_t attn_part_floats(int64_t M, int64_t n_head, int64_t hd, int64_t cap_alloc);
// xq != null: the chunk combine writes the output projection's activation
// operand (xq_dev.h layout, K = n_head * hd) instead of a.out
bool attn_combine_xq_supported(int64_t hd, int64_t n_head);
// xq16: the operand in the layout of the 16x16x32 row-dot GEMV (xq16_emit)
hipError_t launch_attn_mfma(hipStream_t st, AttnMArgs a, float* part, int8_t* xq = nullptr,
                            int xq16 = 0);
// several sequences' attention (and the fp32 combine) in one launch each:
// as[s] as for launch_attn_mfma with the sequence's own partial buffer
// parts[s]; every sequence has the same head size and kv head count
struct AttnMBatch {
    AttnMArgs s[FTX_MAX_SEQ];
    int nch[FTX_MAX_SEQ];        // chunks of each sequence's cache
    int qt0[FTX_MAX_SEQ + 1];    // first 32-row query tile of each sequence
    int qi0[FTX_MAX_SEQ + 1];    // first (token, head) row of each sequence
    int nseq;
};
hipError_t launch_attn_mfma_batch(hipStream_t st, const AttnMArgs* as, const float* const* parts,
                                  int nseq);
// KV commit of an accepted draft path (nodes by value: at most 256)
struct KvCommitArgs {
    int64_t npast;     // committed slots before the draft
    int64_t cap;       // allocated slots per layer
    int64_t n_layer;
    int n_kv, hd;
    int n;             // path length
    int32_t nodes[256];
};
hipError_t launch_kv_commit(hipStream_t st, const KvCommitArgs& a, void* k, void* v, int kv_f16);
// canonical [slot][kdim] <-> device V layout (per layer, all slots)
hipError_t launch_v_layout(hipStream_t st, const void* src, void* dst, int64_t n_layer,
                           int64_t cap, int64_t n_kv, int64_t hd, int elem_bytes, int to_device);

// acceptance
struct RowStats {
    float mx;
    int32_t amax;
    double sum;  // sum_i exp((l_i - mx)/T) in double
};
// Full-vocab statistics of M + 1 logits rows (row 0 = base_row, row 1 + i =
// rows + i V): per 4096-element chunk the first-max argmax and, with
// with_sum, per 128-element sub-chunk the double sum of exp((l - max)/T)
// with the row max.  The acceptance kernel combines them.
struct RowChunks {
    float* cmax;     // [nrows][nch]
    int32_t* carg;   // [nrows][nch]
    double* csub;    // [nrows][nsub] sum of exp((double)((l - max)/T))
    double* csubf;   // [nrows][nsub] sum of the float expf((l - max)/T) (the sampler's)
    float* submax;   // [nrows][nsub] sub-chunk maxima
    int nch, nsub;
};
size_t row_stats_scratch_bytes(int64_t nrows, int64_t V);
RowChunks row_chunks(void* scratch, int64_t nrows, int64_t V);
hipError_t launch_row_stats(hipStream_t st, const float* base_row, const float* rows,
                            int64_t nrows, int64_t V, float temp, int with_sum,
                            const RowChunks& rc);
struct AcceptDev {
    const float* base_row;
    const float* rows;
    const float* q;
    RowChunks rc;            // chunk statistics of the M + 1 rows
    int with_sum;
    RowStats* stats;         // [M+1] written by the kernel: stats[0] base row, stats[1+i] row i
    int64_t M, V;
    const int32_t* props;    // device [M]
    const int32_t* parents;  // device [M] (chain given explicitly)
    const float* pd;         // device [M] or null
    int mode;
    float temp;
    uint64_t* rng;           // device state of the acceptance stream
    uint64_t* sampler_rng;   // device state of the bonus sampler (ratio mode)
    int top_k;
    float top_p;
    double* p;               // scratch [V] (residual mode)
    int32_t* out;            // device: [0]=n_acc, [1]=bonus, [2..2+M) accepted
    float* margin;           // device scalar
};
hipError_t launch_accept(hipStream_t st, const AcceptDev& a);
// n acceptances (GREEDY / RATIO) in one launch, workgroup s taking d_arr[s]
// (device memory)
hipError_t launch_accept_multi(hipStream_t st, const AcceptDev* d_arr, int n);
// the RESIDUAL mode over many workgroups (row statistics included); scratch
// of accept_residual_scratch_bytes(); accept_residual_error copies the grid
// barrier's time-out flag to the host int *err (enqueued on st)
size_t accept_residual_scratch_bytes();
hipError_t launch_accept_residual(hipStream_t st, const AcceptDev& a, void* scratch);
int accept_residual_error(const void* scratch, hipStream_t st, int* err);
// argmax and its T = 1 softmax probability of one row: out = {token, prob
// bits} (scratch: row_stats_scratch_bytes(1, V))
hipError_t launch_argmax_prob(hipStream_t st, const float* row, int64_t V, void* scratch,
                              int32_t* out);
