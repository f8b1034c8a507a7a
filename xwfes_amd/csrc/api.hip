// api.hip -- the C ABI of include/ftx.h: contexts, resident tensors and the
// IBackend-level operations.  The verify step lives in verify.hip.
#include <cstdio>
#include <mutex>
#include <new>

#include "ftx_internal.h"
#include "quant_dev.h"

int64_t dev_row_bytes(int dt, int64_t ncols) {
    return dt == FTX_Q6_K ? q6k_dev_row_bytes(ncols) : ftx_row_bytes(dt, ncols);
}

int64_t ftx_block_elems(int dt) { return blk_elems(dt); }
int64_t ftx_block_bytes(int dt) { return blk_bytes(dt); }

bool ftx_dtype_ok(int dt) {
    switch (dt) {
        case FTX_F32: case FTX_F16: case FTX_BF16: case FTX_Q4_0: case FTX_Q4_1:
        case FTX_Q8_0: case FTX_Q4_K: case FTX_Q6_K:
            return true;
        default:
            return false;
    }
}

int ftx_fail(ftx_ctx* ctx, int code, const std::string& msg) {
    if (ctx) ctx->err = msg;
    return code;
}

int ftx_workspace(ftx_ctx* ctx, size_t bytes, void** out) {
    bytes = (bytes + 255) & ~(size_t)255;
    if (bytes > ctx->ws_bytes) {
        if (ctx->ws) {
            FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
            FTX_HIP(ctx, hipFree(ctx->ws));
            ctx->ws = nullptr;
            ctx->ws_bytes = 0;
        }
        if (hipMalloc(&ctx->ws, bytes) != hipSuccess) {
            (void)hipGetLastError();
            ctx->ws = nullptr;
            return ftx_fail(ctx, FTX_E_NOMEM, "workspace allocation failed");
        }
        ctx->ws_bytes = bytes;
    }
    *out = ctx->ws;
    return FTX_OK;
}

int ftx_pinned(ftx_ctx* ctx, size_t bytes, void** out) {
    if (bytes > ctx->pinned_bytes) {
        if (ctx->pinned) {
            FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
            FTX_HIP(ctx, hipHostFree(ctx->pinned));
            ctx->pinned = nullptr;
            ctx->pinned_bytes = 0;
        }
        FTX_HIP(ctx, hipHostMalloc(&ctx->pinned, bytes, hipHostMallocDefault));
        ctx->pinned_bytes = bytes;
    }
    *out = ctx->pinned;
    return FTX_OK;
}

// Scratch of ftx_down_axpy_noalloc (the split partials of its launches): a
// file-scope device array, one copy per GPU, held until the process ends.
// Host code never passes the array's name to a kernel; it uses the device
// address that hipGetSymbolAddress returns for the current device.
constexpr size_t NOALLOC_SCRATCH_FLOATS = (size_t)4 << 20;  // 16 MiB
static __device__ __align__(256) float scratch[NOALLOC_SCRATCH_FLOATS];

constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

// the scratch address on `device` (looked up once per device, with the
// device current for the lookup and the caller's current device restored
// after it); null on failure
static float* noalloc_scratch(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        int prev = -1;
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        void* ptr = nullptr;
        const bool ok = hipSetDevice(device) == hipSuccess &&
                        hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess;
        if (!ok) (void)hipGetLastError();
        if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
        if (!ok) return nullptr;
        g_scratch_ptr[device] = (float*)ptr;
    }
    return g_scratch_ptr[device];
}

bool ftx_is_device_ptr(const void* p) {
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeManaged;
}

extern "C" {

int64_t ftx_row_bytes(int dtype, int64_t ncols) {
    const int64_t be = blk_elems(dtype), bb = blk_bytes(dtype);
    if (bb == 0 || ncols < 0) return 0;
    return (ncols + be - 1) / be * bb;
}

int ftx_create(int device, ftx_ctx** out) {
    if (!out) return FTX_E_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) {
        (void)hipGetLastError();
        return FTX_E_DEVICE;
    }
    ftx_ctx* c = new (std::nothrow) ftx_ctx;
    if (!c) return FTX_E_NOMEM;
    c->device = device;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreate(&c->own_stream) != hipSuccess) {
        (void)hipGetLastError();
        delete c;
        return FTX_E_DEVICE;
    }
    c->stream = c->own_stream;
    hipDeviceProp_t pr;
    if (hipGetDeviceProperties(&pr, device) == hipSuccess) c->cu_count = pr.multiProcessorCount;
    // the allocation-free entry point's scratch; a failed lookup fails only
    // that entry point (it looks again on its first call)
    c->noalloc_scratch = noalloc_scratch(device);
    *out = c;
    return FTX_OK;
}

int ftx_destroy(ftx_ctx* ctx) {
    if (!ctx) return FTX_OK;
    tr_abort(ctx);  // no armed kernel timer of this thread points into ctx
    (void)hipSetDevice(ctx->device);
    if (ctx->own_stream) (void)hipStreamSynchronize(ctx->own_stream);
    if (ctx->stream && ctx->stream != ctx->own_stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->pinned) (void)hipHostFree(ctx->pinned);
    for (hipEvent_t e : ctx->events) (void)hipEventDestroy(e);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return FTX_OK;
}

int ftx_device_info(ftx_ctx* ctx, ftx_device_info_t* out) {
    if (!ctx || !out) return FTX_E_INVALID;
    hipDeviceProp_t pr;
    FTX_HIP(ctx, hipGetDeviceProperties(&pr, ctx->device));
    memset(out, 0, sizeof(*out));
    snprintf(out->name, sizeof(out->name), "HIP:%s", pr.gcnArchName);
    out->mem_bytes = (int64_t)pr.totalGlobalMem;
    out->compute_units = pr.multiProcessorCount;
    out->arch_major = pr.major;
    out->arch_minor = pr.minor;
    return FTX_OK;
}

const char* ftx_last_error(ftx_ctx* ctx) { return ctx ? ctx->err.c_str() : "no context"; }

int ftx_set_stream(ftx_ctx* ctx, void* stream) {
    if (!ctx) return FTX_E_INVALID;
    ctx->stream = stream ? (hipStream_t)stream : ctx->own_stream;
    return FTX_OK;
}

int ftx_sync(ftx_ctx* ctx) {
    if (!ctx) return FTX_E_INVALID;
    FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FTX_OK;
}

// ---------------------------------------------------------------- tensors

static int make_tensor(ftx_ctx* ctx, int dtype, const int64_t ne[4], ftx_tensor** out) {
    if (!ctx || !ne || !out) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (!ftx_dtype_ok(dtype)) return ftx_fail(ctx, FTX_E_UNSUPPORTED, "unsupported dtype");
    for (int i = 0; i < 4; ++i)
        if (ne[i] < 1 && !(i == 0 && ne[i] == 0))
            return ftx_fail(ctx, FTX_E_INVALID, "tensor dims must be >= 1");
    ftx_tensor* t = new (std::nothrow) ftx_tensor;
    if (!t) return ftx_fail(ctx, FTX_E_NOMEM, "host allocation failed");
    t->ctx = ctx;
    t->dtype = dtype;
    for (int i = 0; i < 4; ++i) t->ne[i] = ne[i];
    t->row_bytes = dev_row_bytes(dtype, ne[0]);
    t->nrows = ne[1] * ne[2] * ne[3];
    const size_t bytes = (size_t)(t->row_bytes * t->nrows);
    if (bytes && hipMalloc(&t->data, bytes) != hipSuccess) {
        (void)hipGetLastError();
        delete t;
        return ftx_fail(ctx, FTX_E_NOMEM, "device allocation failed");
    }
    *out = t;
    return FTX_OK;
}

int ftx_tensor_alloc(ftx_ctx* ctx, int dtype, const int64_t ne[4], ftx_tensor** out) {
    return make_tensor(ctx, dtype, ne, out);
}

int ftx_tensor_upload(ftx_ctx* ctx, int dtype, const int64_t ne[4], int64_t row_stride,
                      const void* host, ftx_tensor** out) {
    if (!host) return ftx_fail(ctx, FTX_E_INVALID, "null host data");
    int rc = make_tensor(ctx, dtype, ne, out);
    if (rc) return rc;
    ftx_tensor* t = *out;
    const int64_t host_rb = ftx_row_bytes(dtype, ne[0]);  // GGUF row size
    const int64_t stride = row_stride > 0 ? row_stride : host_rb;
    if (stride < host_rb) {
        ftx_tensor_free(t);
        *out = nullptr;
        return ftx_fail(ctx, FTX_E_INVALID, "row_stride shorter than a row");
    }
    hipError_t e;
    if (dtype == FTX_Q6_K) {
        // GGUF rows through the workspace, then into the device planes
        uint8_t* tmp;
        rc = ftx_workspace(ctx, (size_t)(host_rb * t->nrows), (void**)&tmp);
        if (rc) {
            ftx_tensor_free(t);
            *out = nullptr;
            return rc;
        }
        e = hipMemcpy2D(tmp, (size_t)host_rb, host, (size_t)stride, (size_t)host_rb,
                        (size_t)t->nrows, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = launch_q6k_repack(ctx->stream, tmp, host_rb, ne[0], t->nrows, t->row_bytes,
                                  t->data);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    } else if (stride == t->row_bytes) {
        e = hipMemcpy(t->data, host, (size_t)(t->row_bytes * t->nrows), hipMemcpyHostToDevice);
    } else {
        e = hipMemcpy2D(t->data, (size_t)t->row_bytes, host, (size_t)stride, (size_t)t->row_bytes,
                        (size_t)t->nrows, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        ftx_tensor_free(t);
        *out = nullptr;
        return ftx_fail(ctx, FTX_E_DEVICE, std::string("upload: ") + hipGetErrorString(e));
    }
    return FTX_OK;
}

int ftx_tensor_free(ftx_tensor* t) {
    if (!t) return FTX_OK;
    if (t->owned && t->data) (void)hipFree(t->data);
    delete t;
    return FTX_OK;
}

void* ftx_tensor_data(ftx_tensor* t) { return t ? t->data : nullptr; }

int64_t ftx_tensor_nbytes(const ftx_tensor* t) { return t ? t->row_bytes * t->nrows : 0; }

int ftx_quantize(ftx_ctx* ctx, const float* src, ftx_tensor* t) {
    if (!ctx || !src || !t) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (t->ne[0] % blk_elems(t->dtype))
        return ftx_fail(ctx, FTX_E_INVALID, "row length is not a whole number of blocks");
    if (!ftx_is_device_ptr(src)) return ftx_fail(ctx, FTX_E_INVALID, "src must be device memory");
    FTX_HIP(ctx, launch_quantize(ctx->stream, src, t->dtype, t->ne[0], t->nrows, t->row_bytes,
                                 t->data));
    FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FTX_OK;
}

int ftx_fill_normal(ftx_ctx* ctx, void* dst, int dtype, int64_t n, uint64_t seed, float std) {
    if (!ctx || !dst || n < 0) return ftx_fail(ctx, FTX_E_INVALID, "bad argument");
    if (dtype != FTX_F32 && dtype != FTX_F16)
        return ftx_fail(ctx, FTX_E_UNSUPPORTED, "fill_normal writes F32 or F16");
    if (!ftx_is_device_ptr(dst)) return ftx_fail(ctx, FTX_E_INVALID, "dst must be device memory");
    FTX_HIP(ctx, launch_fill_normal(ctx->stream, dst, dtype == FTX_F16, n, seed, std));
    FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FTX_OK;
}

// ---------------------------------------------------------------- operations

// Device views of caller buffers: device pointers pass through, host
// buffers are staged in the workspace.
struct Staged {
    const float* x;
    float* y;
    bool y_host;
};

static int stage_xy(ftx_ctx* ctx, const float* x, size_t xn, float* y, size_t yn, bool y_in,
                    size_t extra_floats, Staged& s, float** extra) {
    const bool xd = ftx_is_device_ptr(x), yd = ftx_is_device_ptr(y);
    const size_t need = (xd ? 0 : xn) + (yd ? 0 : yn) + extra_floats;
    float* ws = nullptr;
    if (need) {
        int rc = ftx_workspace(ctx, need * sizeof(float) + 1024, (void**)&ws);
        if (rc) return rc;
    }
    size_t off = 0;
    if (xd) {
        s.x = x;
    } else {
        FTX_HIP(ctx, hipMemcpyAsync(ws + off, x, xn * sizeof(float), hipMemcpyHostToDevice,
                                    ctx->stream));
        s.x = ws + off;
        off += (xn + 63) & ~(size_t)63;
    }
    if (yd) {
        s.y = y;
        s.y_host = false;
    } else {
        s.y = ws + off;
        s.y_host = true;
        if (y_in)
            FTX_HIP(ctx, hipMemcpyAsync(s.y, y, yn * sizeof(float), hipMemcpyHostToDevice,
                                        ctx->stream));
        off += (yn + 63) & ~(size_t)63;
    }
    *extra = extra_floats ? ws + off : nullptr;
    return FTX_OK;
}

int ftx_dequant(ftx_ctx* ctx, const ftx_tensor* W, float* out) {
    if (!ctx || !W || !out) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    const size_t n = (size_t)(W->ne[0] * W->nrows);
    const bool od = ftx_is_device_ptr(out);
    float* dst = out;
    if (!od) {
        int rc = ftx_workspace(ctx, n * sizeof(float), (void**)&dst);
        if (rc) return rc;
    }
    FTX_HIP(ctx, launch_dequant(ctx->stream, W->data, W->dtype, W->row_bytes, W->ne[0], W->nrows,
                                dst));
    if (!od)
        FTX_HIP(ctx, hipMemcpyAsync(out, dst, n * sizeof(float), hipMemcpyDeviceToHost,
                                    ctx->stream));
    FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FTX_OK;
}

int ftx_matmul(ftx_ctx* ctx, const float* x, int64_t M, int64_t K, const ftx_tensor* W,
               float* y) {
    if (!ctx || !x || !W || !y) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (M < 0 || K != W->ne[0])
        return ftx_fail(ctx, FTX_E_INVALID, "matmul: K must equal the weight row length");
    const int64_t N = W->nrows;
    if (M == 0) return FTX_OK;
    Staged s{};
    float* extra;
    const bool mv = mv_supported(W->dtype, K, M);
    const size_t xqf = (xq_bytes(K) + 255) / 4;
    const size_t mvf = mv ? xqf : 0;
    int rc = stage_xy(ctx, x, (size_t)(M * K), y, (size_t)(M * N), false, mvf, s, &extra);
    if (rc) return rc;
    GemvSeg seg{W->data, W->dtype, W->row_bytes, N, s.y, N};
    if (mv) {
        int8_t* xq = (int8_t*)extra;
        FTX_HIP(ctx, launch_xq_prep(ctx->stream, const_cast<float*>(s.x), K, nullptr, nullptr, 0, 0,
                                    K, M, xq));
        FTX_HIP(ctx, launch_mv(ctx->stream, &seg, 1, xq, K, M, EPI_STORE, ctx->cu_count, 0, 0.f));
    } else {
        FTX_HIP(ctx, launch_gemv(ctx->stream, &seg, 1, s.x, K, K, M, EPI_STORE));
    }
    if (s.y_host)
        FTX_HIP(ctx, hipMemcpyAsync(y, s.y, (size_t)(M * N) * sizeof(float),
                                    hipMemcpyDeviceToHost, ctx->stream));
    FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FTX_OK;
}

int ftx_down_axpy(ftx_ctx* ctx, const float* x, int64_t M, int64_t n_in, const ftx_tensor* W,
                  float* y) {
    if (!ctx || !x || !W || !y) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (M < 0 || n_in != W->nrows)
        return ftx_fail(ctx, FTX_E_INVALID, "down_axpy: n_in must equal the weight row count");
    const int64_t N = W->ne[0];
    if (M == 0) return FTX_OK;
    Staged s{};
    float* part;
    const size_t pf = down_scratch_floats(M, n_in, N);
    int rc = stage_xy(ctx, x, (size_t)(M * n_in), y, (size_t)(M * N), true, pf, s, &part);
    if (rc) return rc;
    FTX_HIP(ctx, launch_down(ctx->stream, W->data, W->dtype, W->row_bytes, n_in, N, s.x, n_in, M,
                             s.y, N, part));
    if (s.y_host)
        FTX_HIP(ctx, hipMemcpyAsync(y, s.y, (size_t)(M * N) * sizeof(float),
                                    hipMemcpyDeviceToHost, ctx->stream));
    FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FTX_OK;
}

// ftx_down_axpy on device x / y with its split partials in the library's
// file-scope scratch array instead of the context's workspace: no device or
// host memory is allocated.  Every call on a GPU shares that GPU's array, so
// calls that overlap on one GPU race; each call writes every partial it reads.
int ftx_down_axpy_noalloc(ftx_ctx* ctx, const float* x, int64_t M, int64_t n_in,
                          const ftx_tensor* W, float* y) {
    if (!ctx || !x || !W || !y) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (M < 0 || n_in != W->nrows)
        return ftx_fail(ctx, FTX_E_INVALID, "down_axpy_noalloc: n_in must equal the weight row count");
    if (!ftx_is_device_ptr(x) || !ftx_is_device_ptr(y))
        return ftx_fail(ctx, FTX_E_INVALID, "down_axpy_noalloc: x and y must be device memory");
    const int64_t N = W->ne[0];
    if (M == 0) return FTX_OK;
    const size_t pf = down_scratch_floats(M, n_in, N);
    if (pf > NOALLOC_SCRATCH_FLOATS)
        return ftx_fail(ctx, FTX_E_RANGE,
                        "down_axpy_noalloc: the shape needs " + std::to_string(pf) +
                            " floats of scratch, above the limit of " +
                            std::to_string(NOALLOC_SCRATCH_FLOATS));
    if (!ctx->noalloc_scratch) ctx->noalloc_scratch = noalloc_scratch(ctx->device);
    if (!ctx->noalloc_scratch)
        return ftx_fail(ctx, FTX_E_DEVICE, "down_axpy_noalloc: the scratch array's address "
                                           "could not be looked up on this device");
    FTX_HIP(ctx, launch_down(ctx->stream, W->data, W->dtype, W->row_bytes, n_in, N, x, n_in, M, y,
                             N, ctx->noalloc_scratch));
    // results are stream-ordered: the call returns once the work is enqueued
    // (a capturing stream must not be synchronised)
    return FTX_OK;
}

int ftx_expert_chunk(ftx_ctx* ctx, const ftx_expert_job* j) {
    if (!ctx || !j) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    if (j->IC <= 0 || j->M <= 0 || j->K <= 0) return FTX_OK;  // cpu_backend.cpp:110
    if (!j->x || !j->out || !j->gate || !j->up || !j->down)
        return ftx_fail(ctx, FTX_E_INVALID, "null job pointer");
    if (!ftx_dtype_ok(j->dt)) return ftx_fail(ctx, FTX_E_UNSUPPORTED, "unsupported dtype");
    const int64_t rb = dev_row_bytes(j->dt, j->K);
    if (j->gate_up_row_stride != rb || j->down_row_stride != rb)
        return ftx_fail(ctx, FTX_E_INVALID, "expert rows must be dense (stride == row bytes)");
    if (!ftx_is_device_ptr(j->gate) || !ftx_is_device_ptr(j->up) || !ftx_is_device_ptr(j->down))
        return ftx_fail(ctx, FTX_E_INVALID, "expert weights must be device memory");
    const int64_t M = j->M, K = j->K, IC = j->IC;
    Staged s{};
    float* extra;
    const size_t pf = down_scratch_floats(M, IC, K);
    int rc = stage_xy(ctx, j->x, (size_t)(M * K), j->out, (size_t)(M * K), true,
                      pf + (size_t)(M * IC) + 64, s, &extra);
    if (rc) return rc;
    float* h = extra;
    float* part = extra + (((size_t)(M * IC) + 63) & ~(size_t)63);
    FTX_HIP(ctx, launch_gemv_swiglu(ctx->stream, (const uint8_t*)j->gate, (const uint8_t*)j->up,
                                    j->dt, rb, IC, s.x, K, K, M, h, IC));
    FTX_HIP(ctx, launch_down(ctx->stream, (const uint8_t*)j->down, j->dt, rb, IC, K, h, IC, M, s.y,
                             K, part));
    if (s.y_host)
        FTX_HIP(ctx, hipMemcpyAsync(j->out, s.y, (size_t)(M * K) * sizeof(float),
                                    hipMemcpyDeviceToHost, ctx->stream));
    FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FTX_OK;
}

void* ftx_alloc_staging(ftx_ctx* ctx, size_t bytes) {
    if (!ctx || !bytes) return nullptr;
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        ftx_fail(ctx, FTX_E_NOMEM, "staging allocation failed");
        return nullptr;
    }
    return p;
}

int ftx_free_staging(ftx_ctx* ctx, void* p) {
    if (!ctx) return FTX_E_INVALID;
    if (p) FTX_HIP(ctx, hipFree(p));
    return FTX_OK;
}

int ftx_stage(ftx_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (!bytes)) return ctx ? FTX_OK : FTX_E_INVALID;
    if (!dst || !src) return ftx_fail(ctx, FTX_E_INVALID, "null argument");
    FTX_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, ctx->stream));
    FTX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FTX_OK;
}

}  // extern "C"
