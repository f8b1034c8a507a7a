// ref_harness.cpp -- extern "C" entry points into the reference's own code,
// compiled from the reference sources where they lie (see Makefile.ref).
// TEST INFRASTRUCTURE ONLY: the output library in oracle/_ref/ is used by
// tests/ to pin the oracle; nothing in the product links it.
#include "ft/quant.h"
#include "ft/cpu_backend.h"
#include "ft/sampler.h"
#include "ft/spec.h"
#include "ft/engine.h"

#include <cstdint>
#include <cstring>
#include <vector>

namespace ft {
float softmax_prob(const float* logits, int64_t V, token_t t);  // src/spec.cpp:89
}

using namespace ft;

static HostTensor view(const void* data, int dtype, int64_t ne0, int64_t ne1) {
    HostTensor t;
    t.name = "w";
    t.ne[0] = ne0;
    t.ne[1] = ne1;
    t.n_dims = 2;
    t.dtype = (DType)dtype;
    t.data = (const uint8_t*)data;
    t.nbytes = dtype_row_bytes(t.dtype, ne0) * (size_t)ne1;
    return t;
}

extern "C" {

float ref_half_to_float(uint16_t h) { return half_to_float(h); }
uint16_t ref_float_to_half(float f) { return float_to_half(f); }
float ref_bf16_to_float(uint16_t b) { return bf16_to_float(b); }

void ref_dequant_row(float* dst, const uint8_t* src, int dtype, int64_t n) {
    dequant_row(dst, src, (DType)dtype, n);
}

float ref_dot_row_f32(const float* x, const uint8_t* w, int dtype, int64_t n) {
    return dot_row_f32(x, w, (DType)dtype, n);
}

// CpuBackend::matmul as shipped (M-sum behaviour included): y holds N floats.
void ref_cpu_matmul(const float* x, int64_t M, int64_t K, const void* W,
                    int dtype, int64_t N, float* y, int threads) {
    CpuBackend cpu(threads);
    cpu.matmul(x, M, K, view(W, dtype, K, N), y);
}

void ref_down_axpy(const float* x, int64_t M, int64_t n_in, const void* W,
                   int dtype, int64_t N, float* y) {
    matmul_down_axpy(x, M, n_in, view(W, dtype, N, n_in), y);
}

int ref_argmax(const float* row, int64_t n) { return Sampler::argmax(row, n); }

float ref_softmax_prob(const float* lg, int64_t V, int32_t t) {
    return softmax_prob(lg, V, t);
}

int ref_accept_chain_greedy(const float* base, const float* rows, int64_t V,
                            const int32_t* props, int64_t k) {
    return accept_chain_greedy(base, rows, V, props, k);
}

int ref_accept_chain_sampling(const float* base, const float* rows,
                              const float* pd, int64_t V, const int32_t* props,
                              int64_t k, float temp, uint64_t* rng) {
    return accept_chain_sampling(base, rows, pd, V, props, k, temp, *rng);
}

// Engine: load a GGUF, run steps, copy the logits row out.
void* ref_engine_load(const char* path, int threads, int64_t ctx_len) {
    try {
        EngineOptions eo;
        eo.model_path = path;
        eo.threads = threads;
        eo.igpu = IgpuMode::Off;
        eo.ctx_len = ctx_len;
        eo.throttle.enabled = false;
        Engine* e = new Engine;
        e->load(eo);
        return e;
    } catch (...) {
        return nullptr;
    }
}

void ref_engine_free(void* h) { delete (Engine*)h; }

int64_t ref_engine_vocab(void* h) { return ((Engine*)h)->cfg().vocab; }

int ref_engine_step(void* h, int32_t tok, float* out) {
    try {
        Engine* e = (Engine*)h;
        const float* lg = e->step(tok);
        if (!lg) return -1;
        std::memcpy(out, lg, sizeof(float) * (size_t)e->cfg().vocab);
        return 0;
    } catch (...) {
        return -1;
    }
}

}  // extern "C"
