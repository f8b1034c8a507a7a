// ref_harness.cpp -- extern "C" entry points into the reference's own code,
// compiled from the reference sources where they lie (see Makefile.ref).
// TEST INFRASTRUCTURE ONLY: the output library in oracle/_ref/ is used by
// tests/ to pin the oracle; nothing in the product links it.
#include "ft/quant.h"
#include "ft/cpu_backend.h"
#include "ft/sampler.h"
#include "ft/spec.h"
#include "ft/engine.h"
#include "ft/gguf.h"
#include "ft/graph.h"
#include "ft/chunker.h"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
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

// One expert's FFN through ExpertStreamer::run (include/ft/chunker.h:32-77)
// on a one-thread CpuBackend with `chunk` neurons per window: out[M][K] +=.
// gate / up / down: F rows of K columns of dtype dt.
void ref_expert_stream(const float* x, int64_t M, int64_t K, const void* gate, const void* up,
                       const void* down, int dtype, int64_t F, int64_t chunk, float* out) {
    CpuBackend cpu(1);
    StreamerConfig sc;
    sc.chunk_neurons = chunk;
    ExpertStreamer st(cpu, sc);
    st.run(x, M, K, view(gate, dtype, K, F), view(up, dtype, K, F), view(down, dtype, K, F), out);
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

// generate (src/spec.cpp:245-333) with a DraftModelDrafter (72-119): the
// target loaded from target_path prefills the prompt, the drafter loads
// draft_path; the emitted tokens go to out (up to cap).  Returns their count
// or -1.
int64_t ref_generate(const char* target_path, const char* draft_path, const int32_t* prompt,
                     int64_t n_prompt, int max_new, int spec_k, float temp, int top_k,
                     float top_p, uint64_t seed, int64_t ctx_len, int64_t prefill_batch,
                     int32_t* out, int64_t cap) {
    try {
        EngineOptions eo;
        eo.model_path = target_path;
        eo.prefill_batch = prefill_batch;
        eo.threads = 1;
        eo.igpu = IgpuMode::Off;
        eo.ctx_len = ctx_len;
        eo.throttle.enabled = false;
        Engine eng;
        eng.load(eo);
        EngineOptions dopt = eo;
        dopt.model_path = draft_path;
        DraftModelDrafter drafter(dopt);
        eng.prefill(std::vector<token_t>(prompt, prompt + n_prompt));
        SampleParams sp;
        sp.temp = temp;
        sp.top_k = top_k;
        sp.top_p = top_p;
        sp.seed = seed;
        std::vector<token_t> toks;
        generate(eng, &drafter, sp, max_new, spec_k,
                 [&](token_t t, const std::string&) { toks.push_back(t); });
        const int64_t n = std::min<int64_t>((int64_t)toks.size(), cap);
        for (int64_t i = 0; i < n; ++i) out[i] = toks[(size_t)i];
        return (int64_t)toks.size();
    } catch (...) {
        return -1;
    }
}

// Sampler::sample (include/ft/sampler.h:30-94) from `state`: reset(state)
// then sample with seed 0, which uses the state as it stands; the state after
// one draw is state + the SplitMix64 increment (one next_u32), none at temp
// <= 0 (argmax).
int32_t ref_sampler_sample(const float* logits, int64_t n, float temp, int32_t top_k,
                           float top_p, uint64_t* state) {
    Sampler s;
    s.reset(*state);
    SampleParams p;
    p.temp = temp;
    p.top_k = top_k;
    p.top_p = top_p;
    p.seed = 0;
    const int32_t t = s.sample(logits, n, p);
    if (temp > 0.f) *state += 0x9E3779B97F4A7C15ull;
    return t;
}

// The reference parser's view of a GGUF (ft::Gguf, config_from_gguf) in the
// canonical summary form of xwfes_amd.gguf.summary(offsets=False): the
// config, the typed accessors of `keys` ('\n'-separated, in order) and every
// tensor with a hash of its bytes.  Returns the text length, or -1 when the
// reference throws (the message then fills out).
int64_t ref_gguf_summary(const char* path, const char* keys, char* out, int64_t cap) {
    auto hash = [](const uint8_t* b, size_t n) {
        unsigned long long h = 0;
        for (size_t i = 0; i < n; ++i)
            h += (unsigned long long)b[i] * ((i + 1) * 0x9E3779B97F4A7C15ull);
        return h;
    };
    std::string s;
    char buf[4096];
    int64_t rc = 0;
    try {
        Gguf g(path);
        try {
            const ModelConfig c = config_from_gguf(g);
            std::snprintf(buf, sizeof(buf),
                          "config arch=%s n_layer=%lld n_embd=%lld n_head=%lld n_head_kv=%lld "
                          "head_dim=%lld vocab=%lld n_ff=%lld ctx_train=%lld rms_eps=%.9g "
                          "rope_theta=%.17g rope_neox=%d\n",
                          c.arch.c_str(), (long long)c.n_layer, (long long)c.n_embd,
                          (long long)c.n_head, (long long)c.n_head_kv, (long long)c.head_dim,
                          (long long)c.vocab, (long long)c.n_ff, (long long)c.ctx_train,
                          (double)c.rms_eps, c.rope_theta, (int)c.rope_neox);
            s += buf;
        } catch (...) {
            s += "config error\n";
        }
        std::string ks(keys ? keys : "");
        size_t p = 0;
        while (p < ks.size()) {
            size_t e = ks.find('\n', p);
            if (e == std::string::npos) e = ks.size();
            const std::string k = ks.substr(p, e - p);
            p = e + 1;
            if (k.empty()) continue;
            const std::vector<float> f = g.get_f32_arr(k);
            std::snprintf(buf, sizeof(buf),
                          "kv %s has=%d i64=%lld f64=%.17g str=%s bool=%d nstr=%zu nf32=%zu "
                          "hf32=%llu\n",
                          k.c_str(), (int)g.has(k), (long long)g.get_i64(k, -7),
                          g.get_f64(k, -7.0), g.get_str(k, "-").c_str(), (int)g.get_bool(k, false),
                          g.get_str_arr(k).size(), f.size(),
                          hash((const uint8_t*)f.data(), f.size() * 4));
            s += buf;
        }
        std::vector<std::string> names;
        for (const auto& kv : g.tensors()) names.push_back(kv.first);
        std::sort(names.begin(), names.end());
        for (const std::string& n : names) {
            const HostTensor& t = *g.tensor(n);
            std::snprintf(buf, sizeof(buf),
                          "tensor %s n_dims=%d ne=%lld,%lld,%lld,%lld dtype=%d nbytes=%zu "
                          "hash=%llu\n",
                          n.c_str(), t.n_dims, (long long)t.ne[0], (long long)t.ne[1],
                          (long long)t.ne[2], (long long)t.ne[3], (int)t.dtype, t.nbytes,
                          hash(t.data, t.nbytes));
            s += buf;
        }
        rc = (int64_t)s.size();
    } catch (const std::exception& e) {
        s = e.what();
        rc = -1;
    }
    if (cap > 0) {
        const size_t n = std::min<size_t>(s.size(), (size_t)cap - 1);
        std::memcpy(out, s.data(), n);
        out[n] = 0;
    }
    return rc;
}

}  // extern "C"
