// hip_backend.hpp -- C++ host side of the MI355X verify path, above the C ABI
// of include/ftx.h.
//
// HipBackend mirrors the reference engine's backend interface, ft::IBackend
// (include/ft/backend.h:21-40): the same member names, argument meanings and
// error behaviour (std::runtime_error), so that a maintainer can derive it
// from ft::IBackend and construct it where Engine::load builds its
// accelerator backend (src/engine.cpp:291-300).  The value types below
// restate the reference's HostTensor, DeviceInfo and ExpertChunkJob fields
// (include/ft/types.h:119-147, include/ft/backend.h:7-19).
//
// HipVerifier is the device-resident verify step: Engine::extend_verify ->
// Engine::forward(M) over the KV cache (src/engine.cpp:669-674, 461-596),
// truncate_to (src/engine.cpp:423-428), and the acceptance of
// accept_chain_greedy / accept_chain_sampling plus the bonus token
// (src/spec.cpp:203-238, 302-311), with draft-tree and residual extensions.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "../../include/ftx.h"

namespace ftx_host {

// the reference's DType values (include/ft/types.h:20-27) plus GGUF K-quants
enum class DType : int32_t {
    F32 = FTX_F32,
    F16 = FTX_F16,
    Q4_0 = FTX_Q4_0,
    Q4_1 = FTX_Q4_1,
    Q8_0 = FTX_Q8_0,
    Q4_K = FTX_Q4_K,
    Q6_K = FTX_Q6_K,
    BF16 = FTX_BF16,
};

// a weight tensor as the engine hands it to its backend: ne[0] = cols
// (contiguous, blocked), ne[1] = rows, data = GGUF bytes in host memory
struct HostTensor {
    std::string name;
    int64_t ne[4] = {1, 1, 1, 1};
    int32_t n_dims = 0;
    DType dtype = DType::F32;
    const uint8_t* data = nullptr;
    size_t nbytes = 0;
    int64_t cols() const { return ne[0]; }
    int64_t rows() const { return ne[1]; }
};

struct DeviceInfo {
    std::string name;
    bool integrated = false;
    bool uma = false;
    uint64_t mem_bytes = 0;
};

// gate / up / down point at IC rows of raw expert weights (host memory)
struct ExpertChunkJob {
    const float* x = nullptr;
    float* out = nullptr;
    const void* gate = nullptr;
    const void* up = nullptr;
    const void* down = nullptr;
    DType dt = DType::F32;
    int64_t M = 0;
    int64_t K = 0;
    int64_t IC = 0;
    size_t gate_up_row_stride = 0;
    size_t down_row_stride = 0;
};

class HipBackend {
public:
    explicit HipBackend(int device = 0);
    ~HipBackend();
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;

    std::string name() const;
    DeviceInfo info() const;
    bool ready() const;

    // y[m*N + n] = sum_k x[m*K + k] * W[n, k] for m < M, n < W.rows(); x and
    // y are host or device memory; W is uploaded once and kept resident,
    // keyed by (W.data, dtype, shape): as in the engine, whose weights live in
    // the GGUF mapping for the backend's lifetime, the bytes behind a key
    // must not change while the backend holds them (evict() drops a copy)
    void matmul(const float* x, int64_t M, int64_t K, const HostTensor& W, float* y);

    // h[m, i] = silu(x_m . gate_i) * (x_m . up_i); out[m, :] += sum_i h[m, i] down_i
    void run_expert_chunk(const ExpertChunkJob& job);

    void* alloc_staging(size_t bytes);
    void free_staging(void* p);
    void stage(void* dst, const void* src, size_t bytes);
    void sync();

    // the resident copy of W (uploaded on first use)
    ftx_tensor* resident(const HostTensor& W);
    void evict(const HostTensor& W);
    ftx_ctx* ctx() const { return ctx_; }
    void check(int rc, const char* what) const;

private:
    const void* resident_rows(const void* host, size_t row_stride, int64_t rows, DType dt,
                              int64_t cols, int64_t* dev_stride);
    ftx_ctx* ctx_ = nullptr;
    using Key = std::pair<const void*, std::pair<int32_t, std::pair<int64_t, int64_t>>>;
    static Key key_of(const HostTensor& W);
    std::map<Key, ftx_tensor*> tensors_;
    std::map<std::pair<const void*, size_t>, ftx_tensor*> expert_rows_;
};

struct ModelConfig {
    int64_t n_layer = 0, n_embd = 0, n_head = 0, n_head_kv = 0, head_dim = 0, n_ff = 0, vocab = 0;
    float rms_eps = 1e-5f;
    bool rope_neox = false;
    double rope_theta = 10000.0;
    // MoE layers (ModelConfig::n_experts / n_expert_used, src/graph.cpp:48-50)
    int64_t n_expert = 0, n_expert_used = 0;
};

// per-layer tensors in the order attn_norm, q, k, v, o, ffn_norm, gate, up,
// down (down in the reference orientation: n_ff rows of n_embd columns; the
// three FFN tensors have data == nullptr on a MoE layer), and the optional
// ones in the order of FTX_X_* (data == nullptr: absent; expert planes keep
// their three dims)
struct ModelWeights {
    HostTensor tok_embd, out_norm, output;  // output.data == nullptr: tied
    std::vector<std::vector<HostTensor>> layers;
    std::vector<std::vector<HostTensor>> ext;  // empty, or n_layer x FTX_LAYER_EXT
};

enum class AcceptMode : int32_t {
    Greedy = FTX_ACCEPT_GREEDY,
    Ratio = FTX_ACCEPT_RATIO,
    Residual = FTX_ACCEPT_RESIDUAL,
};

// the ratio-mode bonus sampler: Sampler::sample's parameters and state
// (include/ft/sampler.h:10-19, 30-94); the state carries over between draws
// as the Sampler object of generate does (src/spec.cpp:248-249)
struct BonusSampler {
    uint64_t state = 0x9E3779B97F4A7C15ull;
    int32_t top_k = 40;
    float top_p = 0.95f;
};

struct Accepted {
    std::vector<int32_t> nodes;  // accepted node ids, root first
    int32_t bonus = -1;          // the token that follows them
    float margin = 0.f;          // min |u - ratio| over the stochastic decisions
};

// acceptance over device logits (base_row [V], rows [M][V]); rng is the
// SplitMix64 state (in / out)
Accepted accept_on_device(HipBackend& be, int64_t V, const float* base_row, const float* rows,
                          const std::vector<int32_t>& props, AcceptMode mode, float temp,
                          uint64_t& rng, const std::vector<float>& pd = {},
                          const std::vector<int32_t>& parents = {}, const float* q = nullptr,
                          BonusSampler* sampler = nullptr);

class HipSequence;

class HipVerifier {
public:
    HipVerifier(HipBackend& be, const ModelConfig& cfg, const ModelWeights& w, int64_t ctx_cap,
                int64_t max_tokens, bool kv_f16 = true);
    ~HipVerifier();
    HipVerifier(const HipVerifier&) = delete;
    HipVerifier& operator=(const HipVerifier&) = delete;

    // forward of the draft tokens against the committed context; parents
    // empty = linear chain, else parents[i] in {-1, 0..i-1}; returns the
    // device logits [M][vocab], valid until the next call
    const float* extend_verify(const std::vector<int32_t>& props,
                               const std::vector<int32_t>& parents = {}, bool advance = false);
    // Engine::step (src/engine.cpp:650-658): one token at the committed
    // position; returns its device logits row, the cache one longer
    // logits != nullptr: the row goes there (device [vocab]) instead
    const float* step(int32_t token, float* logits = nullptr);
    // Engine::prefill (src/engine.cpp:598-648, without the prefix cache): the
    // tokens in advancing chains of at most `chunk`, the LM head only on the
    // last; returns the device logits of that last chain (rows [0, n % chunk
    // or chunk)), valid until the next call
    const float* prefill(const std::vector<int32_t>& tokens, int64_t chunk = 8);
    void truncate_to(int64_t npast);
    // keep the accepted path nodes (node ids of the last extend_verify, root
    // first) as the next committed positions; a chain is truncate_to
    void commit(const std::vector<int32_t>& nodes);
    int64_t npast() const;
    // whole cache from / to host arrays [n_layer][cap][n_head_kv*head_dim]
    void write_kv(const void* k, const void* v);
    void read_kv(void* k, void* v);

    // acceptance over device logits; rng is the SplitMix64 state (in / out)
    // the bonus sampler of ratio mode (state carried over between accepts)
    BonusSampler sampler;
    Accepted accept(const float* base_row, const float* rows, const std::vector<int32_t>& props,
                    AcceptMode mode, float temp, uint64_t& rng, const std::vector<float>& pd = {},
                    const std::vector<int32_t>& parents = {}, const float* q = nullptr);

    // several sequences of this model in one step (ftx_verify_batch): each
    // item verifies its draft against its own cache (seq == nullptr: this
    // verifier's cache), every weight streamed once for all of them; the
    // logits pointers are all null or all set (device [M][vocab] each)
    struct BatchItem {
        HipSequence* seq = nullptr;
        std::vector<int32_t> props;
        std::vector<int32_t> parents;  // empty = linear chain
        float* logits = nullptr;
        bool advance = false;
    };
    void verify_batch(const std::vector<BatchItem>& items);

    const ModelConfig& config() const { return cfg_; }
    HipBackend& backend() { return be_; }
    int64_t max_tokens() const { return max_tokens_; }

private:
    friend class HipSequence;
    HipBackend& be_;
    ModelConfig cfg_;
    ftx_model* model_ = nullptr;
    ftx_kv* kv_ = nullptr;
    float* logits_ = nullptr;
    int64_t max_tokens_ = 0;
};

// One more sequence over a HipVerifier's model (no counterpart in the
// reference, whose Engine owns one KvCache, include/ft/kv_cache.h:10-47): a
// cache of its own with the KvCache operations, verified together with
// other sequences by HipVerifier::verify_batch.  Must not outlive the
// verifier.
class HipSequence {
public:
    HipSequence(HipVerifier& ver, int64_t ctx_cap, bool kv_f16 = true);
    ~HipSequence();
    HipSequence(const HipSequence&) = delete;
    HipSequence& operator=(const HipSequence&) = delete;

    void truncate_to(int64_t npast);
    void commit(const std::vector<int32_t>& nodes);
    int64_t npast() const;
    void write_kv(const void* k, const void* v);
    void read_kv(void* k, void* v);

private:
    friend class HipVerifier;
    HipBackend& be_;
    ftx_kv* kv_ = nullptr;
};

// DraftModelDrafter (src/spec.cpp:72-119) over a resident draft model: its
// cache synced to the committed history by prefill, k greedy draft tokens
// each with its T = 1 softmax probability (Sampler::argmax + softmax_prob on
// the device, one draft step per token after the first), the cache cut back
// to the accepted prefix on commit
class DraftModelDrafter {
public:
    explicit DraftModelDrafter(HipVerifier& model) : m_(model) {}
    // src/spec.cpp:77-85: reset when ahead of the history, prefill what it
    // lacks; the logits of the history's last token are then current
    void sync(const std::vector<int32_t>& history);
    // src/spec.cpp:97-112
    void draft(const std::vector<int32_t>& history, int k, std::vector<int32_t>& props,
               std::vector<float>& probs);
    // src/spec.cpp:114-117 with Engine::truncate_to's clamp
    // (src/engine.cpp:423-428)
    void on_commit(int64_t accepted);

private:
    HipVerifier& m_;
    const float* row_ = nullptr;  // device logits of the current last token
    int64_t pending_base_ = 0;
};

// generate's draft cut (src/spec.cpp:276-285): stop at the first probability
// below 0.02f, or after the token that takes the running product below 0.05f
void cut_draft(std::vector<int32_t>& props, std::vector<float>& probs);

struct GenerateStats {
    int64_t rounds = 0, drafted = 0, accepted = 0;
    bool hit_eos = false;
};

// generate's speculative block (src/spec.cpp:245-333) on the device-resident
// path: prefill the prompt, then rounds of draft -> cut -> verify on the
// target -> ratio acceptance with the draft probabilities -> bonus from the
// row after the last accepted token (Sampler::sample with its state carried
// over in target.sampler; temp <= 0: the argmax) -> truncate -> one target
// step on the bonus, until at least max_new tokens are out (a round is
// emitted whole) or the end-of-sequence token eos (the GGUF's
// tokenizer.ggml.eos_token_id, -1 for none) ends it as the reference's loop
// does (316-328): an accepted draft token equal to eos ends it once every
// accepted token is out (no bonus), a bonus equal to eos is emitted and
// stepped, the sampled token of an empty draft is emitted.  The acceptance
// test takes the target at T = 1 whatever temp is (accept_chain_sampling,
// src/spec.cpp:216); temp shapes the bonus.  Returns the generated tokens.
std::vector<int32_t> generate(HipVerifier& target, DraftModelDrafter& drafter,
                              const std::vector<int32_t>& prompt, int64_t max_new, int spec_k = 8,
                              float temp = 0.f, int32_t top_k = 40, float top_p = 0.95f,
                              uint64_t seed = 0, GenerateStats* stats = nullptr,
                              int32_t eos = -1);

}  // namespace ftx_host
