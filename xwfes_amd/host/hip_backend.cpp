// hip_backend.cpp -- HipBackend / HipVerifier over the C ABI (include/ftx.h).
#include "hip_backend.hpp"

#include <algorithm>

#include <stdexcept>

namespace ftx_host {

namespace {
int64_t row_bytes(DType dt, int64_t cols) { return ftx_row_bytes((int)dt, cols); }
}  // namespace

void HipBackend::check(int rc, const char* what) const {
    if (rc != FTX_OK) {
        const char* msg = ctx_ ? ftx_last_error(ctx_) : "no context";
        throw std::runtime_error(std::string("HipBackend: ") + what + ": " + (msg ? msg : ""));
    }
}

HipBackend::HipBackend(int device) {
    // a failed construction throws, as the reference's accelerator backends
    // do; Engine::load then keeps the CPU path (src/engine.cpp:293-299)
    if (ftx_create(device, &ctx_) != FTX_OK) {
        ctx_ = nullptr;
        throw std::runtime_error("HipBackend: no usable HIP device");
    }
}

HipBackend::~HipBackend() {
    for (auto& kv : tensors_) ftx_tensor_free(kv.second);
    for (auto& kv : expert_rows_) ftx_tensor_free(kv.second);
    if (ctx_) ftx_destroy(ctx_);
}

std::string HipBackend::name() const { return "hip"; }

DeviceInfo HipBackend::info() const {
    DeviceInfo d;
    ftx_device_info_t di{};
    if (ctx_ && ftx_device_info(ctx_, &di) == FTX_OK) {
        d.name = di.name;
        d.mem_bytes = (uint64_t)di.mem_bytes;
    }
    return d;  // a discrete GPU: integrated = uma = false
}

bool HipBackend::ready() const { return ctx_ != nullptr; }

HipBackend::Key HipBackend::key_of(const HostTensor& W) {
    return {W.data, {(int32_t)W.dtype, {W.ne[0], W.ne[1] * W.ne[2] * W.ne[3]}}};
}

ftx_tensor* HipBackend::resident(const HostTensor& W) {
    const Key k = key_of(W);
    auto it = tensors_.find(k);
    if (it != tensors_.end()) return it->second;
    ftx_tensor* t = nullptr;
    const int64_t rb = row_bytes(W.dtype, W.ne[0]);
    check(ftx_tensor_upload(ctx_, (int)W.dtype, W.ne, rb, W.data, &t), "upload");
    tensors_[k] = t;
    return t;
}

void HipBackend::evict(const HostTensor& W) {
    auto it = tensors_.find(key_of(W));
    if (it == tensors_.end()) return;
    ftx_tensor_free(it->second);
    tensors_.erase(it);
}

void HipBackend::matmul(const float* x, int64_t M, int64_t K, const HostTensor& W, float* y) {
    if (K != W.cols()) throw std::runtime_error("HipBackend::matmul: K != W.cols()");
    check(ftx_matmul(ctx_, x, M, K, resident(W), y), "matmul");
}

const void* HipBackend::resident_rows(const void* host, size_t row_stride, int64_t rows, DType dt,
                                      int64_t cols, int64_t* dev_stride) {
    const auto key = std::make_pair(host, row_stride * (size_t)rows);
    auto it = expert_rows_.find(key);
    if (it == expert_rows_.end()) {
        ftx_tensor* t = nullptr;
        const int64_t ne[4] = {cols, rows, 1, 1};
        check(ftx_tensor_upload(ctx_, (int)dt, ne, (int64_t)row_stride, host, &t), "upload");
        it = expert_rows_.emplace(key, t).first;
    }
    *dev_stride = ftx_tensor_nbytes(it->second) / rows;
    return ftx_tensor_data(it->second);
}

void HipBackend::run_expert_chunk(const ExpertChunkJob& job) {
    ftx_expert_job j{};
    j.x = job.x;
    j.out = job.out;
    j.dt = (int32_t)job.dt;
    j.M = job.M;
    j.K = job.K;
    j.IC = job.IC;
    // resident rows are packed at the device row size
    int64_t s_gu = 0, s_d = 0;
    j.gate = resident_rows(job.gate, job.gate_up_row_stride, job.IC, job.dt, job.K, &s_gu);
    j.up = resident_rows(job.up, job.gate_up_row_stride, job.IC, job.dt, job.K, &s_gu);
    j.down = resident_rows(job.down, job.down_row_stride, job.IC, job.dt, job.K, &s_d);
    j.gate_up_row_stride = s_gu;
    j.down_row_stride = s_d;
    check(ftx_expert_chunk(ctx_, &j), "run_expert_chunk");
}

void* HipBackend::alloc_staging(size_t bytes) { return ftx_alloc_staging(ctx_, bytes); }
void HipBackend::free_staging(void* p) { check(ftx_free_staging(ctx_, p), "free_staging"); }
void HipBackend::stage(void* dst, const void* src, size_t bytes) {
    check(ftx_stage(ctx_, dst, src, bytes), "stage");
}
void HipBackend::sync() { check(ftx_sync(ctx_), "sync"); }

// ------------------------------------------------------------------ verifier

HipVerifier::HipVerifier(HipBackend& be, const ModelConfig& cfg, const ModelWeights& w,
                         int64_t ctx_cap, int64_t max_tokens, bool kv_f16)
    : be_(be), cfg_(cfg), max_tokens_(max_tokens) {
    if ((int64_t)w.layers.size() != cfg.n_layer)
        throw std::runtime_error("HipVerifier: layer count does not match the config");
    std::vector<const ftx_tensor*> layers, ext;
    for (const auto& L : w.layers) {
        if (L.size() != FTX_LAYER_TENSORS)
            throw std::runtime_error("HipVerifier: a layer needs 9 tensors");
        for (const auto& t : L) layers.push_back(t.data ? be_.resident(t) : nullptr);
    }
    if (!w.ext.empty()) {
        if ((int64_t)w.ext.size() != cfg.n_layer)
            throw std::runtime_error("HipVerifier: ext layer count does not match the config");
        for (const auto& X : w.ext) {
            if (X.size() != FTX_LAYER_EXT)
                throw std::runtime_error("HipVerifier: a layer's ext needs FTX_LAYER_EXT entries");
            for (const auto& t : X) ext.push_back(t.data ? be_.resident(t) : nullptr);
        }
    }
    ftx_model_desc d{};
    d.n_layer = cfg.n_layer;
    d.n_embd = cfg.n_embd;
    d.n_head = cfg.n_head;
    d.n_head_kv = cfg.n_head_kv;
    d.head_dim = cfg.head_dim;
    d.n_ff = cfg.n_ff;
    d.vocab = cfg.vocab;
    d.rms_eps = cfg.rms_eps;
    d.rope_neox = cfg.rope_neox ? 1 : 0;
    d.rope_theta = cfg.rope_theta;
    d.tok_embd = be_.resident(w.tok_embd);
    d.out_norm = be_.resident(w.out_norm);
    d.output = w.output.data ? be_.resident(w.output) : nullptr;
    d.layers = layers.data();
    d.max_tokens = max_tokens;
    d.layer_ext = ext.empty() ? nullptr : ext.data();
    d.n_expert = cfg.n_expert;
    d.n_expert_used = cfg.n_expert_used;
    be_.check(ftx_model_create(be_.ctx(), &d, &model_), "model_create");
    be_.check(ftx_kv_create(be_.ctx(), model_, ctx_cap, kv_f16 ? FTX_KV_F16 : FTX_KV_F32, &kv_),
              "kv_create");
    logits_ = (float*)be_.alloc_staging((size_t)(max_tokens * cfg.vocab) * sizeof(float));
    if (!logits_) throw std::runtime_error("HipVerifier: logits allocation failed");
}

HipVerifier::~HipVerifier() {
    if (logits_) ftx_free_staging(be_.ctx(), logits_);
    if (kv_) ftx_kv_free(kv_);
    if (model_) ftx_model_free(model_);
}

const float* HipVerifier::extend_verify(const std::vector<int32_t>& props,
                                        const std::vector<int32_t>& parents, bool advance) {
    const int64_t M = (int64_t)props.size();
    if (M < 1 || M > max_tokens_) throw std::runtime_error("HipVerifier: bad draft length");
    if (!parents.empty() && (int64_t)parents.size() != M)
        throw std::runtime_error("HipVerifier: parents must match the draft");
    ftx_verify_args a{};
    a.M = M;
    a.tokens = props.data();
    a.parents = parents.empty() ? nullptr : parents.data();
    a.logits = logits_;
    a.advance = advance ? 1 : 0;
    be_.check(ftx_verify_step(be_.ctx(), model_, kv_, &a), "verify_step");
    return logits_;
}

const float* HipVerifier::step(int32_t token, float* logits) {
    if (!logits) return extend_verify({token}, {}, true);
    ftx_verify_args a{};
    a.M = 1;
    a.tokens = &token;
    a.logits = logits;
    a.advance = 1;
    be_.check(ftx_verify_step(be_.ctx(), model_, kv_, &a), "step");
    return logits;
}

const float* HipVerifier::prefill(const std::vector<int32_t>& tokens, int64_t chunk) {
    if (tokens.empty()) return nullptr;
    if (chunk < 1 || chunk > max_tokens_) throw std::runtime_error("HipVerifier: bad prefill chunk");
    const int64_t n = (int64_t)tokens.size();
    for (int64_t i = 0; i < n; i += chunk) {
        const int64_t m = std::min(chunk, n - i);
        ftx_verify_args a{};
        a.M = m;
        a.tokens = tokens.data() + i;
        a.logits = i + chunk >= n ? logits_ : nullptr;  // the LM head on the last chain only
        a.advance = 1;
        be_.check(ftx_verify_step(be_.ctx(), model_, kv_, &a), "prefill");
    }
    return logits_;
}

void HipVerifier::truncate_to(int64_t npast) { be_.check(ftx_kv_truncate(kv_, npast), "truncate"); }

void HipVerifier::commit(const std::vector<int32_t>& nodes) {
    be_.check(ftx_kv_commit(kv_, nodes.data(), (int64_t)nodes.size()), "commit");
}

int64_t HipVerifier::npast() const {
    void *k = nullptr, *v = nullptr;
    int64_t n = 0;
    be_.check(ftx_kv_pointers(kv_, &k, &v, &n), "kv_pointers");
    return n;
}

void HipVerifier::write_kv(const void* k, const void* v) { be_.check(ftx_kv_write(kv_, k, v), "kv_write"); }
void HipVerifier::read_kv(void* k, void* v) { be_.check(ftx_kv_read(kv_, k, v), "kv_read"); }

void HipVerifier::verify_batch(const std::vector<BatchItem>& items) {
    if (items.empty() || items.size() > (size_t)FTX_MAX_SEQ)
        throw std::runtime_error("HipVerifier: 1-16 sequences per batch");
    std::vector<ftx_seq_args> a(items.size());
    for (size_t i = 0; i < items.size(); ++i) {
        const BatchItem& it = items[i];
        const int64_t M = (int64_t)it.props.size();
        if (M < 1) throw std::runtime_error("HipVerifier: empty draft in a batch");
        if (!it.parents.empty() && (int64_t)it.parents.size() != M)
            throw std::runtime_error("HipVerifier: parents must match the draft");
        if (it.seq && &it.seq->be_ != &be_)
            throw std::runtime_error("HipVerifier: sequence of another backend");
        a[i] = ftx_seq_args{};
        a[i].kv = it.seq ? it.seq->kv_ : kv_;
        a[i].M = M;
        a[i].tokens = it.props.data();
        a[i].parents = it.parents.empty() ? nullptr : it.parents.data();
        a[i].logits = it.logits;
        a[i].advance = it.advance ? 1 : 0;
    }
    // the library checks the token total, distinct caches and the logits rule
    be_.check(ftx_verify_batch(be_.ctx(), model_, a.data(), (int64_t)a.size()), "verify_batch");
}

HipSequence::HipSequence(HipVerifier& ver, int64_t ctx_cap, bool kv_f16) : be_(ver.be_) {
    be_.check(ftx_kv_create(be_.ctx(), ver.model_, ctx_cap, kv_f16 ? FTX_KV_F16 : FTX_KV_F32, &kv_),
              "kv_create");
}

HipSequence::~HipSequence() {
    if (kv_) ftx_kv_free(kv_);
}

void HipSequence::truncate_to(int64_t npast) { be_.check(ftx_kv_truncate(kv_, npast), "truncate"); }

void HipSequence::commit(const std::vector<int32_t>& nodes) {
    be_.check(ftx_kv_commit(kv_, nodes.data(), (int64_t)nodes.size()), "commit");
}

int64_t HipSequence::npast() const {
    void *k = nullptr, *v = nullptr;
    int64_t n = 0;
    be_.check(ftx_kv_pointers(kv_, &k, &v, &n), "kv_pointers");
    return n;
}

void HipSequence::write_kv(const void* k, const void* v) { be_.check(ftx_kv_write(kv_, k, v), "kv_write"); }
void HipSequence::read_kv(void* k, void* v) { be_.check(ftx_kv_read(kv_, k, v), "kv_read"); }

Accepted accept_on_device(HipBackend& be, int64_t V, const float* base_row, const float* rows,
                          const std::vector<int32_t>& props, AcceptMode mode, float temp,
                          uint64_t& rng, const std::vector<float>& pd,
                          const std::vector<int32_t>& parents, const float* q,
                          BonusSampler* sampler) {
    const int64_t M = (int64_t)props.size();
    BonusSampler local;
    BonusSampler& bs = sampler ? *sampler : local;
    Accepted out;
    out.nodes.assign((size_t)(M > 0 ? M : 1), -1);
    int32_t n_acc = 0;
    ftx_accept_args a{};
    a.base_row = base_row;
    a.rows = rows;
    a.q = q;
    a.M = M;
    a.V = V;
    const int32_t none = 0;  // an empty draft still passes a props pointer
    a.props = props.empty() ? &none : props.data();
    a.parents = parents.empty() ? nullptr : parents.data();
    a.pd = pd.empty() ? nullptr : pd.data();
    a.mode = (int32_t)mode;
    a.temp = temp;
    a.rng = &rng;
    a.accepted = out.nodes.data();
    a.n_acc = &n_acc;
    a.bonus = &out.bonus;
    a.margin = &out.margin;
    a.sampler_rng = &bs.state;
    a.top_k = bs.top_k;
    a.top_p = bs.top_p;
    be.check(ftx_accept(be.ctx(), &a), "accept");
    out.nodes.resize((size_t)n_acc);
    return out;
}

Accepted HipVerifier::accept(const float* base_row, const float* rows,
                             const std::vector<int32_t>& props, AcceptMode mode, float temp,
                             uint64_t& rng, const std::vector<float>& pd,
                             const std::vector<int32_t>& parents, const float* q) {
    return accept_on_device(be_, cfg_.vocab, base_row, rows, props, mode, temp, rng, pd, parents,
                            q, &sampler);
}

void DraftModelDrafter::sync(const std::vector<int32_t>& history) {
    const int64_t n = (int64_t)history.size();
    if (m_.npast() > n) m_.truncate_to(0);
    const int64_t have = m_.npast();
    if (have < n) {
        constexpr int64_t chunk = 8;
        const std::vector<int32_t> rest(history.begin() + have, history.end());
        const float* lg = m_.prefill(rest, chunk);
        row_ = lg + ((int64_t)rest.size() - 1) % chunk * m_.config().vocab;
    }
}

void DraftModelDrafter::draft(const std::vector<int32_t>& history, int k,
                              std::vector<int32_t>& props, std::vector<float>& probs) {
    sync(history);
    if (!row_) throw std::runtime_error("DraftModelDrafter: no logits (empty history)");
    pending_base_ = (int64_t)history.size();
    props.clear();
    probs.clear();
    for (int j = 0; j < k; ++j) {
        int32_t t = 0;
        float p = 0.f;
        m_.backend().check(ftx_argmax_prob(m_.backend().ctx(), row_, m_.config().vocab, &t, &p),
                           "argmax_prob");
        props.push_back(t);
        probs.push_back(p);
        if (j + 1 < k) row_ = m_.step(t);
    }
}

void DraftModelDrafter::on_commit(int64_t accepted) {
    m_.truncate_to(std::min(pending_base_ + accepted, m_.npast()));
}

void cut_draft(std::vector<int32_t>& props, std::vector<float>& probs) {
    size_t cut = props.size();
    double cum = 1.0;
    for (size_t i = 0; i < probs.size(); ++i) {
        const float p = probs[i];
        if (p >= 0.f && p < 0.02f) {
            cut = i;
            break;
        }
        cum *= p > 0.f ? (double)p : 1.0;
        if (cum < (double)0.05f) {
            cut = i + 1;
            break;
        }
    }
    props.resize(cut);
    probs.resize(cut);
}

std::vector<int32_t> generate(HipVerifier& target, DraftModelDrafter& drafter,
                              const std::vector<int32_t>& prompt, int64_t max_new, int spec_k,
                              float temp, int32_t top_k, float top_p, uint64_t seed,
                              GenerateStats* stats, int32_t eos) {
    HipBackend& be = target.backend();
    const int64_t V = target.config().vocab;
    constexpr int64_t chunk = 8;
    if (spec_k < 1 || spec_k > 8 || spec_k > target.max_tokens() || target.max_tokens() < chunk)
        throw std::runtime_error("generate: spec_k must be in 1..8 within the target's max_tokens");
    if (prompt.empty()) throw std::runtime_error("generate: empty prompt");
    float* base = (float*)be.alloc_staging((size_t)V * sizeof(float));
    if (!base) throw std::runtime_error("generate: base row allocation failed");
    std::vector<int32_t> out;
    try {
        target.truncate_to(0);
        const float* lg = target.prefill(prompt, chunk);
        be.stage(base, lg + ((int64_t)prompt.size() - 1) % chunk * V, (size_t)V * sizeof(float));
        std::vector<int32_t> history = prompt;
        uint64_t rsamp = seed ? seed : 88172645463325252ull;  // src/spec.cpp:259
        target.sampler.state = seed ? seed : 0x9E3779B97F4A7C15ull;
        // the ratio test at T = 1 (src/spec.cpp:216); temp <= 0: a top-1
        // bonus (the argmax)
        const float acc_temp = 1.f;
        target.sampler.top_k = temp > 0.f ? top_k : 1;
        target.sampler.top_p = temp > 0.f ? top_p : 1.f;
        std::vector<int32_t> props;
        std::vector<float> probs;
        while ((int64_t)out.size() < max_new) {
            drafter.draft(history, spec_k, props, probs);
            cut_draft(props, probs);
            const int64_t np_before = target.npast();
            const float* rows = props.empty() ? nullptr : target.extend_verify(props);
            const Accepted r = target.accept(base, rows, props, AcceptMode::Ratio, acc_temp, rsamp,
                                             probs);
            const int64_t acc = (int64_t)r.nodes.size();
            target.truncate_to(np_before + acc);
            if (stats) {
                ++stats->rounds;
                stats->drafted += (int64_t)props.size();
                stats->accepted += acc;
            }
            if (props.empty() && r.bonus == eos) {  // an empty draft's sampled token
                out.push_back(r.bonus);
                if (stats) stats->hit_eos = true;
                break;
            }
            // a round is emitted whole (src/spec.cpp:314-322), every accepted
            // token even past an eos among them
            bool eos_acc = false;
            for (int64_t i = 0; i < acc; ++i) {
                out.push_back(props[(size_t)i]);
                eos_acc |= eos >= 0 && props[(size_t)i] == eos;
            }
            history.insert(history.end(), props.begin(), props.begin() + acc);
            if (eos_acc) {
                drafter.on_commit(acc);
                if (stats) stats->hit_eos = true;
                break;
            }
            out.push_back(r.bonus);
            history.push_back(r.bonus);
            // one target step on the bonus: the next round's base row
            target.step(r.bonus, base);
            drafter.on_commit(acc);
            if (r.bonus == eos) {
                if (stats) stats->hit_eos = true;
                break;
            }
        }
    } catch (...) {
        ftx_free_staging(be.ctx(), base);
        throw;
    }
    ftx_free_staging(be.ctx(), base);
    return out;
}

}  // namespace ftx_host
