// gguf.hpp -- the on-disk boundary of the verify path in C++: a GGUF parser
// with the reference's interface and behaviour (ft::Gguf, include/ft/gguf.h,
// src/gguf.cpp:168-345), the model config it implies (config_from_gguf,
// src/graph.cpp:24-80) and the dense model's tensors by role (the name
// lookups of Engine::load, src/engine.cpp:282-396), ready for HipVerifier.
//
// Differences from the reference, each an extension: the Q4_K (12) and
// Q6_K (14) tensor dtypes of the public GGUF format are accepted (the
// reference throws at load); keys() and file_offset() expose what the
// reference keeps private; an offset past the end of the file is an error
// before the size check (the reference's unsigned subtraction wraps).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "hip_backend.hpp"

namespace ftx_host {

class Gguf {
public:
    explicit Gguf(const std::string& path);  // throws std::runtime_error
    ~Gguf();
    Gguf(const Gguf&) = delete;
    Gguf& operator=(const Gguf&) = delete;

    bool has(const std::string& key) const;
    std::string get_str(const std::string& key, const std::string& def = "") const;
    int64_t get_i64(const std::string& key, int64_t def = 0) const;
    double get_f64(const std::string& key, double def = 0) const;
    bool get_bool(const std::string& key, bool def = false) const;
    std::vector<std::string> get_str_arr(const std::string& key) const;
    std::vector<float> get_f32_arr(const std::string& key) const;
    std::vector<int32_t> get_i32_arr(const std::string& key) const;

    const HostTensor* tensor(const std::string& name) const;
    const std::map<std::string, HostTensor>& tensors() const { return tensors_; }

    std::vector<std::string> keys() const;
    uint64_t file_offset(const HostTensor& t) const;
    uint32_t alignment() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
    std::map<std::string, HostTensor> tensors_;
};

// the model config of the file; arch / ctx_train / moe alongside
struct GgufConfig {
    ModelConfig cfg;
    std::string arch;
    int64_t ctx_train = 4096;
    bool moe = false;
};
GgufConfig config_from_gguf(const Gguf& g);

// the model's tensors by role, each as a matrix of ne[0] columns (a tensor
// of more than two dims is taken as all its planes' rows: the reference's
// [d, 1, V] embedding is V rows of d) except the expert planes, which keep
// their three dims; the optional per-layer tensors (attention bias, q / k
// norms, MoE router, experts, router bias, shared expert) in w.ext; fills
// cfg.n_ff (and, for MoE, n_expert / n_expert_used) as Engine::load does
// (src/engine.cpp:318-387) when the metadata has none
ModelWeights weights_from_gguf(const Gguf& g, ModelConfig& cfg);

}  // namespace ftx_host
