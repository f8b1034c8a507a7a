// gguf_summary <file> [--hash] [key ...] -- prints the canonical summary of
// a GGUF as the C++ host parser (xwfes_amd/host/gguf.cpp) reads it, in the
// form of xwfes_amd.gguf.summary(): the config, the typed accessors of the
// keys (default: every key, sorted) and every tensor with its file offset,
// or with --hash a hash of its bytes.  Test infrastructure (CPU only).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../xwfes_amd/host/gguf.hpp"

using namespace ftx_host;

static unsigned long long hash_bytes(const uint8_t* b, size_t n) {
    unsigned long long h = 0;
    for (size_t i = 0; i < n; ++i) h += (unsigned long long)b[i] * ((i + 1) * 0x9E3779B97F4A7C15ull);
    return h;
}

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: gguf_summary <file> [--hash] [key ...]\n");
        return 2;
    }
    bool hash = false;
    std::vector<std::string> keys;
    for (int i = 2; i < argc; ++i) {
        if (!std::strcmp(argv[i], "--hash")) hash = true;
        else keys.push_back(argv[i]);
    }
    try {
        Gguf g(argv[1]);
        try {
            const GgufConfig r = config_from_gguf(g);
            const ModelConfig& c = r.cfg;
            std::printf("config arch=%s n_layer=%lld n_embd=%lld n_head=%lld n_head_kv=%lld "
                        "head_dim=%lld vocab=%lld n_ff=%lld ctx_train=%lld rms_eps=%.9g "
                        "rope_theta=%.17g rope_neox=%d\n",
                        r.arch.c_str(), (long long)c.n_layer, (long long)c.n_embd,
                        (long long)c.n_head, (long long)c.n_head_kv, (long long)c.head_dim,
                        (long long)c.vocab, (long long)c.n_ff, (long long)r.ctx_train,
                        (double)c.rms_eps, c.rope_theta, (int)c.rope_neox);
        } catch (const std::exception&) {
            std::printf("config error\n");
        }
        if (keys.empty()) {
            keys = g.keys();
            std::sort(keys.begin(), keys.end());
        }
        for (const std::string& k : keys) {
            const std::vector<float> f = g.get_f32_arr(k);
            std::printf("kv %s has=%d i64=%lld f64=%.17g str=%s bool=%d nstr=%zu nf32=%zu hf32=%llu\n",
                        k.c_str(), (int)g.has(k), (long long)g.get_i64(k, -7), g.get_f64(k, -7.0),
                        g.get_str(k, "-").c_str(), (int)g.get_bool(k, false),
                        g.get_str_arr(k).size(), f.size(),
                        hash_bytes((const uint8_t*)f.data(), f.size() * 4));
        }
        for (const auto& [name, t] : g.tensors()) {
            std::printf("tensor %s n_dims=%d ne=%lld,%lld,%lld,%lld dtype=%d nbytes=%zu ",
                        name.c_str(), t.n_dims, (long long)t.ne[0], (long long)t.ne[1],
                        (long long)t.ne[2], (long long)t.ne[3], (int)t.dtype, t.nbytes);
            if (hash) std::printf("hash=%llu\n", hash_bytes(t.data, t.nbytes));
            else std::printf("offset=%llu\n", (unsigned long long)g.file_offset(t));
        }
    } catch (const std::exception& e) {
        std::printf("error %s\n", e.what());
        return 1;
    }
    return 0;
}
