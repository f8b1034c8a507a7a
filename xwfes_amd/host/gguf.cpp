// gguf.cpp -- GGUF parser, model config and tensor lookup (see gguf.hpp).
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <climits>
#include <cstring>
#include <stdexcept>
#include <unordered_map>

namespace ftx_host {

namespace {

constexpr uint32_t kMagic = 0x46554747;  // "GGUF"
enum : uint32_t {
    K_U8, K_I8, K_U16, K_I16, K_U32, K_I32, K_F32, K_BOOL, K_STR, K_ARR, K_U64, K_I64, K_F64
};

// one metadata value: integers in i, floats in f, bools in b, strings in s;
// arrays keep their element kind, count and raw bytes (or strings)
struct Val {
    uint32_t kind = 0;
    int64_t i = 0;
    double f = 0;
    bool b = false;
    std::string s;
    uint32_t ekind = 0;
    uint64_t count = 0;
    std::vector<std::string> strs;
    std::vector<uint8_t> raw;
};

size_t kind_bytes(uint32_t k) {
    switch (k) {
        case K_U8: case K_I8: case K_BOOL: return 1;
        case K_U16: case K_I16: return 2;
        case K_U32: case K_I32: case K_F32: return 4;
        case K_U64: case K_I64: case K_F64: return 8;
        default: return 0;
    }
}

// (elements, bytes) per block of each accepted tensor dtype
bool block_of(uint32_t dt, int64_t& eb, int64_t& bb) {
    switch (dt) {
        case FTX_F32: eb = 1; bb = 4; return true;
        case FTX_F16: case FTX_BF16: eb = 1; bb = 2; return true;
        case FTX_Q4_0: eb = 32; bb = 18; return true;
        case FTX_Q4_1: eb = 32; bb = 20; return true;
        case FTX_Q8_0: eb = 32; bb = 34; return true;
        case FTX_Q4_K: eb = 256; bb = 144; return true;
        case FTX_Q6_K: eb = 256; bb = 210; return true;
        default: return false;
    }
}

class Cursor {
public:
    Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
    void need(uint64_t k) const {
        if (k > n_ - off_) throw std::runtime_error("gguf: truncated file");
    }
    template <typename T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p_ + off_, sizeof(T));
        off_ += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        need(n);
        std::string s((const char*)p_ + off_, (size_t)n);
        off_ += (size_t)n;
        return s;
    }
    Val value(uint32_t kind) {
        Val v;
        v.kind = kind;
        switch (kind) {
            case K_U8: v.i = get<uint8_t>(); break;
            case K_I8: v.i = get<int8_t>(); break;
            case K_U16: v.i = get<uint16_t>(); break;
            case K_I16: v.i = get<int16_t>(); break;
            case K_U32: v.i = get<uint32_t>(); break;
            case K_I32: v.i = get<int32_t>(); break;
            case K_U64: v.i = (int64_t)get<uint64_t>(); break;
            case K_I64: v.i = get<int64_t>(); break;
            case K_F32: v.f = get<float>(); break;
            case K_F64: v.f = get<double>(); break;
            case K_BOOL: v.b = get<uint8_t>() != 0; break;
            case K_STR: v.s = str(); break;
            case K_ARR: {
                v.ekind = get<uint32_t>();
                v.count = get<uint64_t>();
                if (v.ekind == K_STR) {
                    for (uint64_t i = 0; i < v.count; ++i) v.strs.push_back(str());
                } else if (kind_bytes(v.ekind)) {
                    const uint64_t nb = kind_bytes(v.ekind) * v.count;
                    if (v.count && nb / v.count != kind_bytes(v.ekind))
                        throw std::runtime_error("gguf: truncated file");
                    need(nb);
                    v.raw.assign(p_ + off_, p_ + off_ + nb);
                    off_ += (size_t)nb;
                } else {
                    throw std::runtime_error("gguf: unsupported array element type");
                }
                break;
            }
            default: throw std::runtime_error("gguf: unsupported kv type");
        }
        return v;
    }
    size_t offset() const { return off_; }

private:
    const uint8_t* p_;
    size_t n_;
    size_t off_ = 0;
};

}  // namespace

struct Gguf::Impl {
    int fd = -1;
    const uint8_t* data = nullptr;
    size_t size = 0;
    std::unordered_map<std::string, Val> kv;
    std::vector<std::string> order;  // keys in file order
    uint64_t data_start = 0;
    uint32_t align = 32;
    ~Impl() {
        if (data) munmap((void*)data, size);
        if (fd >= 0) ::close(fd);
    }
    const Val* find(const std::string& k) const {
        auto it = kv.find(k);
        return it == kv.end() ? nullptr : &it->second;
    }
};

Gguf::Gguf(const std::string& path) : impl_(new Impl) {
    Impl& I = *impl_;
    I.fd = ::open(path.c_str(), O_RDONLY);
    if (I.fd < 0) throw std::runtime_error("cannot open " + path);
    struct stat st {};
    if (fstat(I.fd, &st) != 0) throw std::runtime_error("cannot stat " + path);
    I.size = (size_t)st.st_size;
    if (I.size < 24) throw std::runtime_error("gguf: empty or tiny file");
    void* m = mmap(nullptr, I.size, PROT_READ, MAP_PRIVATE, I.fd, 0);
    if (m == MAP_FAILED) throw std::runtime_error("cannot map " + path);
    I.data = (const uint8_t*)m;

    Cursor c(I.data, I.size);
    if (c.get<uint32_t>() != kMagic) throw std::runtime_error("not a GGUF file");
    const uint32_t version = c.get<uint32_t>();
    if (version != 2 && version != 3)
        throw std::runtime_error("unsupported GGUF version " + std::to_string(version));
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = c.str();
        const uint32_t kind = c.get<uint32_t>();
        Val v = c.value(kind);
        if (I.kv.emplace(key, std::move(v)).second) I.order.push_back(key);
    }
    if (const Val* a = I.find("general.alignment")) {
        const int64_t al = (a->kind == K_STR) ? 0 : a->i;
        I.align = al > 0 && (al & (al - 1)) == 0 && al <= INT32_MAX ? (uint32_t)al : 32;
    }
    struct Info {
        std::string name;
        int32_t n_dims;
        int64_t ne[4];
        uint32_t dt;
        uint64_t off;
    };
    std::vector<Info> infos;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Info t{};
        t.name = c.str();
        t.n_dims = c.get<int32_t>();
        if (t.n_dims < 1 || t.n_dims > 4) throw std::runtime_error("gguf: bad dims for " + t.name);
        for (int d = 0; d < 4; ++d) t.ne[d] = 1;
        for (int d = 0; d < t.n_dims; ++d) t.ne[d] = (int64_t)c.get<uint64_t>();
        t.dt = c.get<uint32_t>();
        int64_t eb, bb;
        if (!block_of(t.dt, eb, bb))
            throw std::runtime_error("gguf: unsupported tensor dtype " + std::to_string(t.dt));
        t.off = c.get<uint64_t>();
        infos.push_back(std::move(t));
    }
    const uint64_t pos = (c.offset() + I.align - 1) / I.align * I.align;
    if (pos > I.size) throw std::runtime_error("gguf: data out of bounds");
    I.data_start = pos;
    for (const Info& t : infos) {
        if (tensors_.count(t.name)) continue;  // a repeated name keeps its first info
        int64_t eb, bb;
        block_of(t.dt, eb, bb);
        for (int d = 0; d < 4; ++d)
            if (t.ne[d] < 0) throw std::runtime_error("gguf: bad dims for " + t.name);
        const uint64_t row = (uint64_t)((t.ne[0] + eb - 1) / eb * bb);
        const uint64_t nb = row * (uint64_t)t.ne[1] * (uint64_t)t.ne[2] * (uint64_t)t.ne[3];
        const uint64_t room = I.size - pos;
        if (t.off > room || nb > room - t.off)
            throw std::runtime_error("gguf: tensor out of bounds: " + t.name);
        HostTensor h;
        h.name = t.name;
        for (int d = 0; d < 4; ++d) h.ne[d] = t.ne[d];
        h.n_dims = t.n_dims;
        h.dtype = (DType)t.dt;
        h.data = I.data + pos + t.off;
        h.nbytes = (size_t)nb;
        tensors_.emplace(t.name, std::move(h));
    }
}

Gguf::~Gguf() = default;

bool Gguf::has(const std::string& key) const { return impl_->find(key) != nullptr; }

std::string Gguf::get_str(const std::string& key, const std::string& def) const {
    const Val* v = impl_->find(key);
    return v && v->kind == K_STR ? v->s : def;
}

// src/gguf.cpp:258-265: every non-string kind answers with its integer slot,
// which holds 0 for floats, bools and arrays
int64_t Gguf::get_i64(const std::string& key, int64_t def) const {
    const Val* v = impl_->find(key);
    if (!v || v->kind == K_STR) return def;
    return v->i;
}

double Gguf::get_f64(const std::string& key, double def) const {
    const Val* v = impl_->find(key);
    if (!v || v->kind == K_STR) return def;
    if (v->kind == K_F32 || v->kind == K_F64) return v->f;
    return (double)v->i;
}

bool Gguf::get_bool(const std::string& key, bool def) const {
    const Val* v = impl_->find(key);
    return v && v->kind == K_BOOL ? v->b : def;
}

std::vector<std::string> Gguf::get_str_arr(const std::string& key) const {
    const Val* v = impl_->find(key);
    if (!v || v->kind != K_ARR || v->ekind != K_STR) return {};
    return v->strs;
}

// numeric arrays as float; string and bool arrays read as zeros of their
// length (src/gguf.cpp:288-330)
std::vector<float> Gguf::get_f32_arr(const std::string& key) const {
    const Val* v = impl_->find(key);
    if (!v || v->kind != K_ARR) return {};
    std::vector<float> out((size_t)v->count, 0.f);
    const uint8_t* r = v->raw.data();
    for (uint64_t i = 0; i < v->count; ++i) {
        switch (v->ekind) {
            case K_F32: { float f; std::memcpy(&f, r + i * 4, 4); out[i] = f; break; }
            case K_F64: { double d; std::memcpy(&d, r + i * 8, 8); out[i] = (float)d; break; }
            case K_U8: out[i] = (float)r[i]; break;
            case K_I8: out[i] = (float)(int8_t)r[i]; break;
            case K_U16: { uint16_t x; std::memcpy(&x, r + i * 2, 2); out[i] = (float)x; break; }
            case K_I16: { int16_t x; std::memcpy(&x, r + i * 2, 2); out[i] = (float)x; break; }
            case K_U32: { uint32_t x; std::memcpy(&x, r + i * 4, 4); out[i] = (float)x; break; }
            case K_I32: { int32_t x; std::memcpy(&x, r + i * 4, 4); out[i] = (float)x; break; }
            case K_U64: { uint64_t x; std::memcpy(&x, r + i * 8, 8); out[i] = (float)(int64_t)x; break; }
            case K_I64: { int64_t x; std::memcpy(&x, r + i * 8, 8); out[i] = (float)x; break; }
            default: break;  // strings, bools
        }
    }
    return out;
}

std::vector<int32_t> Gguf::get_i32_arr(const std::string& key) const {
    const std::vector<float> f = get_f32_arr(key);
    std::vector<int32_t> out(f.size());
    for (size_t i = 0; i < f.size(); ++i) out[i] = (int32_t)f[i];
    return out;
}

const HostTensor* Gguf::tensor(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

std::vector<std::string> Gguf::keys() const { return impl_->order; }

uint64_t Gguf::file_offset(const HostTensor& t) const {
    return (uint64_t)(t.data - impl_->data);
}

uint32_t Gguf::alignment() const { return impl_->align; }

// ---------------------------------------------------------------- config

namespace {

// src/graph.cpp:9-21: the arch's key, then the llama.* key
int64_t kv_i(const Gguf& g, const std::string& arch, std::initializer_list<const char*> sfx,
             int64_t def) {
    for (const char* s : sfx) {
        const int64_t v = g.get_i64(arch + "." + s, INT64_MIN);
        if (v != INT64_MIN) return v;
    }
    for (const char* s : sfx) {
        const int64_t v = g.get_i64(std::string("llama.") + s, INT64_MIN);
        if (v != INT64_MIN) return v;
    }
    return def;
}

}  // namespace

GgufConfig config_from_gguf(const Gguf& g) {
    GgufConfig r;
    ModelConfig& c = r.cfg;
    r.arch = g.get_str("general.architecture", "unknown");
    const std::string& a = r.arch;
    c.n_layer = kv_i(g, a, {"block_count"}, 0);
    c.n_embd = kv_i(g, a, {"embedding_length"}, 0);
    c.n_head = kv_i(g, a, {"attention.head_count"}, 0);
    c.n_head_kv = kv_i(g, a, {"attention.head_count_kv"}, c.n_head);
    c.head_dim = kv_i(g, a, {"attention.key_length", "attention.head_dim"},
                      c.n_head ? c.n_embd / c.n_head : 0);
    c.vocab = kv_i(g, a, {"vocab_size"}, 0);
    if (!c.vocab) c.vocab = (int64_t)g.get_str_arr("tokenizer.ggml.tokens").size();
    r.ctx_train = kv_i(g, a, {"context_length"}, 4096);
    // the epsilon goes through the integer accessor (src/graph.cpp:42-43): a
    // float-typed key reads as 0 and the default applies
    c.rms_eps = (float)kv_i(g, a, {"attention.layer_norm_rms_epsilon"}, 0);
    if (!c.rms_eps) c.rms_eps = 1e-5f;
    double theta = g.get_f64(a + ".rope.freq_base", 0);
    if (!theta) theta = g.get_f64("llama.rope.freq_base", 10000.0);
    c.rope_theta = theta;
    const int64_t ne = kv_i(g, a, {"expert_count"}, 0);
    const int64_t nu = kv_i(g, a, {"expert_used_count"}, 0);
    r.moe = ne > 1 && nu > 0;
    std::string al = a;
    std::transform(al.begin(), al.end(), al.begin(), [](unsigned char ch) { return (char)std::tolower(ch); });
    c.rope_neox = false;
    for (const char* n : {"qwen", "deepseek", "phi", "glm", "minicpm"})
        if (al.find(n) != std::string::npos) c.rope_neox = true;
    c.n_ff = kv_i(g, a, {"expert_feed_forward_length", "feed_forward_length"}, 0);
    if (!c.n_layer || !c.n_embd || !c.n_head || !c.head_dim || !c.vocab)
        throw std::runtime_error("gguf: incomplete model config for arch " + a);
    return r;
}

// ---------------------------------------------------------------- weights

namespace {

std::string layer_name(const char* pat, int64_t l) {
    char buf[256];
    std::snprintf(buf, sizeof(buf), pat, (int)l);
    return buf;
}

const HostTensor* first_of(const Gguf& g, int64_t l, std::initializer_list<const char*> pats) {
    for (const char* p : pats)
        if (const HostTensor* t = g.tensor(layer_name(p, l))) return t;
    return nullptr;
}

HostTensor as_matrix(const HostTensor& t) {
    HostTensor m = t;
    m.ne[1] = t.ne[1] * t.ne[2] * t.ne[3];
    m.ne[2] = m.ne[3] = 1;
    m.n_dims = 2;
    return m;
}

}  // namespace

ModelWeights weights_from_gguf(const Gguf& g, ModelConfig& cfg) {
    if (config_from_gguf(g).moe)
        throw std::runtime_error("gguf: MoE models go through run_expert_chunk, not the resident model");
    ModelWeights w;
    for (int64_t l = 0; l < cfg.n_layer; ++l) {
        const HostTensor* t[9] = {
            first_of(g, l, {"blk.%d.attn_norm.weight", "blk.%d.input_layernorm.weight"}),
            first_of(g, l, {"blk.%d.attn_q.weight", "blk.%d.self_attn.q_proj.weight"}),
            first_of(g, l, {"blk.%d.attn_k.weight", "blk.%d.self_attn.k_proj.weight"}),
            first_of(g, l, {"blk.%d.attn_v.weight", "blk.%d.self_attn.v_proj.weight"}),
            first_of(g, l, {"blk.%d.attn_output.weight", "blk.%d.self_attn.o_proj.weight"}),
            first_of(g, l, {"blk.%d.post_attention_norm.weight",
                            "blk.%d.post_attention_layernorm.weight", "blk.%d.ffn_norm.weight"}),
            first_of(g, l, {"blk.%d.ffn_gate.weight", "blk.%d.mlp.gate_proj.weight"}),
            first_of(g, l, {"blk.%d.ffn_up.weight", "blk.%d.mlp.up_proj.weight"}),
            first_of(g, l, {"blk.%d.ffn_down.weight", "blk.%d.mlp.down_proj.weight"})};
        static const char* roles[9] = {"attn_norm", "q", "k", "v", "o", "ffn_norm", "gate", "up",
                                       "down"};
        std::vector<HostTensor> L;
        for (int i = 0; i < 9; ++i) {
            if (!t[i])
                throw std::runtime_error(std::string("gguf: missing ") + roles[i] +
                                         " tensor at layer " + std::to_string(l));
            L.push_back(as_matrix(*t[i]));
        }
        for (const char* p : {"blk.%d.attn_q.bias", "blk.%d.attn_k.bias", "blk.%d.attn_v.bias",
                              "blk.%d.attn_q_norm.weight", "blk.%d.self_attn.q_norm.weight",
                              "blk.%d.attn_k_norm.weight", "blk.%d.self_attn.k_norm.weight",
                              "blk.%d.ffn_gate_inp.weight"})
            if (g.tensor(layer_name(p, l)))
                throw std::runtime_error("gguf: " + layer_name(p, l) +
                                         " is not supported by the resident model");
        w.layers.push_back(std::move(L));
    }
    const HostTensor* e = g.tensor("token_embd.weight");
    if (!e) throw std::runtime_error("gguf: missing token_embd.weight");
    const HostTensor* on = g.tensor("output_norm.weight");
    if (!on) throw std::runtime_error("gguf: missing output_norm.weight");
    w.tok_embd = as_matrix(*e);
    w.out_norm = as_matrix(*on);
    const HostTensor* o = g.tensor("output.weight");
    w.output = as_matrix(o ? *o : *e);  // tied embeddings
    if (!cfg.n_ff) cfg.n_ff = w.layers.empty() ? 0 : w.layers[0][6].rows();
    return w;
}

}  // namespace ftx_host
