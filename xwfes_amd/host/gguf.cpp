// gguf.cpp -- GGUF parser, model config and tensor lookup (see gguf.hpp).
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <unordered_map>
#include <variant>

namespace ftx_host {

// The container format as the GGUF specification lays it out (versions 2 and
// 3): a 24-byte header (magic "GGUF", version, tensor count, metadata
// count), the metadata entries (key string, type, value), the tensor
// directory (name, dims, sizes, dtype, offset into the data section), then
// the data section at the next multiple of general.alignment (32 unless the
// file says otherwise).  Strings are a u64 length and the bytes; arrays an
// element type, a u64 count and the elements.

namespace {

enum MetaType : uint32_t {
    MT_U8 = 0, MT_I8 = 1, MT_U16 = 2, MT_I16 = 3, MT_U32 = 4, MT_I32 = 5, MT_F32 = 6,
    MT_BOOL = 7, MT_STRING = 8, MT_ARRAY = 9, MT_U64 = 10, MT_I64 = 11, MT_F64 = 12,
    MT_END = 13
};

// bytes of a fixed-size metadata type (0: string, array, unknown)
int fixed_width(uint32_t t) {
    static const int8_t w[MT_END] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return t < MT_END ? w[t] : 0;
}

std::string fmt(const char* f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char* f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    std::vsnprintf(buf, sizeof(buf), f, ap);
    va_end(ap);
    return buf;
}

// The mapped file seen as a byte range with a read position; every read
// names the part of the file it belongs to, for the error message.
struct Span {
    const uint8_t* base;
    uint64_t size;
    uint64_t pos = 0;

    const uint8_t* take(uint64_t n, const char* part) {
        if (n > size - pos)
            throw std::runtime_error(
                fmt("gguf: the file ends inside the %s (byte %llu of %llu)", part,
                    (unsigned long long)pos, (unsigned long long)size));
        const uint8_t* at = base + pos;
        pos += n;
        return at;
    }
    template <typename T>
    T scalar(const char* part) {
        T v;
        std::memcpy(&v, take(sizeof(T), part), sizeof(T));
        return v;
    }
    std::string text(const char* part) {
        const uint64_t n = scalar<uint64_t>(part);
        const uint8_t* at = take(n, part);
        return std::string((const char*)at, (size_t)n);
    }
};

// A metadata array: its element type and count, the strings of a string
// array or the packed little-endian elements of a numeric one.
struct MetaArray {
    uint32_t elem = 0;
    uint64_t count = 0;
    std::vector<std::string> strings;
    std::vector<uint8_t> packed;
};

// A decoded metadata value: integers of every width widened to int64, both
// float widths to double.
struct Meta {
    uint32_t type = 0;
    std::variant<int64_t, double, bool, std::string, MetaArray> v;
};

int64_t widen_int(const uint8_t* p, uint32_t t) {
    switch (t) {
        case MT_U8: return p[0];
        case MT_I8: return (int8_t)p[0];
        case MT_U16: { uint16_t x; std::memcpy(&x, p, 2); return x; }
        case MT_I16: { int16_t x; std::memcpy(&x, p, 2); return x; }
        case MT_U32: { uint32_t x; std::memcpy(&x, p, 4); return x; }
        case MT_I32: { int32_t x; std::memcpy(&x, p, 4); return x; }
        case MT_U64: { uint64_t x; std::memcpy(&x, p, 8); return (int64_t)x; }
        case MT_I64: { int64_t x; std::memcpy(&x, p, 8); return x; }
        default: return 0;
    }
}

Meta decode_meta(Span& in, uint32_t type) {
    Meta m;
    m.type = type;
    switch (type) {
        case MT_F32: m.v = (double)in.scalar<float>("metadata"); break;
        case MT_F64: m.v = in.scalar<double>("metadata"); break;
        case MT_BOOL: m.v = in.scalar<uint8_t>("metadata") != 0; break;
        case MT_STRING: m.v = in.text("metadata"); break;
        case MT_ARRAY: {
            MetaArray a;
            a.elem = in.scalar<uint32_t>("metadata");
            a.count = in.scalar<uint64_t>("metadata");
            if (a.elem == MT_STRING) {
                for (uint64_t i = 0; i < a.count; ++i) a.strings.push_back(in.text("metadata"));
            } else if (const int w = fixed_width(a.elem)) {
                if (a.count > (in.size - in.pos) / (uint64_t)w)
                    throw std::runtime_error("gguf: a metadata array runs past the end of the file");
                const uint8_t* at = in.take(a.count * (uint64_t)w, "metadata");
                a.packed.assign(at, at + a.count * (uint64_t)w);
            } else {
                throw std::runtime_error(fmt("gguf: arrays of metadata type %u are not supported", a.elem));
            }
            m.v = std::move(a);
            break;
        }
        default: {
            const int w = fixed_width(type);
            if (!w) throw std::runtime_error(fmt("gguf: metadata type %u is not supported", type));
            m.v = widen_int(in.take((uint64_t)w, "metadata"), type);
        }
    }
    return m;
}

// (elements, bytes) of one block of a tensor dtype this library reads
bool dtype_block(uint32_t dt, int64_t& elems, int64_t& bytes) {
    switch (dt) {
        case FTX_F32: elems = 1; bytes = 4; return true;
        case FTX_F16: case FTX_BF16: elems = 1; bytes = 2; return true;
        case FTX_Q4_0: elems = 32; bytes = 18; return true;
        case FTX_Q4_1: elems = 32; bytes = 20; return true;
        case FTX_Q8_0: elems = 32; bytes = 34; return true;
        case FTX_Q4_K: elems = 256; bytes = 144; return true;
        case FTX_Q6_K: elems = 256; bytes = 210; return true;
        default: return false;
    }
}

struct DirEntry {
    std::string name;
    int32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint32_t dtype = 0;
    uint64_t offset = 0;
};

}  // namespace

struct Gguf::Impl {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    std::unordered_map<std::string, Meta> meta;
    std::vector<std::string> key_order;  // first occurrence of each key, in file order
    uint32_t align = 32;
    ~Impl() {
        if (map) munmap((void*)map, size);
        if (fd >= 0) ::close(fd);
    }
    const Meta* lookup(const std::string& k) const {
        const auto it = meta.find(k);
        return it == meta.end() ? nullptr : &it->second;
    }
};

Gguf::Gguf(const std::string& path) : impl_(new Impl) {
    Impl& F = *impl_;
    F.fd = ::open(path.c_str(), O_RDONLY);
    if (F.fd < 0) throw std::runtime_error("gguf: cannot open '" + path + "'");
    struct stat st {};
    if (fstat(F.fd, &st) != 0) throw std::runtime_error("gguf: cannot stat '" + path + "'");
    F.size = (size_t)st.st_size;
    if (F.size < 24) throw std::runtime_error("gguf: '" + path + "' is too small for a GGUF header");
    void* mp = mmap(nullptr, F.size, PROT_READ, MAP_PRIVATE, F.fd, 0);
    if (mp == MAP_FAILED) throw std::runtime_error("gguf: cannot map '" + path + "'");
    F.map = (const uint8_t*)mp;

    Span in{F.map, (uint64_t)F.size};
    if (std::memcmp(in.take(4, "header"), "GGUF", 4) != 0)
        throw std::runtime_error("gguf: bad magic, '" + path + "' is not a GGUF file");
    const uint32_t version = in.scalar<uint32_t>("header");
    if (version < 2 || version > 3)
        throw std::runtime_error(fmt("gguf: version %u is not supported (2 or 3 expected)", version));
    const uint64_t n_tensors = in.scalar<uint64_t>("header");
    const uint64_t n_meta = in.scalar<uint64_t>("header");

    for (uint64_t i = 0; i < n_meta; ++i) {
        std::string key = in.text("metadata");
        const uint32_t type = in.scalar<uint32_t>("metadata");
        Meta m = decode_meta(in, type);
        if (F.meta.emplace(key, std::move(m)).second) F.key_order.push_back(std::move(key));
    }
    // general.alignment is read through its integer slot and cut to 32 bits;
    // zero or a non-power of two keeps the default
    if (const Meta* a = F.lookup("general.alignment"))
        if (const int64_t* iv = std::get_if<int64_t>(&a->v)) {
            const uint32_t al = (uint32_t)*iv;
            if (al && !(al & (al - 1))) F.align = al;
        }

    std::vector<DirEntry> dir;
    dir.reserve((size_t)std::min<uint64_t>(n_tensors, 1u << 16));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        DirEntry e;
        e.name = in.text("tensor directory");
        e.n_dims = in.scalar<int32_t>("tensor directory");
        if (e.n_dims < 1 || e.n_dims > 4)
            throw std::runtime_error(fmt("gguf: tensor '%s' has %d dims (1 to 4 allowed)",
                                         e.name.c_str(), e.n_dims));
        for (int d = 0; d < e.n_dims; ++d)
            e.ne[d] = (int64_t)in.scalar<uint64_t>("tensor directory");
        e.dtype = in.scalar<uint32_t>("tensor directory");
        int64_t be, bb;
        if (!dtype_block(e.dtype, be, bb))
            throw std::runtime_error(fmt("gguf: tensor '%s' has dtype %u, which is not supported",
                                         e.name.c_str(), e.dtype));
        e.offset = in.scalar<uint64_t>("tensor directory");
        dir.push_back(std::move(e));
    }
    const uint64_t data0 = (in.pos + F.align - 1) / F.align * F.align;
    if (data0 > F.size) throw std::runtime_error("gguf: the data section starts past the end of the file");
    const uint64_t room = F.size - data0;

    for (const DirEntry& e : dir) {
        if (tensors_.count(e.name)) continue;  // a name listed twice keeps its first entry
        int64_t be, bb;
        dtype_block(e.dtype, be, bb);
        uint64_t nbytes = 0;
        bool fits = e.offset <= room;
        for (int d = 0; fits && d < 4; ++d) fits = e.ne[d] >= 0;
        if (fits) {
            // bytes = rows * row bytes, each product checked against the room left
            const uint64_t row = (uint64_t)((e.ne[0] + be - 1) / be) * (uint64_t)bb;
            nbytes = row;
            for (int d = 1; fits && d < 4; ++d) {
                const uint64_t n = (uint64_t)e.ne[d];
                fits = n == 0 || nbytes <= (room - e.offset) / n;
                nbytes *= n;
            }
            fits = fits && nbytes <= room - e.offset;
        }
        if (!fits) throw std::runtime_error("gguf: tensor '" + e.name + "' lies outside the file");
        HostTensor t;
        t.name = e.name;
        std::copy(e.ne, e.ne + 4, t.ne);
        t.n_dims = e.n_dims;
        t.dtype = (DType)e.dtype;
        t.data = F.map + data0 + e.offset;
        t.nbytes = (size_t)nbytes;
        tensors_.emplace(e.name, std::move(t));
    }
}

Gguf::~Gguf() = default;

bool Gguf::has(const std::string& key) const { return impl_->lookup(key) != nullptr; }

std::string Gguf::get_str(const std::string& key, const std::string& def) const {
    const Meta* m = impl_->lookup(key);
    const std::string* s = m ? std::get_if<std::string>(&m->v) : nullptr;
    return s ? *s : def;
}

// The typed accessors keep the reference's answers for every stored type
// (src/gguf.cpp:258-285): an integer read of a float, bool or array key is 0
// (not the default), a float read of an integer key converts it, and only a
// missing or string key gives the default.
int64_t Gguf::get_i64(const std::string& key, int64_t def) const {
    const Meta* m = impl_->lookup(key);
    if (!m || m->type == MT_STRING) return def;
    const int64_t* iv = std::get_if<int64_t>(&m->v);
    return iv ? *iv : 0;
}

double Gguf::get_f64(const std::string& key, double def) const {
    const Meta* m = impl_->lookup(key);
    if (!m || m->type == MT_STRING) return def;
    if (const double* dv = std::get_if<double>(&m->v)) return *dv;
    const int64_t* iv = std::get_if<int64_t>(&m->v);
    return iv ? (double)*iv : 0.0;
}

bool Gguf::get_bool(const std::string& key, bool def) const {
    const Meta* m = impl_->lookup(key);
    const bool* bv = m ? std::get_if<bool>(&m->v) : nullptr;
    return bv ? *bv : def;
}

std::vector<std::string> Gguf::get_str_arr(const std::string& key) const {
    const Meta* m = impl_->lookup(key);
    const MetaArray* a = m ? std::get_if<MetaArray>(&m->v) : nullptr;
    return a && a->elem == MT_STRING ? a->strings : std::vector<std::string>{};
}

// any array as floats, one per element: numbers converted, strings and bools
// as zeros (src/gguf.cpp:288-330)
std::vector<float> Gguf::get_f32_arr(const std::string& key) const {
    const Meta* m = impl_->lookup(key);
    const MetaArray* a = m ? std::get_if<MetaArray>(&m->v) : nullptr;
    if (!a) return {};
    std::vector<float> out((size_t)a->count, 0.f);
    const int w = a->elem == MT_BOOL ? 0 : fixed_width(a->elem);
    for (uint64_t i = 0; w && i < a->count; ++i) {
        const uint8_t* p = a->packed.data() + i * (uint64_t)w;
        if (a->elem == MT_F32) {
            float f;
            std::memcpy(&f, p, 4);
            out[i] = f;
        } else if (a->elem == MT_F64) {
            double f;
            std::memcpy(&f, p, 8);
            out[i] = (float)f;
        } else {
            out[i] = (float)widen_int(p, a->elem);
        }
    }
    return out;
}

std::vector<int32_t> Gguf::get_i32_arr(const std::string& key) const {
    const std::vector<float> f = get_f32_arr(key);
    return std::vector<int32_t>(f.begin(), f.end());
}

const HostTensor* Gguf::tensor(const std::string& name) const {
    const auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

std::vector<std::string> Gguf::keys() const { return impl_->key_order; }

uint64_t Gguf::file_offset(const HostTensor& t) const { return (uint64_t)(t.data - impl_->map); }

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
    c.n_expert = kv_i(g, a, {"expert_count"}, 0);
    c.n_expert_used = kv_i(g, a, {"expert_used_count"}, 0);
    r.moe = c.n_expert > 1 && c.n_expert_used > 0;
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
    ModelWeights w;
    // src/engine.cpp:318-387: MoE from the metadata, or from the first layer
    // holding a router and expert planes (then every later layer is MoE)
    bool moe = cfg.n_expert > 1 && cfg.n_expert_used > 0;
    bool any_ext = false;
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
        const HostTensor* x[FTX_LAYER_EXT] = {
            first_of(g, l, {"blk.%d.attn_q.bias"}),
            first_of(g, l, {"blk.%d.attn_k.bias"}),
            first_of(g, l, {"blk.%d.attn_v.bias"}),
            first_of(g, l, {"blk.%d.attn_q_norm.weight", "blk.%d.self_attn.q_norm.weight"}),
            first_of(g, l, {"blk.%d.attn_k_norm.weight", "blk.%d.self_attn.k_norm.weight"}),
            first_of(g, l, {"blk.%d.ffn_gate_inp.weight"}),
            first_of(g, l, {"blk.%d.ffn_gate_exps.weight"}),
            first_of(g, l, {"blk.%d.ffn_up_exps.weight"}),
            first_of(g, l, {"blk.%d.ffn_down_exps.weight"}),
            first_of(g, l, {"blk.%d.exp_probs_b.bias"}),
            first_of(g, l, {"blk.%d.ffn_gate_shexp.weight"}),
            first_of(g, l, {"blk.%d.ffn_up_shexp.weight"}),
            first_of(g, l, {"blk.%d.ffn_down_shexp.weight"})};
        if (!moe && x[FTX_X_GATE_INP] && x[FTX_X_GATE_EXPS]) moe = true;
        std::vector<HostTensor> L;
        for (int i = 0; i < 9; ++i) {
            if (i >= 6 && moe) {
                L.push_back(HostTensor{});  // the dense FFN has no place on a MoE layer
                continue;
            }
            if (!t[i])
                throw std::runtime_error(std::string("gguf: missing ") + roles[i] +
                                         " tensor at layer " + std::to_string(l));
            L.push_back(as_matrix(*t[i]));
        }
        std::vector<HostTensor> X(FTX_LAYER_EXT);
        if (moe) {
            if (!x[FTX_X_GATE_INP] || !x[FTX_X_GATE_EXPS] || !x[FTX_X_UP_EXPS] || !x[FTX_X_DOWN_EXPS])
                throw std::runtime_error("gguf: incomplete MoE tensors at layer " + std::to_string(l));
            if (!cfg.n_expert) {
                cfg.n_expert = x[FTX_X_GATE_EXPS]->ne[2];
                cfg.n_expert_used = cfg.n_expert >= 8 ? 8 : 2;
            }
            if (!cfg.n_ff) cfg.n_ff = x[FTX_X_GATE_EXPS]->rows();
        }
        for (int i = 0; i < FTX_LAYER_EXT; ++i) {
            if (!x[i]) continue;
            const bool moe_part = i >= FTX_X_GATE_INP;
            if (moe_part && !moe) continue;  // the reference reads them on MoE layers only
            // expert planes keep their three dims; the rest are matrices
            X[i] = (i == FTX_X_GATE_EXPS || i == FTX_X_UP_EXPS || i == FTX_X_DOWN_EXPS)
                       ? *x[i]
                       : as_matrix(*x[i]);
            any_ext = true;
        }
        w.layers.push_back(std::move(L));
        w.ext.push_back(std::move(X));
    }
    if (!moe) cfg.n_expert = cfg.n_expert_used = 0;
    if (!any_ext) w.ext.clear();
    const HostTensor* e = g.tensor("token_embd.weight");
    if (!e) throw std::runtime_error("gguf: missing token_embd.weight");
    const HostTensor* on = g.tensor("output_norm.weight");
    if (!on) throw std::runtime_error("gguf: missing output_norm.weight");
    w.tok_embd = as_matrix(*e);
    w.out_norm = as_matrix(*on);
    const HostTensor* o = g.tensor("output.weight");
    w.output = as_matrix(o ? *o : *e);  // tied embeddings
    if (!cfg.n_ff && !w.layers.empty() && w.layers[0][6].data) cfg.n_ff = w.layers[0][6].rows();
    return w;
}

}  // namespace ftx_host
