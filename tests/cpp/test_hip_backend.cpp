// test_hip_backend.cpp -- GPU tests of the C++ host mirror (HipBackend,
// HipVerifier) against the CPU oracle, in the style of the reference's own
// tests (src/tests/test_core.cpp: one function per property, CHECK with a
// message, non-zero exit on the first failure).
//
// Run by tests/test_gpu_host_cpp.py on a machine with a GPU; built by
// tests/cpp/Makefile (called from the package build).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../oracle/ftx_oracle.h"
#include "../../xwfes_amd/host/gguf.hpp"
#include "../../xwfes_amd/host/hip_backend.hpp"

using namespace ftx_host;

static int g_checks = 0;
#define CHECK(cond, msg)                                                   \
    do {                                                                   \
        ++g_checks;                                                        \
        if (!(cond)) {                                                     \
            std::fprintf(stderr, "CHECK failed: %s (%s:%d)\n", msg, __FILE__, \
                         __LINE__);                                        \
            std::exit(1);                                                  \
        }                                                                  \
    } while (0)

static std::mt19937_64 rng_gen(12345);
static float rnd() { return std::normal_distribution<float>(0.f, 1.f)(rng_gen); }

// quantised rows through the oracle's test quantiser
struct QTensor {
    std::vector<uint8_t> bytes;
    HostTensor t;
};
static QTensor make_tensor(DType dt, int64_t rows, int64_t cols, float scale, const char* name) {
    QTensor q;
    const int64_t rb = orc_row_bytes((int)dt, cols);
    q.bytes.resize((size_t)(rb * rows));
    std::vector<float> row((size_t)cols);
    for (int64_t r = 0; r < rows; ++r) {
        for (auto& v : row) v = rnd() * scale;
        if (orc_quantize_row(q.bytes.data() + r * rb, row.data(), (int)dt, cols) != 0) {
            std::fprintf(stderr, "quantise failed\n");
            std::exit(1);
        }
    }
    q.t.name = name;
    q.t.ne[0] = cols;
    q.t.ne[1] = rows;
    q.t.n_dims = 2;
    q.t.dtype = dt;
    q.t.data = q.bytes.data();
    q.t.nbytes = q.bytes.size();
    return q;
}

// max over rows of max|got - want| / max|want|
static double rel_err(const float* got, const float* want, int64_t M, int64_t N) {
    double worst = 0;
    for (int64_t m = 0; m < M; ++m) {
        double num = 0, den = 0;
        for (int64_t n = 0; n < N; ++n) {
            num = std::max(num, (double)std::fabs(got[m * N + n] - want[m * N + n]));
            den = std::max(den, (double)std::fabs(want[m * N + n]));
        }
        worst = std::max(worst, num / (den + 1e-30));
    }
    return worst;
}

static void test_backend_info(HipBackend& be) {
    CHECK(be.ready(), "backend ready");
    CHECK(be.name() == "hip", "backend name");
    const DeviceInfo d = be.info();
    CHECK(d.mem_bytes > 0 && !d.name.empty(), "device info");
    CHECK(!d.integrated && !d.uma, "discrete device");
}

// IBackend::matmul: y[m*N + n] per row (the CPU backend's M-row sum fixed)
static void test_matmul(HipBackend& be) {
    const DType dts[] = {DType::Q4_0, DType::Q8_0, DType::Q4_K, DType::Q6_K, DType::F32};
    for (DType dt : dts) {
        const int64_t K = 4096, N = 96;
        QTensor W = make_tensor(dt, N, K, 0.02f, "w");
        for (int64_t M : {1, 5, 8}) {
            std::vector<float> x((size_t)(M * K)), y((size_t)(M * N), -1.f), want((size_t)(M * N));
            for (auto& v : x) v = rnd();
            be.matmul(x.data(), M, K, W.t, y.data());
            orc_matmul(x.data(), M, K, W.bytes.data(), (int)dt, N, want.data());
            char msg[96];
            std::snprintf(msg, sizeof msg, "matmul dtype %d M %lld", (int)dt, (long long)M);
            CHECK(rel_err(y.data(), want.data(), M, N) < 1e-4, msg);
        }
        // the test's buffers are freed and their addresses reused: drop the
        // resident copy with them
        be.evict(W.t);
    }
    // the resident copy is reused: a second call with the same tensor agrees
    QTensor W = make_tensor(DType::Q4_K, 32, 4096, 0.02f, "w2");
    std::vector<float> x(4096), y1(32), y2(32);
    for (auto& v : x) v = rnd();
    be.matmul(x.data(), 1, 4096, W.t, y1.data());
    be.matmul(x.data(), 1, 4096, W.t, y2.data());
    CHECK(std::memcmp(y1.data(), y2.data(), sizeof(float) * 32) == 0, "matmul repeatable");
    bool threw = false;
    try {
        be.matmul(x.data(), 1, 2048, W.t, y1.data());
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK(threw, "matmul K mismatch throws");
}

// run_expert_chunk == the direct SwiGLU + down-axpy loop (the reference's
// chunker equivalence, src/tests/test_core.cpp:307-346, at its sizes: M 3,
// 48 neurons, K 16 for F32 and one 32-element block for the block formats).
// The device sums in a different order than the sequential CPU dot, so the
// error is measured against the largest output of each row.
static void test_expert_chunk(HipBackend& be) {
    std::vector<QTensor> keep;  // buffers stay alive: resident copies are keyed by address
    keep.reserve(16);
    for (DType dt : {DType::F32, DType::Q4_0, DType::Q8_0}) {
        const int64_t K = dt == DType::F32 ? 16 : 32, IC = 48, M = 3;
        keep.push_back(make_tensor(dt, IC, K, 0.5f, "gate"));
        keep.push_back(make_tensor(dt, IC, K, 0.5f, "up"));
        keep.push_back(make_tensor(dt, IC, K, 0.5f, "down"));
        const QTensor& g = keep[keep.size() - 3];
        const QTensor& u = keep[keep.size() - 2];
        const QTensor& d = keep[keep.size() - 1];
        std::vector<float> x((size_t)(M * K)), out((size_t)(M * K), 0.f), ref((size_t)(M * K), 0.f);
        for (auto& v : x) v = rnd();
        const int64_t rb = orc_row_bytes((int)dt, K);
        ExpertChunkJob job;
        job.x = x.data();
        job.out = out.data();
        job.gate = g.bytes.data();
        job.up = u.bytes.data();
        job.down = d.bytes.data();
        job.dt = dt;
        job.M = M;
        job.K = K;
        job.IC = IC;
        job.gate_up_row_stride = (size_t)rb;
        job.down_row_stride = (size_t)rb;
        be.run_expert_chunk(job);
        std::vector<float> drow((size_t)K);
        for (int64_t m = 0; m < M; ++m)
            for (int64_t i = 0; i < IC; ++i) {
                const float gv = orc_dot_row_f32(&x[(size_t)(m * K)], g.bytes.data() + i * rb, (int)dt, K);
                const float uv = orc_dot_row_f32(&x[(size_t)(m * K)], u.bytes.data() + i * rb, (int)dt, K);
                const float h = gv / (1.f + std::exp(-gv)) * uv;
                orc_dequant_row(drow.data(), d.bytes.data() + i * rb, (int)dt, K);
                for (int64_t k = 0; k < K; ++k) ref[(size_t)(m * K + k)] += h * drow[(size_t)k];
            }
        char msg[64];
        std::snprintf(msg, sizeof msg, "chunked expert equivalence, dtype %d", (int)dt);
        CHECK(rel_err(out.data(), ref.data(), M, K) < 1e-4, msg);
    }
}

// accept_chain_greedy's reference known answer (src/tests/test_core.cpp:348-356)
static void test_accept_chain(HipBackend& be) {
    const int64_t V = 4;
    const float base[V] = {9, 1, 1, 1};
    const float rows[3 * V] = {1, 9, 1, 1, 1, 1, 9, 1, 1, 1, 1, 9};
    float* dev = (float*)be.alloc_staging(sizeof(float) * 4 * V);
    CHECK(dev != nullptr, "staging");
    be.stage(dev, base, sizeof(base));
    be.stage(dev + V, rows, sizeof(rows));
    uint64_t s = 7;
    Accepted a1 = accept_on_device(be, V, dev, dev + V, {0, 1, 2}, AcceptMode::Greedy, 1.f, s);
    Accepted a2 = accept_on_device(be, V, dev, dev + V, {0, 3, 2}, AcceptMode::Greedy, 1.f, s);
    CHECK(a1.nodes.size() == 3, "accept full");
    CHECK(a2.nodes.size() == 1, "reject early");
    CHECK(a1.bonus == 3 && a2.bonus == 1, "bonus = argmax of the row after the last accepted");
    be.free_staging(dev);
}

// HipVerifier: a 2-layer model, chain and tree verify against the oracle
// forward, then greedy and ratio acceptance against the oracle's
static void test_verifier(HipBackend& be) {
    ModelConfig c;
    c.n_layer = 2;
    c.n_embd = 256;
    c.n_head = 4;
    c.n_head_kv = 2;
    c.head_dim = 64;
    c.n_ff = 512;
    c.vocab = 512;
    c.rope_theta = 10000.0;
    std::vector<QTensor> keep;
    auto add = [&](DType dt, int64_t rows, int64_t cols, float scale, const char* nm) -> HostTensor {
        keep.push_back(make_tensor(dt, rows, cols, scale, nm));
        return keep.back().t;
    };
    keep.reserve(64);
    ModelWeights w;
    w.tok_embd = add(DType::F32, c.vocab, c.n_embd, 1.f, "tok_embd");
    // RMSNorm weights of 1 + 0.3 N(0, 1), one vector per
    // layer and role, so that a norm applied with the wrong vector shows
    std::vector<std::vector<float>> norms((size_t)(2 * c.n_layer + 1));
    for (auto& v : norms) {
        v.resize((size_t)c.n_embd);
        for (auto& x : v) x = 1.f + 0.3f * rnd();
    }
    auto norm_of = [&](size_t i) {
        HostTensor t;
        t.ne[0] = c.n_embd;
        t.dtype = DType::F32;
        t.data = (const uint8_t*)norms[i].data();
        t.nbytes = norms[i].size() * 4;
        return t;
    };
    w.out_norm = norm_of(2 * (size_t)c.n_layer);
    w.output = add(DType::Q6_K, c.vocab, c.n_embd, 0.05f, "output");
    const int64_t kdim = c.n_head_kv * c.head_dim, qdim = c.n_head * c.head_dim;
    for (int64_t l = 0; l < c.n_layer; ++l) {
        std::vector<HostTensor> L(9);
        L[0] = norm_of(2 * (size_t)l);
        L[1] = add(DType::Q4_K, qdim, c.n_embd, 0.05f, "q");
        L[2] = add(DType::Q4_K, kdim, c.n_embd, 0.05f, "k");
        L[3] = add(DType::Q6_K, kdim, c.n_embd, 0.05f, "v");
        L[4] = add(DType::Q4_K, c.n_embd, qdim, 0.05f, "o");
        L[5] = norm_of(2 * (size_t)l + 1);
        L[6] = add(DType::Q4_K, c.n_ff, c.n_embd, 0.05f, "gate");
        L[7] = add(DType::Q4_K, c.n_ff, c.n_embd, 0.05f, "up");
        L[8] = add(DType::Q4_K, c.n_ff, c.n_embd, 0.05f, "down");  // n_ff rows x n_embd cols
        w.layers.push_back(L);
    }
    const int64_t cap = 96, npast = 40, M = 6;
    HipVerifier ver(be, c, w, cap, 16);
    // committed context: random fp16 K/V in the reference layout
    std::vector<uint16_t> kc((size_t)(c.n_layer * cap * kdim)), vc(kc.size());
    for (auto& v : kc) v = orc_float_to_half(rnd());
    for (auto& v : vc) v = orc_float_to_half(rnd());
    ver.write_kv(kc.data(), vc.data());
    ver.truncate_to(npast);
    CHECK(ver.npast() == npast, "truncate_to");

    // the oracle model over the same bytes
    std::vector<orc_tensor> ol;
    auto ot = [](const HostTensor& t) {
        orc_tensor o{};
        o.data = t.data;
        o.dtype = (int32_t)t.dtype;
        o.ne0 = t.ne[0];
        o.ne1 = t.ne[1];
        return o;
    };
    for (const auto& L : w.layers)
        for (const auto& t : L) ol.push_back(ot(t));
    orc_model om{};
    om.n_layer = c.n_layer;
    om.n_embd = c.n_embd;
    om.n_head = c.n_head;
    om.n_head_kv = c.n_head_kv;
    om.head_dim = c.head_dim;
    om.n_ff = c.n_ff;
    om.vocab = c.vocab;
    om.rms_eps = c.rms_eps;
    om.rope_neox = 0;
    om.rope_theta = c.rope_theta;
    om.tok_embd = ot(w.tok_embd);
    om.out_norm = ot(w.out_norm);
    om.output = ot(w.output);
    om.layers = ol.data();

    const std::vector<int32_t> props = {5, 77, 300, 12, 9, 401};
    for (int tree = 0; tree < 2; ++tree) {
        const std::vector<int32_t> parents =
            tree ? std::vector<int32_t>{-1, 0, 0, 1, 1, 2} : std::vector<int32_t>{};
        const float* dev = ver.extend_verify(props, parents);
        std::vector<float> got((size_t)(M * c.vocab)), want(got.size());
        be.stage(got.data(), dev, got.size() * sizeof(float));
        std::vector<uint16_t> k2 = kc, v2 = vc;
        CHECK(orc_forward(&om, k2.data(), v2.data(), ORC_KV_F16, cap, npast, props.data(), M,
                          tree ? parents.data() : nullptr, 0, want.data()) == 0,
              "oracle forward");
        CHECK(rel_err(got.data(), want.data(), M, c.vocab) < 1e-3, tree ? "tree logits" : "chain logits");
        if (tree) {
            // accept the path 0 -> 1 -> 3, commit it, verify one more token:
            // the logits are the oracle chain forward of the path + that token
            const std::vector<int32_t> path = {0, 1, 3};
            ver.commit(path);
            CHECK(ver.npast() == npast + 3, "commit advances the committed length");
            const std::vector<int32_t> nxt = {42};
            const float* d1 = ver.extend_verify(nxt);
            std::vector<float> g1((size_t)c.vocab), w1((size_t)(4 * c.vocab));
            be.stage(g1.data(), d1, g1.size() * sizeof(float));
            std::vector<uint16_t> k4 = kc, v4 = vc;
            const int32_t chain[4] = {props[0], props[1], props[3], nxt[0]};
            CHECK(orc_forward(&om, k4.data(), v4.data(), ORC_KV_F16, cap, npast, chain, 4, nullptr,
                              0, w1.data()) == 0,
                  "oracle chain of the committed path");
            CHECK(rel_err(g1.data(), w1.data() + 3 * c.vocab, 1, c.vocab) < 1e-3,
                  "logits after commit");
            ver.truncate_to(npast);
            continue;
        }
        // acceptance on these logits: base row = oracle logits of position npast - 1
        std::vector<float> base((size_t)c.vocab);
        {
            std::vector<uint16_t> k3 = kc, v3 = vc;
            const int32_t t0 = 3;
            CHECK(orc_forward(&om, k3.data(), v3.data(), ORC_KV_F16, cap, npast - 1, &t0, 1,
                              nullptr, 0, base.data()) == 0,
                  "oracle base row");
        }
        float* dbase = (float*)be.alloc_staging(base.size() * sizeof(float));
        be.stage(dbase, base.data(), base.size() * sizeof(float));
        for (AcceptMode mode : {AcceptMode::Greedy, AcceptMode::Ratio}) {
            const std::vector<float> pd = {0.3f, 0.5f, 0.9f, 0.2f, 0.6f, 0.7f};
            uint64_t s_gpu = 5, s_orc = 5;
            const bool ratio = mode == AcceptMode::Ratio;
            uint64_t ss_orc = ver.sampler.state;
            Accepted a = ver.accept(dbase, dev, props, mode, 0.8f, s_gpu,
                                    ratio ? pd : std::vector<float>{});
            std::vector<int32_t> acc((size_t)M);
            int32_t n_acc = 0, bonus = -1;
            float margin = 0.f;
            CHECK(orc_verify_accept(base.data(), got.data(), M, c.vocab, props.data(), nullptr,
                                    ratio ? pd.data() : nullptr, nullptr, (int)mode, 0.8f, &s_orc,
                                    &ss_orc, ver.sampler.top_k, ver.sampler.top_p, acc.data(),
                                    &n_acc, &bonus, &margin) == 0,
                  "oracle accept");
            CHECK(ver.sampler.state == ss_orc, "sampler state matches the oracle");
            CHECK((int32_t)a.nodes.size() == n_acc, "accepted count matches the oracle");
            for (int32_t i = 0; i < n_acc; ++i) CHECK(a.nodes[(size_t)i] == acc[(size_t)i], "accepted ids");
            CHECK(a.bonus == bonus, "bonus token matches the oracle");
            CHECK(s_gpu == s_orc, "rng state matches the oracle");
        }
        be.free_staging(dbase);
    }

    // two sequences in one batched step: the verifier's own cache (a chain,
    // advancing) and a second sequence with its own history (a tree); each
    // one's logits equal the oracle forward of that sequence alone
    {
        const int64_t np2 = 29;
        HipSequence seq(ver, cap);
        std::vector<uint16_t> kb(kc.size()), vb(kc.size());
        for (auto& v : kb) v = orc_float_to_half(rnd());
        for (auto& v : vb) v = orc_float_to_half(rnd());
        seq.write_kv(kb.data(), vb.data());
        seq.truncate_to(np2);
        CHECK(seq.npast() == np2 && ver.npast() == npast, "batch histories");
        const std::vector<int32_t> pa = {7, 250, 31}, pb = {11, 400, 2, 99, 64};
        const std::vector<int32_t> parb = {-1, 0, 0, 2, 1};
        float* la = (float*)be.alloc_staging(pa.size() * c.vocab * sizeof(float));
        float* lb = (float*)be.alloc_staging(pb.size() * c.vocab * sizeof(float));
        std::vector<HipVerifier::BatchItem> items(2);
        items[0].props = pa;
        items[0].logits = la;
        items[0].advance = true;
        items[1].seq = &seq;
        items[1].props = pb;
        items[1].parents = parb;
        items[1].logits = lb;
        ver.verify_batch(items);
        CHECK(ver.npast() == npast + (int64_t)pa.size(), "an advancing item moves its cache");
        CHECK(seq.npast() == np2, "a non-advancing item leaves its cache");
        std::vector<float> ga(pa.size() * c.vocab), wa(ga.size()), gb(pb.size() * c.vocab),
            wb(gb.size());
        be.stage(ga.data(), la, ga.size() * sizeof(float));
        be.stage(gb.data(), lb, gb.size() * sizeof(float));
        std::vector<uint16_t> k5 = kc, v5 = vc, k6 = kb, v6 = vb;
        CHECK(orc_forward(&om, k5.data(), v5.data(), ORC_KV_F16, cap, npast, pa.data(),
                          (int64_t)pa.size(), nullptr, 0, wa.data()) == 0,
              "oracle forward, sequence 0");
        CHECK(orc_forward(&om, k6.data(), v6.data(), ORC_KV_F16, cap, np2, pb.data(),
                          (int64_t)pb.size(), parb.data(), 0, wb.data()) == 0,
              "oracle forward, sequence 1");
        CHECK(rel_err(ga.data(), wa.data(), (int64_t)pa.size(), c.vocab) < 1e-3,
              "batched chain logits");
        CHECK(rel_err(gb.data(), wb.data(), (int64_t)pb.size(), c.vocab) < 1e-3,
              "batched tree logits");
        // the second sequence keeps its tree path 0 -> 2 -> 3; one more
        // batched step over it alone continues from that path
        seq.commit({0, 2, 3});
        CHECK(seq.npast() == np2 + 3, "commit on a sequence");
        std::vector<HipVerifier::BatchItem> one(1);
        one[0].seq = &seq;
        one[0].props = {123};
        one[0].logits = lb;
        ver.verify_batch(one);
        std::vector<float> g1((size_t)c.vocab), w1((size_t)(4 * c.vocab));
        be.stage(g1.data(), lb, g1.size() * sizeof(float));
        std::vector<uint16_t> k7 = kb, v7 = vb;
        const int32_t chain[4] = {pb[0], pb[2], pb[3], 123};
        CHECK(orc_forward(&om, k7.data(), v7.data(), ORC_KV_F16, cap, np2, chain, 4, nullptr, 0,
                          w1.data()) == 0,
              "oracle chain of the sequence's path");
        CHECK(rel_err(g1.data(), w1.data() + 3 * c.vocab, 1, c.vocab) < 1e-3,
              "batched logits after a sequence commit");
        bool threw = false;
        try {
            std::vector<HipVerifier::BatchItem> bad(2);
            bad[0].props = {1};
            bad[0].logits = la;
            bad[1].props = {2};  // the verifier's cache twice
            bad[1].logits = lb;
            ver.verify_batch(bad);
        } catch (const std::runtime_error&) {
            threw = true;
        }
        CHECK(threw, "a cache given twice is refused");
        be.free_staging(la);
        be.free_staging(lb);
        ver.truncate_to(npast);
    }
}

// a GGUF model through the C++ loader: Gguf -> config_from_gguf ->
// weights_from_gguf -> HipVerifier, a chain verify against the oracle run on
// the same mapped bytes
static void test_gguf_verifier(HipBackend& be, const char* path) {
    Gguf g(path);
    GgufConfig gc = config_from_gguf(g);
    ModelConfig& c = gc.cfg;
    ModelWeights w = weights_from_gguf(g, c);
    CHECK(w.layers[0][6].data ? c.n_ff == w.layers[0][6].rows() : c.n_expert > 1,
          "n_ff from the gate rows");
    const int64_t cap = 64, npast = 9, M = 5;
    const int64_t kdim = c.n_head_kv * c.head_dim;
    {
    HipVerifier ver(be, c, w, cap, 8);
    std::vector<uint16_t> kc((size_t)(c.n_layer * cap * kdim)), vc(kc.size());
    for (auto& v : kc) v = orc_float_to_half(rnd());
    for (auto& v : vc) v = orc_float_to_half(rnd());
    ver.write_kv(kc.data(), vc.data());
    ver.truncate_to(npast);
    // the oracle takes every tensor as ne0 columns of all its rows
    auto ot = [](const HostTensor& t) {
        orc_tensor o{};
        o.data = t.data;
        o.dtype = (int32_t)t.dtype;
        o.ne0 = t.ne[0];
        o.ne1 = t.ne[1] * t.ne[2] * t.ne[3];
        return o;
    };
    std::vector<orc_tensor> ol, ox;
    for (const auto& L : w.layers)
        for (const auto& t : L) ol.push_back(ot(t));
    for (const auto& X : w.ext)
        for (const auto& t : X) ox.push_back(ot(t));
    orc_model om{};
    om.n_layer = c.n_layer;
    om.n_embd = c.n_embd;
    om.n_head = c.n_head;
    om.n_head_kv = c.n_head_kv;
    om.head_dim = c.head_dim;
    om.n_ff = c.n_ff;
    om.vocab = c.vocab;
    om.rms_eps = c.rms_eps;
    om.rope_neox = c.rope_neox ? 1 : 0;
    om.rope_theta = c.rope_theta;
    om.tok_embd = ot(w.tok_embd);
    om.out_norm = ot(w.out_norm);
    om.output = ot(w.output);
    om.layers = ol.data();
    om.ext = ox.empty() ? nullptr : ox.data();
    om.n_expert = c.n_expert;
    om.n_expert_used = c.n_expert_used;
    const std::vector<int32_t> toks = {1, (int32_t)c.vocab - 1, 7, 0, 3};
    const float* dev = ver.extend_verify(toks);
    std::vector<float> got((size_t)(M * c.vocab)), want(got.size());
    be.stage(got.data(), dev, got.size() * sizeof(float));
    std::vector<uint16_t> k2 = kc, v2 = vc;
    CHECK(orc_forward(&om, k2.data(), v2.data(), ORC_KV_F16, cap, npast, toks.data(), M, nullptr,
                      0, want.data()) == 0,
          "oracle forward of the GGUF model");
    CHECK(rel_err(got.data(), want.data(), M, c.vocab) < 1e-3, "GGUF model logits");
    // Engine::prefill + Engine::step from an empty cache: 13 prompt tokens in
    // chains of 8 (+5), then one step, against the forward of all 14
    {
        std::vector<int32_t> prompt;
        for (int i = 0; i < 13; ++i) prompt.push_back((int32_t)((i * 37 + 5) % c.vocab));
        const int32_t nxt = (int32_t)(c.vocab / 2);
        ver.truncate_to(0);
        const float* pl = ver.prefill(prompt, 8);
        std::vector<float> gp((size_t)(5 * c.vocab)), gs((size_t)c.vocab);
        be.stage(gp.data(), pl, gp.size() * sizeof(float));
        const float* sl = ver.step(nxt);
        be.stage(gs.data(), sl, gs.size() * sizeof(float));
        CHECK(ver.npast() == 14, "prefill + step advance the cache");
        std::vector<int32_t> all = prompt;
        all.push_back(nxt);
        std::vector<float> w14((size_t)(14 * c.vocab));
        std::vector<uint16_t> k3(kc.size(), 0), v3(vc.size(), 0);
        CHECK(orc_forward(&om, k3.data(), v3.data(), ORC_KV_F16, cap, 0, all.data(), 14, nullptr,
                          0, w14.data()) == 0,
              "oracle forward of prompt + step");
        CHECK(rel_err(gp.data(), w14.data() + 8 * c.vocab, 5, c.vocab) < 1e-3, "prefill logits");
        CHECK(rel_err(gs.data(), w14.data() + 13 * c.vocab, 1, c.vocab) < 1e-3, "step logits");
    }
    std::printf("gguf model %s: %lld layers, d %lld, vocab %lld verified\n", path,
                (long long)c.n_layer, (long long)c.n_embd, (long long)c.vocab);
    }
    // the resident copies are keyed by host address: drop them before the
    // mapping goes away (the verifier, which reads them, is gone already)
    for (const auto& L : w.layers)
        for (const auto& t : L) be.evict(t);
    be.evict(w.tok_embd);
    be.evict(w.out_norm);
    be.evict(w.output);
}

// speculative generate through the C++ host path: target and draft models
// from GGUF files (C++ loader), DraftModelDrafter + generate on the device;
// prints the emitted tokens and the round statistics for the caller to
// compare with the oracle's generate.
// args: target.gguf draft.gguf temp spec_k max_new cap prompt tokens...
static int run_generate(HipBackend& be, int argc, char** argv) {
    if (argc < 9) {
        std::fprintf(stderr, "--generate target draft temp spec_k max_new cap tokens...\n");
        return 2;
    }
    const float temp = (float)std::atof(argv[4]);
    const int spec_k = std::atoi(argv[5]);
    const int64_t max_new = std::atoll(argv[6]), cap = std::atoll(argv[7]);
    std::vector<int32_t> prompt;
    for (int i = 8; i < argc; ++i) prompt.push_back((int32_t)std::atoi(argv[i]));
    Gguf gt(argv[2]), gd(argv[3]);
    GgufConfig ct = config_from_gguf(gt), cd = config_from_gguf(gd);
    ModelWeights wt = weights_from_gguf(gt, ct.cfg), wd = weights_from_gguf(gd, cd.cfg);
    std::vector<int32_t> out;
    GenerateStats st;
    {
        HipVerifier target(be, ct.cfg, wt, cap, 8), draft(be, cd.cfg, wd, cap, 8);
        DraftModelDrafter drafter(draft);
        // the end-of-sequence id as the reference's tokenizer reads it
        // (src/tokenizer.cpp:68)
        const int32_t eos = (int32_t)gt.get_i64("tokenizer.ggml.eos_token_id", -1);
        out = generate(target, drafter, prompt, max_new, spec_k, temp, 40, 0.95f, 0, &st, eos);
    }
    std::printf("generate tokens:");
    for (int32_t t : out) std::printf(" %d", t);
    std::printf("\ngenerate stats: %lld %lld %lld %d\n", (long long)st.rounds,
                (long long)st.drafted, (long long)st.accepted, st.hit_eos ? 1 : 0);
    for (ModelWeights* w : {&wt, &wd}) {
        for (const auto& L : w->layers)
            for (const auto& t : L) be.evict(t);
        be.evict(w->tok_embd);
        be.evict(w->out_norm);
        be.evict(w->output);
    }
    return 0;
}

int main(int argc, char** argv) {
    HipBackend be(0);
    if (argc > 1 && !std::strcmp(argv[1], "--generate")) return run_generate(be, argc, argv);
    if (argc > 2 && !std::strcmp(argv[1], "--gguf")) {
        for (int i = 2; i < argc; ++i) test_gguf_verifier(be, argv[i]);
        std::printf("test_hip_backend: all %d checks passed\n", g_checks);
        return 0;
    }
    test_backend_info(be);
    test_matmul(be);
    test_expert_chunk(be);
    test_accept_chain(be);
    test_verifier(be);
    std::printf("test_hip_backend: all %d checks passed\n", g_checks);
    return 0;
}
