"""GPU parity of the verify step (ftx_verify_step) and of the acceptance
sampler (ftx_accept) against the CPU oracle, through the C ABI.

Logits: per row max|gpu - oracle| / max|oracle| <= 1e-3 (LOGIT_TOL), fp32
accumulation on both sides in different orders.
Acceptance: given identical logits and the same SplitMix64 state, accepted
node lists, bonus tokens and the advanced rng state are identical.
"""
import numpy as np
import pytest

import pyoracle as P
from builders import norm_raw, q_rows
from xwfes_amd import ftx

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def rel_err_rows(a, b):
    a = np.atleast_2d(a).astype(np.float64)
    b = np.atleast_2d(b).astype(np.float64)
    return (np.abs(a - b).max(axis=1) / np.maximum(np.abs(b).max(axis=1), 1e-30)).max()


def upload_model(gctx, model):
    cfg = model["cfg"]
    tensors = {}
    for name, t in model.items():
        if name == "cfg":
            continue
        tensors[name] = gctx.upload(t["raw"], t["dtype"], (t["ne0"], t["ne1"]))
    return tensors


def free_all(tensors):
    for t in tensors.values():
        t.free()


def kv_context(cfg, cap, npast, seed):
    rng = np.random.default_rng(seed)
    shape = (cfg["n_layer"], cap, cfg["n_head_kv"] * cfg["head_dim"])
    k = np.zeros(shape, np.float16)
    v = np.zeros(shape, np.float16)
    k[:, :npast] = rng.standard_normal((shape[0], npast, shape[2]))
    v[:, :npast] = rng.standard_normal((shape[0], npast, shape[2]))
    return k, v


def run_both(gctx, orc, model, toks, npast, cap, parents=None, seed=5):
    cfg = model["cfg"]
    tensors = upload_model(gctx, model)
    gm = gctx.model(cfg, tensors, max_tokens=max(8, len(toks)))
    kv = gm.kv(cap)
    k0, v0 = kv_context(cfg, cap, npast, seed)
    kv.write(k0, v0)
    kv.truncate(npast)
    M, V = len(toks), cfg["vocab"]
    buf = gctx.buffer(M * V * 4)
    gm.verify(kv, toks, buf.ptr, parents=parents)
    gctx.sync()
    got = buf.read(np.float32, M * V).reshape(M, V)
    kg, vg = kv.read()
    kc, vc = k0.copy(), v0.copy()
    want = orc.forward(model, kc, vc, npast, toks, parents=parents)
    buf.free()
    kv.free()
    gm.free()
    free_all(tensors)
    return got, want, (kg, vg), (kc, vc)


TINY = P.model_cfg(2, 64, 4, 2, 16, 96, 50, rope_theta=10000.0)
TINY_DT = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q4_0, k=P.Q8_0, v=P.Q4_0, o=P.Q8_0,
               gate=P.Q4_0, up=P.Q4_0, down=P.Q8_0)


def test_verify_chain_tiny(gctx, orc):
    model = P.make_model(orc, TINY, TINY_DT, seed=3)
    got, want, (kg, vg), (kc, vc) = run_both(gctx, orc, model, [3, 17, 42, 0, 9], 7, 32)
    assert rel_err_rows(got, want) < LOGIT_TOL
    # the draft rows written to the cache agree to fp16 rounding
    assert np.abs(kg.astype(np.float32) - kc.astype(np.float32)).max() < 2e-2
    assert np.abs(vg.astype(np.float32) - vc.astype(np.float32)).max() < 2e-2
    assert np.array_equal(kg[:, :7], kc[:, :7])


def test_verify_tree_tiny(gctx, orc):
    model = P.make_model(orc, TINY, TINY_DT, seed=4)
    parents = [-1, -1, 0, 0, 3, 1, 5]
    got, want, _, _ = run_both(gctx, orc, model, [5, 6, 7, 8, 9, 10, 11], 6, 32, parents=parents)
    assert rel_err_rows(got, want) < LOGIT_TOL


def test_verify_tree_equals_paths_on_gpu(gctx, orc):
    """Tree invariant on the device: node i's logits equal the chain forward
    of its root-to-i path."""
    model = P.make_model(orc, TINY, TINY_DT, seed=8)
    cfg = model["cfg"]
    tensors = upload_model(gctx, model)
    gm = gctx.model(cfg, tensors, max_tokens=8)
    kv = gm.kv(32)
    k0, v0 = kv_context(cfg, 32, 6, 9)
    parents = [-1, -1, 0, 0, 3]
    toks = [5, 6, 7, 8, 9]
    V = cfg["vocab"]
    buf = gctx.buffer(8 * V * 4)
    kv.write(k0, v0)
    kv.truncate(6)
    gm.verify(kv, toks, buf.ptr, parents=parents)
    gctx.sync()
    tree = buf.read(np.float32, 5 * V).reshape(5, V)
    paths = {0: [0], 1: [1], 2: [0, 2], 3: [0, 3], 4: [0, 3, 4]}
    for node, path in paths.items():
        kv.write(k0, v0)
        kv.truncate(6)
        gm.verify(kv, [toks[i] for i in path], buf.ptr)
        gctx.sync()
        chain = buf.read(np.float32, len(path) * V).reshape(len(path), V)
        assert rel_err_rows(chain[-1], tree[node]) < 1e-5, node
    buf.free()
    kv.free()
    gm.free()
    free_all(tensors)


HD128 = P.model_cfg(1, 1024, 8, 2, 128, 1024, 1000, rope_theta=500000.0)
HD128_DT = dict(tok_embd=P.Q8_0, output=P.Q8_0, q=P.Q8_0, k=P.Q8_0, v=P.Q8_0, o=P.Q8_0,
                gate=P.Q8_0, up=P.Q8_0, down=P.Q8_0)


@pytest.mark.parametrize("npast,parents", [
    (1000, None),                                   # chain over 16 context chunks
    (77, [-1, -1, 0, 0, 1, 1, 2, 3, 3, 4, 7, 7]),   # tree, context not chunk aligned
    (0, [-1, 0, 0, 1, 1, 2]),                        # tree with no context at all
    (64, [-1] * 9),                                  # 9 siblings: 36 query rows, 2 tiles
])
def test_verify_mfma_attention(gctx, orc, npast, parents):
    """head_dim 128 / fp16 KV takes the chunked MFMA attention; the chain and
    tree masks, chunk boundaries and query tiles agree with the oracle."""
    model = P.make_model(orc, HD128, HD128_DT, seed=11)
    M = 8 if parents is None else len(parents)
    toks = list(np.random.default_rng(npast).integers(0, 1000, M))
    got, want, _, _ = run_both(gctx, orc, model, toks, npast, npast + M + 5, parents=parents)
    assert rel_err_rows(got, want) < LOGIT_TOL


def test_verify_mfma_down(gctx, orc):
    """ffn_down in Q4_K (layer 0) and Q6_K (layer 1) takes the re-tiled MFMA
    down kernel (two 256-column super-blocks, 32 row slices)."""
    cfg = P.model_cfg(2, 512, 4, 1, 128, 1024, 500, rope_theta=10000.0)
    model = {"cfg": dict(cfg)}
    rng = np.random.default_rng(31)

    def q(rows, cols, dt):
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        return dict(raw=orc.quantize(w, dt), dtype=dt, ne0=cols, ne1=rows)

    model["tok_embd"] = q(500, 512, P.Q8_0)
    model["output"] = q(500, 512, P.Q8_0)
    model["out_norm"] = norm_raw(rng, 512)
    for l, ddt in enumerate((P.Q4_K, P.Q6_K)):
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, 512)
        model[p + "ffn_norm"] = norm_raw(rng, 512)
        model[p + "q"] = q(512, 512, P.Q8_0)
        model[p + "k"] = q(128, 512, P.Q8_0)
        model[p + "v"] = q(128, 512, P.Q8_0)
        model[p + "o"] = q(512, 512, P.Q8_0)
        model[p + "gate"] = q(1024, 512, P.Q8_0)
        model[p + "up"] = q(1024, 512, P.Q8_0)
        model[p + "down"] = q(1024, 512, ddt)
    for M in (1, 5, 8):
        toks = rng.integers(0, 500, M).tolist()
        got, want, _, _ = run_both(gctx, orc, model, toks, 40, 64)
        assert rel_err_rows(got, want) < LOGIT_TOL, M


CFG1 = P.model_cfg(2, 512, 8, 8, 64, 1408, 32000, rope_theta=10000.0)
CFG1_DT = dict(tok_embd=P.F32, output=P.Q4_0, q=P.Q4_0, k=P.Q4_0, v=P.Q4_0, o=P.Q4_0,
               gate=P.Q4_0, up=P.Q4_0, down=P.Q4_0)


def test_verify_tiny_llama_shape(gctx, orc):
    """The tiny-Llama workload's layer shape (d 512, 8 heads x 64, FFN 1408,
    V 32000, Q4_0 in the reference nibble order, F32 embedding), 2 layers,
    K=4 draft after a 128-token context."""
    orc.set_threads(8)
    model = P.make_model(orc, CFG1, CFG1_DT, seed=1)
    rng = np.random.default_rng(3)
    toks = rng.integers(0, 32000, 4).tolist()
    got, want, _, _ = run_both(gctx, orc, model, toks, 128, 160)
    assert rel_err_rows(got, want) < LOGIT_TOL


def q4k_m_dtypes(layer, n_layer):
    """Q4_K_M mix: Q6_K for attn_v and ffn_down on the 'more bits' layers."""
    more = layer < n_layer // 8 or layer >= 7 * n_layer // 8 or (layer - n_layer // 8) % 3 == 2
    dv = P.Q6_K if more else P.Q4_K
    return dict(q=P.Q4_K, k=P.Q4_K, v=dv, o=P.Q4_K, gate=P.Q4_K, up=P.Q4_K, down=dv)


@pytest.mark.parametrize("npast", [64, 2040])
def test_verify_8b_shape_two_layers(gctx, orc, npast):
    """8B layer shape (d 4096, 32/8 heads x 128, FFN 14336, V 128256), Q4_K
    with Q6_K attn_v / ffn_down on one layer and a Q6_K head, 2 layers, an
    8-token chain at context 64 and at the headline workload's context 2048
    (17 attention chunks through the Q4_K o-projection's fused combine),
    theta 500000."""
    orc.set_threads(16)
    cfg = P.model_cfg(2, 4096, 32, 8, 128, 14336, 128256, rope_theta=500000.0)
    model = {"cfg": dict(cfg)}
    rng = np.random.default_rng(21)

    def q(rows, cols, dt):
        # 2048 random rows repeated with moved scales (host quantisation stays short)
        return q_rows(orc, rng, rows, cols, dt)

    model["tok_embd"] = q(128256, 4096, P.Q4_K)
    model["output"] = q(128256, 4096, P.Q6_K)
    model["out_norm"] = norm_raw(rng, 4096)
    for l in range(2):
        dts = q4k_m_dtypes(l if l == 0 else 5, 32)
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, 4096)
        model[p + "ffn_norm"] = norm_raw(rng, 4096)
        model[p + "q"] = q(4096, 4096, dts["q"])
        model[p + "k"] = q(1024, 4096, dts["k"])
        model[p + "v"] = q(1024, 4096, dts["v"])
        model[p + "o"] = q(4096, 4096, dts["o"])
        model[p + "gate"] = q(14336, 4096, dts["gate"])
        model[p + "up"] = q(14336, 4096, dts["up"])
        model[p + "down"] = q(14336, 4096, dts["down"])
    toks = rng.integers(0, 128256, 8).tolist()
    got, want, _, _ = run_both(gctx, orc, model, toks, npast, max(96, npast + 8))
    assert rel_err_rows(got, want) < LOGIT_TOL


@pytest.mark.parametrize("parents", [None, [-1, 0, 1, 1, 2, 3, 3, 4, -1, 8, 9, 9]])
def test_verify_generic_mfma_dtypes(gctx, orc, parents):
    """More than 8 tokens on non-K-quant weights: the fp16 hi/lo MFMA kernel
    over every block dtype (F16 q, BF16 k, Q4_1 v, F32 o, Q8_0 gate / up,
    Q4_0 down, Q4_1 head; d 512, 8 x 64 heads), a 12-token chain and tree at
    context 40, logits within 1e-3 relative of the oracle's."""
    cfg = P.model_cfg(2, 512, 8, 4, 64, 1024, 1000, rope_theta=10000.0)
    dts = dict(tok_embd=P.F32, output=P.Q4_1, q=P.F16, k=P.BF16, v=P.Q4_1, o=P.F32,
               gate=P.Q8_0, up=P.Q8_0, down=P.Q4_0)
    model = P.make_model(orc, cfg, dts, seed=12)
    toks = np.random.default_rng(12).integers(0, 1000, 12).tolist()
    got, want, (kg, vg), (kc, vc) = run_both(gctx, orc, model, toks, 40, 64, parents=parents)
    assert rel_err_rows(got, want) < LOGIT_TOL
    assert np.abs(kg.astype(np.float32) - kc.astype(np.float32)).max() < 2e-2


def tree_parents(branching):
    """Parents of a full draft tree in breadth-first order."""
    parents, level = [], [-1]
    for b in branching:
        nxt = []
        for par in level:
            for _ in range(b):
                parents.append(par)
                nxt.append(len(parents) - 1)
        level = nxt
    return parents


@pytest.mark.parametrize("nodes", [52, 32])
def test_verify_8b_tree52_q8_attention(gctx, orc, nodes):
    """The tree workload's shape: 8B layers (d 4096, 32/8 heads x 128, FFN
    14336) with Q8_0 attention projections and a Q4_K FFN, 2 layers, a
    52-node draft tree (branching 4, 4, 2) -- and the same tree pruned to
    its first 32 nodes in breadth-first order -- at context 4096, then
    residual acceptance of the device's logits against the oracle's on the
    same rows, over the full Llama-3 vocabulary (128256) with a Q6_K head."""
    orc.set_threads(16)
    V = 128256
    cfg = P.model_cfg(2, 4096, 32, 8, 128, 14336, V, rope_theta=500000.0)
    model = {"cfg": dict(cfg)}
    rng = np.random.default_rng(52)

    def q(rows, cols, dt):
        return q_rows(orc, rng, rows, cols, dt)

    model["tok_embd"] = q(V, 4096, P.Q4_K)
    model["output"] = q(V, 4096, P.Q6_K)
    model["out_norm"] = norm_raw(rng, 4096)
    for l in range(2):
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, 4096)
        model[p + "ffn_norm"] = norm_raw(rng, 4096)
        for nm, rows, cols in (("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096),
                               ("o", 4096, 4096)):
            model[p + nm] = q(rows, cols, P.Q8_0)
        for nm in ("gate", "up", "down"):
            model[p + nm] = q(14336, 4096, P.Q4_K)
    parents = tree_parents((4, 4, 2))[:nodes]
    assert len(parents) == nodes and all(p < i for i, p in enumerate(parents))
    toks = rng.integers(0, V, nodes).tolist()
    got, want, _, _ = run_both(gctx, orc, model, toks, 4096, 4096 + 64, parents=parents)
    assert rel_err_rows(got, want) < LOGIT_TOL
    base = (rng.standard_normal(V) * 2).astype(np.float32)
    qd = rng.dirichlet(np.ones(V), size=nodes).astype(np.float32)
    props = np.array(toks, np.int32)
    g, o = accept_both(gctx, orc, base, got, props, ftx.ACCEPT_RESIDUAL, 0.8, 77,
                       parents=parents, q=qd)
    assert (g["accepted"], g["bonus"], g["rng"]) == (o["accepted"], o["bonus"], o["rng"])


@pytest.mark.parametrize("d,ff,hd", [(2048, 8192, 64), (3072, 8192, 128), (512, 1024, 64)])
def test_verify_narrow_widths(gctx, orc, d, ff, hd):
    """Widths below 4096 on the MFMA row-dot path (Llama-3.2-1B: d 2048, head
    64; 3B: d 3072, head 128; a 2-super-block 512), Q4_K with Q6_K attn_v /
    ffn_down, 2 layers: an 8-token chain and a tree at context 70."""
    orc.set_threads(16)
    nh = d // hd
    cfg = P.model_cfg(2, d, nh, max(nh // 4, 1), hd, ff, 3000, rope_theta=500000.0)
    dts_l = [q4k_m_dtypes(0, 32), q4k_m_dtypes(5, 32)]
    model = P.make_model(orc, cfg, dict(dts_l[0], tok_embd=P.Q4_K, output=P.Q6_K), seed=d)
    for name in ("v", "down"):  # the second layer's mix
        w = (np.random.default_rng(d + 1).standard_normal(
            (model["blk.1." + name]["ne1"], model["blk.1." + name]["ne0"])) * 0.02).astype(np.float32)
        model["blk.1." + name] = dict(raw=orc.quantize(w, dts_l[1][name]), dtype=dts_l[1][name],
                                      ne0=model["blk.1." + name]["ne0"],
                                      ne1=model["blk.1." + name]["ne1"])
    rng = np.random.default_rng(d + 2)
    toks = rng.integers(0, 3000, 8).tolist()
    for parents in (None, [-1, 0, 0, 1, 2, 2, 4, -1]):
        got, want, _, _ = run_both(gctx, orc, model, toks, 70, 96, parents=parents)
        assert rel_err_rows(got, want) < LOGIT_TOL, parents


def _wide_model(orc, neox, seed):
    """one 8B-width layer (d 4096, 32/8 heads x 128) with Q4_K projections and a
    Q6_K attn_v: the int8-MFMA projections and the MFMA attention both apply"""
    cfg = P.model_cfg(1, 4096, 32, 8, 128, 4096, 1000, rope_theta=500000.0, rope_neox=neox)
    model = {"cfg": dict(cfg)}
    rng = np.random.default_rng(seed)

    def q(rows, cols, dt):
        return q_rows(orc, rng, rows, cols, dt, unique=1024)

    model["tok_embd"] = q(1000, 4096, P.Q4_K)
    model["output"] = q(1000, 4096, P.Q6_K)
    model["out_norm"] = norm_raw(rng, 4096)
    model["blk.0.attn_norm"] = norm_raw(rng, 4096)
    model["blk.0.ffn_norm"] = norm_raw(rng, 4096)
    for nm, rows, dt in (("q", 4096, P.Q4_K), ("k", 1024, P.Q4_K), ("v", 1024, P.Q6_K),
                         ("o", 4096, P.Q4_K), ("gate", 4096, P.Q4_K), ("up", 4096, P.Q4_K),
                         ("down", 4096, P.Q4_K)):
        model["blk.0." + nm] = q(rows, 4096, dt)
    return model


@pytest.mark.parametrize("neox", [0, 1])
@pytest.mark.parametrize("parents", [None, [-1, 0, 0, 1, 2, 2, 3]])
def test_verify_fused_rope_kv(gctx, orc, neox, parents):
    """Interleaved RoPE and the KV-cache write run in the q/k/v projection's
    epilogue (neox pairs take the separate RoPE kernel): logits, the written
    K/V rows and the untouched rest of the cache agree with the oracle, for
    a chain and a tree at a context that is not chunk aligned."""
    orc.set_threads(16)
    model = _wide_model(orc, neox, seed=31 + neox)
    M = 6 if parents is None else len(parents)
    toks = list(np.random.default_rng(7).integers(0, 1000, M))
    npast = 93
    got, want, (kg, vg), (kc, vc) = run_both(gctx, orc, model, toks, npast, npast + M + 3,
                                             parents=parents)
    assert rel_err_rows(got, want) < LOGIT_TOL
    # the draft rows written to the cache agree to fp16 rounding
    np.testing.assert_allclose(kg.astype(np.float32), kc.astype(np.float32), rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(vg.astype(np.float32), vc.astype(np.float32), rtol=2e-3, atol=2e-3)
    assert np.array_equal(kg[:, :npast], kc[:, :npast]) and np.array_equal(vg[:, :npast], vc[:, :npast])


@pytest.mark.parametrize("parents", [None, [-1, 0, 0, 1, 1, 2, 2, 3]])
def test_verify_long_context_8192(gctx, orc, parents):
    """Context 8180 (64 whole attention chunks and a partial one: more than
    the combine's 32-chunk prefetch batch and its 64-chunk loops) on one
    8B-width layer whose Q4_K o-projection takes the fused combine, an
    8-token chain and a tree."""
    orc.set_threads(16)
    model = _wide_model(orc, 0, seed=81)
    toks = list(np.random.default_rng(82).integers(0, 1000, 8))
    npast = 8180
    got, want, _, _ = run_both(gctx, orc, model, toks, npast, npast + 12, parents=parents)
    assert rel_err_rows(got, want) < LOGIT_TOL


def test_kv_of_another_model_rejected(gctx, orc):
    """A cache made for one model is refused by a model of the same layer
    count and K width but more query heads or a larger step (its attention
    partials were sized for the creating model)."""
    a = P.model_cfg(1, 256, 4, 2, 64, 256, 100)
    b = P.model_cfg(1, 512, 8, 2, 64, 256, 100)
    ma, mb = P.make_model(orc, a, TINY_DT, seed=1), P.make_model(orc, b, TINY_DT, seed=2)
    ta, tb = upload_model(gctx, ma), upload_model(gctx, mb)
    ga = gctx.model(a, ta, max_tokens=8)
    gb = gctx.model(b, tb, max_tokens=8)
    gc = gctx.model(a, ta, max_tokens=16)
    kv = ga.kv(64)
    buf = gctx.buffer(16 * 100 * 4)
    for gm, M in ((gb, 4), (gc, 12)):
        with pytest.raises(ftx.FtxError) as e:
            gm.verify(kv, list(range(M)), buf.ptr)
        assert e.value.code == -1  # FTX_E_INVALID
    ga.verify(kv, [1, 2, 3], buf.ptr)  # the creating model still runs
    gctx.sync()
    for o in (buf, kv, ga, gb, gc):
        o.free()
    free_all(ta)
    free_all(tb)



@pytest.mark.parametrize("cfg_name,kv_dtype", [("tiny", ftx.KV_F16), ("tiny", ftx.KV_F32),
                                               ("hd128", ftx.KV_F16)])
def test_kv_commit_tree_path(gctx, orc, cfg_name, kv_dtype):
    """Tree verify, commit the accepted path, verify the next token: the
    committed rows are the path nodes' rows moved bit for bit, the rest of
    the cache is untouched, and the next step's logits match the oracle's
    chain forward of the path plus the next token."""
    if cfg_name == "tiny":
        model = P.make_model(orc, TINY, TINY_DT, seed=12)
    else:
        model = P.make_model(orc, HD128, HD128_DT, seed=12)
    cfg = model["cfg"]
    npast, cap = 70, 160
    parents = [-1, -1, 0, 0, 3, 1, 4, 2]
    toks = [5, 6, 7, 8, 9, 10, 11, 12]
    path = [0, 3, 4, 6]
    nxt = 13
    tensors = upload_model(gctx, model)
    gm = gctx.model(cfg, tensors, max_tokens=8)
    kv = gm.kv(cap, kv_dtype)
    k0, v0 = kv_context(cfg, cap, npast, 21)
    kv.write(k0, v0)
    kv.truncate(npast)
    V = cfg["vocab"]
    buf = gctx.buffer(8 * V * 4)
    gm.verify(kv, toks, buf.ptr, parents=parents)
    gctx.sync()
    kt, vt = kv.read()
    kv.commit(path)
    gctx.sync()
    assert kv.pointers()[2] == npast + len(path)
    kc, vc = kv.read()
    slots = [npast + j for j in path]
    assert np.array_equal(kc[:, npast:npast + len(path)], kt[:, slots])
    assert np.array_equal(vc[:, npast:npast + len(path)], vt[:, slots])
    assert np.array_equal(kc[:, :npast], kt[:, :npast]) and np.array_equal(vc[:, :npast], vt[:, :npast])
    gm.verify(kv, [nxt], buf.ptr)
    gctx.sync()
    got = buf.read(np.float32, V)
    dt = np.float16 if kv_dtype == ftx.KV_F16 else np.float32
    ko, vo = k0.astype(dt), v0.astype(dt)
    want = orc.forward(model, ko, vo, npast, [toks[j] for j in path] + [nxt])
    assert rel_err_rows(got, want[-1]) < LOGIT_TOL
    # a chain commit moves nothing and only advances the committed length
    kv.truncate(npast)
    gm.verify(kv, toks[:3], buf.ptr)
    gctx.sync()
    kt, vt = kv.read()
    kv.commit([0, 1, 2])
    gctx.sync()
    kc, vc = kv.read()
    assert kv.pointers()[2] == npast + 3
    assert np.array_equal(kc, kt) and np.array_equal(vc, vt)
    buf.free()
    kv.free()
    gm.free()
    free_all(tensors)


def test_kv_commit_errors(gctx, orc):
    model = P.make_model(orc, TINY, TINY_DT, seed=3)
    tensors = upload_model(gctx, model)
    gm = gctx.model(TINY, tensors, max_tokens=8)
    kv = gm.kv(16)
    kv.truncate(10)
    for bad, code in (([1, 1], -1), ([2, 1], -1), ([0, 0], -1), ([1], None),
                      ([0, 6], -5), (list(range(7)), -5)):
        if code is None:
            kv.commit(bad)  # node 1 at slot 11 < 16 is in range
            assert kv.pointers()[2] == 11
            kv.truncate(10)
            continue
        with pytest.raises(ftx.FtxError) as e:
            kv.commit(bad)
        assert e.value.code == code, bad
        assert kv.pointers()[2] == 10
    kv.free()
    gm.free()
    free_all(tensors)


def test_verify_errors(gctx, orc):
    model = P.make_model(orc, TINY, TINY_DT, seed=3)
    tensors = upload_model(gctx, model)
    gm = gctx.model(TINY, tensors, max_tokens=8)
    kv = gm.kv(16)
    buf = gctx.buffer(8 * 50 * 4)
    with pytest.raises(ftx.FtxError) as e:
        gm.verify(kv, [1, 50], buf.ptr)
    assert e.value.code == -5
    with pytest.raises(ftx.FtxError) as e:
        gm.verify(kv, [1, 2], buf.ptr, parents=[-1, 1])
    assert e.value.code == -1
    kv.truncate(12)
    with pytest.raises(ftx.FtxError) as e:
        gm.verify(kv, [1, 2, 3, 4, 5], buf.ptr)
    assert e.value.code == -5
    buf.free()
    kv.free()
    gm.free()
    free_all(tensors)


# ---------------------------------------------------------------- acceptance

def accept_both(gctx, orc, base, rows, props, mode, temp, seed, parents=None, pd=None, q=None,
                sampler_state=ftx.SAMPLER_SEED, top_k=40, top_p=0.95):
    M, V = rows.shape
    b = gctx.buffer((M + 1) * V * 4)
    b.write(np.ascontiguousarray(base, np.float32))
    b.write(np.ascontiguousarray(rows, np.float32), V * 4)
    qb = None
    if q is not None:
        qb = gctx.buffer(M * V * 4)
        qb.write(np.ascontiguousarray(q, np.float32))
    g = gctx.accept(b.ptr, b.ptr + V * 4, M, V, props, mode, temp=temp, rng=seed,
                    parents=parents, pd=pd, q_ptr=qb.ptr if qb else None,
                    sampler_state=sampler_state, top_k=top_k, top_p=top_p)
    b.free()
    if qb:
        qb.free()
    o = orc.verify_accept(base, rows, props, mode, temp=temp, seed=seed, parents=parents, pd=pd,
                          q=q, sampler_state=sampler_state, top_k=top_k, top_p=top_p)
    return g, o


def case(rng, k, V, spread=2.0, hit=0.7):
    base = (rng.standard_normal(V) * spread).astype(np.float32)
    rows = (rng.standard_normal((k, V)) * spread).astype(np.float32)
    props = rng.integers(0, V, k).astype(np.int32)
    for a in range(k):
        if rng.random() < hit:
            props[a] = int(np.argmax(base if a == 0 else rows[a - 1]))
    return base, rows, props


def test_accept_reference_kat(gctx, orc):
    """src/tests/test_core.cpp:348-356: props {0,1,2} -> 3, {0,3,2} -> 1."""
    base = np.array([9, 1, 1, 1], np.float32)
    rows = np.array([[1, 9, 1, 1], [1, 1, 9, 1], [1, 1, 1, 9]], np.float32)
    for props, n in (([0, 1, 2], 3), ([0, 3, 2], 1)):
        g, o = accept_both(gctx, orc, base, rows, props, ftx.ACCEPT_GREEDY, 1.0, 0)
        assert len(g["accepted"]) == n == len(o["accepted"])
        assert g == o or (g["accepted"], g["bonus"]) == (o["accepted"], o["bonus"])


@pytest.mark.parametrize("V", [64, 32000])
def test_accept_greedy_chain_and_tree(gctx, orc, V):
    rng = np.random.default_rng(V)
    for trial in range(20):
        base, rows, props = case(rng, 8, V)
        g, o = accept_both(gctx, orc, base, rows, props, ftx.ACCEPT_GREEDY, 1.0, 0)
        assert (g["accepted"], g["bonus"]) == (o["accepted"], o["bonus"])
        parents = [-1, -1, 0, 0, 1, 2, 2, 4]
        g, o = accept_both(gctx, orc, base, rows, props, ftx.ACCEPT_GREEDY, 1.0, 0,
                           parents=parents)
        assert (g["accepted"], g["bonus"]) == (o["accepted"], o["bonus"])


# 1001: rows not 16-byte aligned, a partial last sub-chunk; 262147: several
# sub-chunks per scanning thread in the bonus pick
@pytest.mark.parametrize("V,temp", [(64, 1.0), (1001, 0.7), (32000, 0.8), (128256, 0.8),
                                    (262147, 1.3)])
def test_accept_ratio_chain(gctx, orc, V, temp):
    rng = np.random.default_rng(V + 1)
    for trial in range(12 if V > 1000 else 60):
        base, rows, props = case(rng, 8, V, spread=1.0)
        pd = (rng.random(8) * 0.05).astype(np.float32)
        pd[rng.random(8) < 0.1] = 0.0
        seed = int(rng.integers(1, 2**63))
        g, o = accept_both(gctx, orc, base, rows, props, ftx.ACCEPT_RATIO, temp, seed, pd=pd)
        assert (g["accepted"], g["bonus"], g["rng"], g["sampler_state"]) == \
            (o["accepted"], o["bonus"], o["rng"], o["sampler_state"])


@pytest.mark.parametrize("V", [24, 32000])
def test_accept_residual_chain_and_tree(gctx, orc, V):
    rng = np.random.default_rng(V + 2)
    for trial in range(10 if V > 1000 else 50):
        parents = [-1, -1, -1, 0, 0, 1, 3, 3] if trial % 2 else list(range(-1, 7))
        base, rows, props = case(rng, 8, V, spread=1.0, hit=0.5)
        q = rng.dirichlet(np.ones(V), size=8).astype(np.float32)
        for c in range(8):
            if rng.random() < 0.5:
                props[c] = int(np.argmax(q[c]))
        seed = int(rng.integers(1, 2**63))
        g, o = accept_both(gctx, orc, base, rows, props, ftx.ACCEPT_RESIDUAL, 0.8, seed,
                           parents=parents, q=q)
        assert (g["accepted"], g["bonus"], g["rng"], g["sampler_state"]) == \
            (o["accepted"], o["bonus"], o["rng"], o["sampler_state"])


def test_accept_residual_wide_tree(gctx, orc):
    """130-node trees (more than 64 children scanned per node, children of
    one node spread over several 64-node groups) with draft tokens drawn near
    the target, so that walks go several levels deep."""
    rng = np.random.default_rng(77)
    V, M = 3000, 130
    for trial in range(6):
        parents = [-1] + [int(rng.integers(-1, i)) if trial % 2 else int(rng.integers(max(-1, i - 70), i))
                          for i in range(1, M)]
        base, rows, props = case(rng, M, V, spread=1.0, hit=0.7)
        q = rng.dirichlet(np.ones(V) * 0.3, size=M).astype(np.float32)
        seed = int(rng.integers(1, 2**63))
        g, o = accept_both(gctx, orc, base, rows, props, ftx.ACCEPT_RESIDUAL, 0.8, seed,
                           parents=parents, q=q)
        assert (g["accepted"], g["bonus"], g["rng"]) == (o["accepted"], o["bonus"], o["rng"])


@pytest.mark.parametrize("V", [1001, 32000])
def test_accept_batch_matches_single(gctx, orc, V):
    """ftx_accept_batch over six sequences -- ratio chains of 8 and 3 nodes
    (their own acceptance and sampler streams), a greedy tree, a residual
    chain and tree, an empty draft -- returns for each what ftx_accept
    returns for it alone, and what the oracle's acceptance gives."""
    rng = np.random.default_rng(V + 9)
    bufs, items, want = [], [], []
    for kind, M in (("ratio", 8), ("ratio", 3), ("greedy", 8), ("residual", 8), ("residual", 6),
                    ("empty", 0)):
        base, rows, props = case(rng, max(M, 1), V, spread=1.0)
        rows, props = rows[:M], props[:M]
        b = gctx.buffer((M + 1) * V * 4)
        b.write(np.ascontiguousarray(base, np.float32))
        if M:
            b.write(np.ascontiguousarray(rows, np.float32), V * 4)
        it = dict(base_ptr=b.ptr, rows_ptr=b.ptr + V * 4 if M else None, M=M, V=V, props=props,
                  temp=0.8, rng=int(rng.integers(1, 2**63)),
                  sampler_state=int(rng.integers(1, 2**63)))
        o_kw = dict(temp=0.8, seed=it["rng"], sampler_state=it["sampler_state"])
        if kind == "ratio":
            it["mode"] = ftx.ACCEPT_RATIO
            it["pd"] = (rng.random(M) * 0.05).astype(np.float32)
            o_kw["pd"] = it["pd"]
        elif kind == "residual":
            it["mode"] = ftx.ACCEPT_RESIDUAL
            q = rng.dirichlet(np.ones(V), size=M).astype(np.float32)
            qb = gctx.buffer(M * V * 4)
            qb.write(q)
            bufs.append(qb)
            it["q_ptr"] = qb.ptr
            it["parents"] = [-1, -1, 0, 0, 1, 3, 3, 5][:M] if M == 6 else None
            o_kw.update(q=q, parents=it["parents"])
        else:
            it["mode"] = ftx.ACCEPT_GREEDY
            it["parents"] = [-1, -1, 0, 0, 1, 2, 2, 4] if M == 8 else None
            o_kw["parents"] = it["parents"]
        bufs.append(b)
        items.append(it)
        if M:
            want.append(orc.verify_accept(base, rows, props, it["mode"], **o_kw))
        else:
            want.append(None)
    got = gctx.accept_batch(items)
    for it, g, o in zip(items, got, want):
        kw = {k: it[k] for k in ("temp", "rng", "parents", "pd", "q_ptr", "sampler_state")
              if k in it}
        one = gctx.accept(it["base_ptr"], it["rows_ptr"], it["M"], V, it["props"], it["mode"],
                          **kw)
        assert g == one
        if o is not None:
            assert (g["accepted"], g["bonus"], g["rng"]) == (o["accepted"], o["bonus"], o["rng"])
            if it["mode"] == ftx.ACCEPT_RATIO:
                assert g["sampler_state"] == o["sampler_state"]
    for b in bufs:
        b.free()


def test_accept_empty_draft(gctx, orc):
    """M = 0: only the bonus token is drawn."""
    rng = np.random.default_rng(4)
    base = rng.standard_normal(1000).astype(np.float32)
    b = gctx.buffer(1000 * 4)
    b.write(base)
    g = gctx.accept(b.ptr, None, 0, 1000, [], ftx.ACCEPT_GREEDY)
    b.free()
    assert g["accepted"] == [] and g["bonus"] == int(np.argmax(base))


# vocab sizes: 33 (no top-k: k >= V), 64, 1001 (a partial last sub-chunk),
# 128256 (the 8B vocab), 262147 (more than 2048 sub-chunks)
@pytest.mark.parametrize("V", [33, 64, 1001, 128256, 262147])
def test_bonus_sampler(gctx, orc, V):
    """The ratio-mode bonus is Sampler::sample (include/ft/sampler.h:30-94):
    an empty draft draws it from the base row alone; token and sampler state
    equal the oracle's over temperatures, top-k and top-p, the state carried
    from draw to draw.  Rows with near-equal top logits (ties at the top-k
    boundary after rounding) are part of the mix."""
    rng = np.random.default_rng(V + 7)
    state = ftx.SAMPLER_SEED
    b = gctx.buffer(V * 4)
    for trial in range(16 if V > 100000 else 40):
        spread = float(rng.choice([0.5, 2.0, 8.0]))
        base = (rng.standard_normal(V) * spread).astype(np.float32)
        if trial % 5 == 4:
            base[rng.integers(0, V, 6)] = base.max()  # equal maxima
        temp = float(rng.choice([0.3, 0.7, 1.0, 1.6]))
        top_k = int(rng.choice([1, 5, 40, 64])) if V > 64 else int(rng.choice([V, V + 5, 0]))
        top_p = float(rng.choice([0.5, 0.9, 0.95, 1.0]))
        b.write(base)
        g = gctx.accept(b.ptr, None, 0, V, [], ftx.ACCEPT_RATIO, temp=temp, rng=3,
                        sampler_state=state, top_k=top_k, top_p=top_p)
        o = orc.verify_accept(base, base[None, :0].reshape(0, V), np.zeros(0, np.int32),
                              P.ACCEPT_RATIO, temp=temp, seed=3, pd=np.zeros(0, np.float32),
                              sampler_state=state, top_k=top_k, top_p=top_p)
        assert (g["bonus"], g["sampler_state"]) == (o["bonus"], o["sampler_state"]), \
            (trial, temp, top_k, top_p)
        assert g["rng"] == 3 and g["accepted"] == []
        state = g["sampler_state"]
    b.free()


def test_bonus_sampler_limits(gctx):
    V = 1000
    b = gctx.buffer(V * 4)
    b.write(np.zeros(V, np.float32))
    for top_k in (65, 0):  # top-k beyond 64, or none over more than 64 tokens
        with pytest.raises(ftx.FtxError) as e:
            gctx.accept(b.ptr, None, 0, V, [], ftx.ACCEPT_RATIO, temp=0.7, top_k=top_k)
        assert e.value.code == -2
    b.free()
