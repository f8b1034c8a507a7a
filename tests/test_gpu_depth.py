"""Full-depth parity of the headline verify step and a regression test of the
trace timer on an error path, on the GPU through the C ABI.

test_verify_8b_full_depth: the Llama-3-8B shape (d 4096, 32 / 8 heads x 128,
FFN 14336, V 128256) at its full 32 layers with the Q4_K_M mix (Q6_K attn_v
and ffn_down on the 'more bits' layers, a Q6_K head), an 8-token chain at
context 2040: the logits within 1e-3 relative of the oracle's forward
(src/engine.cpp:461-596, Engine::forward).  The layers draw their large
tensors from a pool of four (two per mix), each with its own norm weights,
so that a layer index error changes the result; the error of the int8 x 2-limb
activations accumulates over all 32 layers here.

test_tree52_full_depth: the same shape at 32 layers with Q8_0 attention
projections and a Q4_K FFN, the 52-node draft tree (branching 4, 4, 2) at
context 4096: every projection on the one-pass GEMMs (fp16 hi + lo
activations), attention on the many-row tree kernel, all 32 layers' error.

test_mixtral_full_depth: the Mixtral 8x7B shape (8 experts of FFN 14336,
top-2, Q4_0, vocab 32000) at its full 32 layers, four sequences of 8 tokens
at context 1024 in one batched step: the routing, the expert GEMMs and the
combine of every layer, against the oracle's forward of each sequence
(src/engine.cpp:179-258, moe_ffn).
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


def more_bits(layer, n_layer):
    return layer < n_layer // 8 or layer >= 7 * n_layer // 8 or (layer - n_layer // 8) % 3 == 2


def test_verify_8b_full_depth(gctx, orc):
    orc.set_threads(16)
    L, D, F, V = 32, 4096, 14336, 128256
    cfg = P.model_cfg(L, D, 32, 8, 128, F, V, rope_theta=500000.0)
    rng = np.random.default_rng(77)

    def q(rows, cols, dt):
        return q_rows(orc, rng, rows, cols, dt)

    pool = []
    for i in range(4):
        dv = P.Q6_K if i < 2 else P.Q4_K
        pool.append(dict(q=q(4096, D, P.Q4_K), k=q(1024, D, P.Q4_K), v=q(1024, D, dv),
                         o=q(4096, D, P.Q4_K), gate=q(F, D, P.Q4_K), up=q(F, D, P.Q4_K),
                         down=q(F, D, dv)))
    model = {"cfg": dict(cfg)}
    model["tok_embd"] = q(V, D, P.Q4_K)
    model["output"] = q(V, D, P.Q6_K)
    model["out_norm"] = norm_raw(rng, D)
    for l in range(L):
        src = pool[(l % 2) if more_bits(l, L) else 2 + (l % 2)]
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, D)
        model[p + "ffn_norm"] = norm_raw(rng, D)
        for nm, t in src.items():
            model[p + nm] = t
    up, tensors = _upload_dedup(gctx, model)
    npast, M = 2040, 8
    cap = npast + M
    gm = gctx.model(cfg, tensors, max_tokens=M)
    kv = gm.kv(cap)
    krng = np.random.default_rng(5)
    shape = kv.shape
    k0 = np.zeros(shape, np.float16)
    v0 = np.zeros(shape, np.float16)
    k0[:, :npast] = krng.standard_normal((L, npast, shape[2]))
    v0[:, :npast] = krng.standard_normal((L, npast, shape[2]))
    kv.write(k0, v0)
    kv.truncate(npast)
    toks = rng.integers(0, V, M).tolist()
    buf = gctx.buffer(M * V * 4)
    gm.verify(kv, toks, buf.ptr)
    gctx.sync()
    got = buf.read(np.float32, M * V).reshape(M, V)
    buf.free()
    kv.free()
    gm.free()
    for t in up.values():
        t.free()
    want = orc.forward(model, k0, v0, npast, toks)
    err = rel_err_rows(got, want)
    print("32-layer 8B chain at context 2040: max row error %.3g" % err)
    assert err < LOGIT_TOL


def _upload_dedup(gctx, model):
    """One device tensor per distinct host tensor (expert tensors as
    (cols, rows per expert, experts))."""
    E = model["cfg"].get("n_expert", 0)
    up, tensors = {}, {}
    for name, t in model.items():
        if name == "cfg":
            continue
        if id(t) not in up:
            ne = (t["ne0"], t["ne1"])
            if name.endswith("_exps"):
                ne = (t["ne0"], t["ne1"] // E, E)
            up[id(t)] = gctx.upload(t["raw"], t["dtype"], ne)
        tensors[name] = up[id(t)]
    return up, tensors


def _tree_parents(branching):
    parents, level = [], [-1]
    for b in branching:
        nxt = []
        for par in level:
            for _ in range(b):
                parents.append(par)
                nxt.append(len(parents) - 1)
        level = nxt
    return parents


def test_tree52_full_depth(gctx, orc):
    orc.set_threads(16)
    L, D, F, V = 32, 4096, 14336, 128256
    cfg = P.model_cfg(L, D, 32, 8, 128, F, V, rope_theta=500000.0)
    rng = np.random.default_rng(5252)

    def q(rows, cols, dt):
        return q_rows(orc, rng, rows, cols, dt)

    pool = [dict(q=q(4096, D, P.Q8_0), k=q(1024, D, P.Q8_0), v=q(1024, D, P.Q8_0),
                 o=q(4096, D, P.Q8_0), gate=q(F, D, P.Q4_K), up=q(F, D, P.Q4_K),
                 down=q(F, D, P.Q4_K)) for _ in range(4)]
    model = {"cfg": dict(cfg)}
    model["tok_embd"] = q(V, D, P.Q4_K)
    model["output"] = q(V, D, P.Q6_K)
    model["out_norm"] = norm_raw(rng, D)
    for l in range(L):
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, D)
        model[p + "ffn_norm"] = norm_raw(rng, D)
        for nm, t in pool[(l * 3) % 4].items():
            model[p + nm] = t
    up, tensors = _upload_dedup(gctx, model)
    parents = _tree_parents((4, 4, 2))
    M = len(parents)
    npast, cap = 4096, 4096 + 64
    gm = gctx.model(cfg, tensors, max_tokens=M)
    kv = gm.kv(cap)
    krng = np.random.default_rng(6)
    shape = kv.shape
    k0 = np.zeros(shape, np.float16)
    v0 = np.zeros(shape, np.float16)
    k0[:, :npast] = krng.standard_normal((L, npast, shape[2]))
    v0[:, :npast] = krng.standard_normal((L, npast, shape[2]))
    kv.write(k0, v0)
    kv.truncate(npast)
    toks = rng.integers(0, V, M).tolist()
    buf = gctx.buffer(M * V * 4)
    gm.verify(kv, toks, buf.ptr, parents=parents)
    gctx.sync()
    got = buf.read(np.float32, M * V).reshape(M, V)
    buf.free()
    kv.free()
    gm.free()
    for t in up.values():
        t.free()
    want = orc.forward(model, k0, v0, npast, toks, parents=parents)
    err = rel_err_rows(got, want)
    print("32-layer 8B 52-node tree at context 4096: max row error %.3g" % err)
    assert err < LOGIT_TOL


def test_mixtral_full_depth(gctx, orc):
    orc.set_threads(16)
    L, D, F, V, E = 32, 4096, 14336, 32000, 8
    cfg = P.model_cfg(L, D, 32, 8, 128, F, V, rope_theta=1e6, n_expert=E, n_expert_used=2)
    rng = np.random.default_rng(3232)

    def layer():
        t = {nm: q_rows(orc, rng, rows, D, P.Q4_0)
             for nm, rows in (("q", D), ("k", 1024), ("v", 1024), ("o", D))}
        w = (rng.standard_normal((E, D)) * (2.0 / np.sqrt(D))).astype(np.float32)
        t["gate_inp"] = dict(raw=w.view(np.uint8).ravel().copy(), dtype=P.F32, ne0=D, ne1=E)
        for nm in ("gate_exps", "up_exps", "down_exps"):
            planes = [q_rows(orc, rng, F, D, P.Q4_0, unique=1024)["raw"] for _ in range(E)]
            t[nm] = dict(raw=np.concatenate(planes), dtype=P.Q4_0, ne0=D, ne1=E * F)
        return t

    pool = [layer(), layer()]
    model = {"cfg": dict(cfg)}
    model["tok_embd"] = q_rows(orc, rng, V, D, P.Q8_0, unique=1024)
    model["output"] = q_rows(orc, rng, V, D, P.Q4_0, unique=1024)
    model["out_norm"] = norm_raw(rng, D)
    for l in range(L):
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, D)
        model[p + "ffn_norm"] = norm_raw(rng, D)
        for nm, t in pool[l % 2].items():
            model[p + nm] = t
    up, tensors = _upload_dedup(gctx, model)
    gm = gctx.model(cfg, tensors, max_tokens=32)
    seqs = [(rng.integers(0, V, 8).tolist(), 1024 - 8 - s, 1024) for s in range(4)]
    kvs, bufs, ctxs, args = [], [], [], []
    for i, (toks, npast, cap) in enumerate(seqs):
        kv = gm.kv(cap)
        krng = np.random.default_rng(60 + i)
        shape = kv.shape
        k0 = np.zeros(shape, np.float16)
        v0 = np.zeros(shape, np.float16)
        k0[:, :npast] = krng.standard_normal((L, npast, shape[2]))
        v0[:, :npast] = krng.standard_normal((L, npast, shape[2]))
        kv.write(k0, v0)
        kv.truncate(npast)
        buf = gctx.buffer(len(toks) * V * 4)
        kvs.append(kv)
        bufs.append(buf)
        ctxs.append((k0, v0))
        args.append((kv, toks, buf.ptr, None, False))
    gm.verify_batch(args)
    gctx.sync()
    got = [b.read(np.float32, 8 * V).reshape(8, V) for b in bufs]
    for o in bufs + kvs:
        o.free()
    gm.free()
    for t in up.values():
        t.free()
    errs = []
    for (toks, npast, cap), g, (k0, v0) in zip(seqs, got, ctxs):
        want = orc.forward(model, k0, v0, npast, toks)
        errs.append(rel_err_rows(g, want))
    print("32-layer Mixtral-shaped batch, 4 x 8 tokens at context 1024: max row errors %s"
          % ", ".join("%.3g" % e for e in errs))
    assert max(errs) < LOGIT_TOL


def test_trace_disarmed_after_failed_launch(orc):
    """A traced verify step whose attention launch fails (a cache of more
    than 1024 attention blocks) returns its error; the context is then
    destroyed and a second context's traced and untraced launches run and
    give the oracle's logits: no kernel timer of the first context is left
    armed on the calling thread."""
    cfg = P.model_cfg(2, 256, 4, 2, 64, 512, 300, rope_theta=10000.0)
    dts = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q4_K, k=P.Q4_K, v=P.Q4_K, o=P.Q4_K,
               gate=P.Q4_K, up=P.Q4_K, down=P.Q4_K)
    model = P.make_model(orc, cfg, dts, seed=9)
    toks = [5, 17, 250]

    def build(ctx, cap):
        tensors = {n: ctx.upload(t["raw"], t["dtype"], (t["ne0"], t["ne1"]))
                   for n, t in model.items() if n != "cfg"}
        gm = ctx.model(cfg, tensors, max_tokens=8)
        gm.owned = list(tensors.values())
        return gm, gm.kv(cap)

    a = ftx.Context(0)
    gm, kv = build(a, 64 * 1025)
    kv.truncate(4)
    buf = a.buffer(len(toks) * cfg["vocab"] * 4)
    a.trace(True)
    with pytest.raises(ftx.FtxError):
        gm.verify(kv, toks, buf.ptr)
    a.sync()
    buf.free()
    kv.free()
    gm.free()
    a.close()
    b = ftx.Context(0)
    gm, kv = build(b, 64)
    shape = kv.shape
    k0 = np.zeros(shape, np.float16)
    v0 = np.zeros(shape, np.float16)
    kv.write(k0, v0)
    kv.truncate(4)
    buf = b.buffer(len(toks) * cfg["vocab"] * 4)
    for traced in (False, True):
        kv.truncate(4)
        b.trace(traced)
        gm.verify(kv, toks, buf.ptr)
        b.sync()
        got = buf.read(np.float32, len(toks) * cfg["vocab"]).reshape(len(toks), -1)
        want = orc.forward(model, k0.copy(), v0.copy(), 4, toks)
        assert rel_err_rows(got, want) < LOGIT_TOL
    b.trace(False)
    buf.free()
    kv.free()
    gm.free()
    b.close()
