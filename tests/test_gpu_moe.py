"""GPU parity of the MoE FFN (router, top-k routing, the routed experts'
gate / up / down, the weighted sum, a router bias and a shared expert;
src/engine.cpp:179-258) and of the attention extras (q / k / v bias and the
per-head q / k RMSNorm, src/engine.cpp:519-542) in the verify step, against
the CPU oracle's forward of each sequence alone (the oracle's MoE and extras
are pinned bit-exact against the reference Engine in test_moe_oracle.py).

Logits: per row max|gpu - oracle| / max|oracle| <= 1e-3 (LOGIT_TOL); K / V
rows within 3e-3.
"""
import numpy as np
import pytest

import pyoracle as P
from builders import norm_raw, q_rows

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def rel_err_rows(a, b):
    a = np.atleast_2d(a).astype(np.float64)
    b = np.atleast_2d(b).astype(np.float64)
    return (np.abs(a - b).max(axis=1) / np.maximum(np.abs(b).max(axis=1), 1e-30)).max()


def upload(gctx, model):
    E = model["cfg"].get("n_expert", 0)
    out = {}
    for n, t in model.items():
        if n == "cfg":
            continue
        ne = (t["ne0"], t["ne1"])
        if n.endswith("_exps"):
            ne = (t["ne0"], t["ne1"] // E, E)
        out[n] = gctx.upload(t["raw"], t["dtype"], ne)
    return out


def run(gctx, orc, model, seqs, max_tokens, kv_seed=40):
    """seqs: [(tokens, parents or None, npast, cap)] in one verify_batch
    call; returns per sequence (device logits, oracle logits, device K,
    oracle K)."""
    cfg = model["cfg"]
    V = cfg["vocab"]
    tensors = upload(gctx, model)
    gm = gctx.model(cfg, tensors, max_tokens=max_tokens)
    kvs, bufs, ctxs, args = [], [], [], []
    for i, (toks, parents, npast, cap) in enumerate(seqs):
        kv = gm.kv(cap)
        rng = np.random.default_rng(kv_seed + i)
        shape = (cfg["n_layer"], cap, cfg["n_head_kv"] * cfg["head_dim"])
        k0 = np.zeros(shape, np.float16)
        v0 = np.zeros(shape, np.float16)
        k0[:, :npast] = rng.standard_normal((shape[0], npast, shape[2]))
        v0[:, :npast] = rng.standard_normal((shape[0], npast, shape[2]))
        kv.write(k0, v0)
        kv.truncate(npast)
        buf = gctx.buffer(len(toks) * V * 4)
        kvs.append(kv)
        bufs.append(buf)
        ctxs.append((k0, v0))
        args.append((kv, toks, buf.ptr, parents, False))
    gm.verify_batch(args)
    gctx.sync()
    out = []
    for (toks, parents, npast, cap), kv, buf, (k0, v0) in zip(seqs, kvs, bufs, ctxs):
        got = buf.read(np.float32, len(toks) * V).reshape(len(toks), V)
        kg, _ = kv.read()
        kc, vc = k0.copy(), v0.copy()
        want = orc.forward(model, kc, vc, npast, toks, parents=parents)
        out.append((got, want, kg, kc))
    for o in bufs + kvs:
        o.free()
    gm.free()
    for t in tensors.values():
        t.free()
    return out


def check(res, seqs):
    for (got, want, kg, kc), (toks, par, npast, cap) in zip(res, seqs):
        assert rel_err_rows(got, want) < LOGIT_TOL, (npast, par)
        np.testing.assert_allclose(kg.astype(np.float32), kc.astype(np.float32), rtol=3e-3,
                                   atol=3e-3)


DT = dict(tok_embd=P.Q8_0, output=P.Q8_0, q=P.Q8_0, k=P.Q8_0, v=P.Q8_0, o=P.Q8_0,
          gate=P.Q4_0, up=P.Q4_0, down=P.Q4_0, gate_inp=P.F32, gate_exps=P.Q4_0,
          up_exps=P.Q4_0, down_exps=P.Q4_0, gate_sh=P.Q8_0, up_sh=P.Q8_0, down_sh=P.Q8_0)

MOE = P.model_cfg(2, 256, 4, 2, 64, 256, 500, n_expert=8, n_expert_used=2)


@pytest.mark.parametrize("case", ["q4_0", "q8_0_gate_up", "bias_shared_top3"])
@pytest.mark.parametrize("M", [1, 7, 40, 100, 250])
def test_moe_chain(gctx, orc, case, M):
    """One sequence of M tokens (decode, a short chain, long chains) through
    the MoE layers: Q4_0 experts; Q8_0 gate / up experts; a router bias, a
    shared expert and top-3 of 8.  Above 64 tokens (top-2; 43 for top-3) the
    routing takes 64-row tiles, and up to 250 router workgroups meet at the
    grouping."""
    cfg, dts, extras = dict(MOE), dict(DT), ()
    if case == "q8_0_gate_up":
        dts.update(gate_exps=P.Q8_0, up_exps=P.Q8_0)
    if case == "bias_shared_top3":
        cfg["n_expert_used"] = 3
        extras = ("router_bias", "gate_sh", "up_sh", "down_sh")
    model = P.make_model(orc, cfg, dts, seed=100 + M, extras=extras)
    toks = np.random.default_rng(M).integers(0, 500, M).tolist()
    seqs = [(toks, None, 11, 11 + M + 2)]
    check(run(gctx, orc, model, seqs, max(64, M)), seqs)


def test_moe_three_sequences_and_tree(gctx, orc):
    """Three sequences in one step (a 5-token chain, a 9-node tree, one
    token), each routed and weighted as the oracle's forward of it alone."""
    model = P.make_model(orc, MOE, DT, seed=7)
    rng = np.random.default_rng(8)
    seqs = [(rng.integers(0, 500, 5).tolist(), None, 20, 40),
            (rng.integers(0, 500, 9).tolist(), [-1, 0, 0, 1, 1, 2, -1, 6, 6], 33, 48),
            (rng.integers(0, 500, 1).tolist(), None, 0, 16)]
    check(run(gctx, orc, model, seqs, 16), seqs)


@pytest.mark.parametrize("E,U,M,router", [(64, 6, 40, "f32"), (64, 6, 40, "q8_0_bias"),
                                          (100, 4, 130, "f32_bias"), (256, 8, 33, "f32")])
def test_moe_many_experts(gctx, orc, E, U, M, router):
    """Routers of 64 to 256 experts at top-4 to top-8: the per-token softmax
    on one lane per expert (up to 64) and on four experts per lane (above),
    and the grouping's per-expert prefix sums over several 64-expert rounds
    with 64-entry chunks of (token, rank) entries (264 to 520 entries); a
    router bias on both softmax forms, and a Q8_0 router (the dequantising
    router path)."""
    cfg = dict(MOE)
    cfg["n_expert"] = E
    cfg["n_expert_used"] = U
    dts = dict(DT)
    if router.startswith("q8_0"):
        dts["gate_inp"] = P.Q8_0
    extras = ("router_bias",) if router.endswith("bias") else ()
    model = P.make_model(orc, cfg, dts, seed=300 + E, extras=extras)
    toks = np.random.default_rng(E).integers(0, 500, M).tolist()
    seqs = [(toks, None, 5, 5 + M + 2)]
    check(run(gctx, orc, model, seqs, max(64, M)), seqs)


@pytest.mark.parametrize("extras,neox", [(("q_bias", "k_bias", "v_bias"), 1),
                                         (("q_norm", "k_norm"), 1),
                                         (("q_bias", "k_bias", "v_bias", "q_norm", "k_norm"), 0)])
@pytest.mark.parametrize("M", [1, 6, 20])
def test_attention_extras(gctx, orc, extras, neox, M):
    """q / k / v bias and per-head q / k RMSNorm ahead of RoPE (neox and
    interleaved pairs), on decode, a chain and a 20-node tree."""
    cfg = P.model_cfg(2, 256, 4, 2, 64, 512, 300, rope_neox=neox)
    dts = dict(DT, gate=P.Q8_0, up=P.Q8_0, down=P.Q8_0)
    model = P.make_model(orc, cfg, dts, seed=200 + M, extras=extras)
    rng = np.random.default_rng(M)
    par = None if M < 20 else [-1] + [int(rng.integers(0, i)) for i in range(1, M)]
    seqs = [(rng.integers(0, 300, M).tolist(), par, 17, 17 + M + 1)]
    check(run(gctx, orc, model, seqs, 32), seqs)


def test_moe_mixtral_layer_shape(gctx, orc):
    """The Mixtral 8x7B layer shape (d 4096, 32 / 8 heads x 128, 8 experts
    of FFN 14336, top-2, Q4_0, vocab 32000), 2 layers, four sequences of 8
    tokens at context 1024 in one step."""
    orc.set_threads(16)
    V, d, ff, E = 32000, 4096, 14336, 8
    cfg = P.model_cfg(2, d, 32, 8, 128, ff, V, rope_theta=1e6, n_expert=E, n_expert_used=2)
    rng = np.random.default_rng(901)
    model = {"cfg": dict(cfg)}
    model["tok_embd"] = q_rows(orc, rng, V, d, P.Q8_0, unique=1024)
    model["output"] = q_rows(orc, rng, V, d, P.Q4_0, unique=1024)
    model["out_norm"] = norm_raw(rng, d)
    for l in range(2):
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, d)
        model[p + "ffn_norm"] = norm_raw(rng, d)
        for nm, rows, cols in (("q", d, d), ("k", 1024, d), ("v", 1024, d), ("o", d, d)):
            model[p + nm] = q_rows(orc, rng, rows, cols, P.Q4_0)
        w = (rng.standard_normal((E, d)) * (2.0 / np.sqrt(d))).astype(np.float32)
        model[p + "gate_inp"] = dict(raw=w.view(np.uint8).ravel().copy(), dtype=P.F32, ne0=d,
                                     ne1=E)
        for nm in ("gate_exps", "up_exps", "down_exps"):
            # every expert its own 1024 distinct rows (repeated with moved
            # scales inside the plane)
            planes = [q_rows(orc, rng, ff, d, P.Q4_0, unique=1024)["raw"] for _ in range(E)]
            model[p + nm] = dict(raw=np.concatenate(planes), dtype=P.Q4_0, ne0=d, ne1=E * ff)
    seqs = [(rng.integers(0, V, 8).tolist(), None, 1024 - 8 - s, 1024) for s in range(4)]
    check(run(gctx, orc, model, seqs, 32), seqs)
