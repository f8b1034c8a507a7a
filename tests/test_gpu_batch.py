"""GPU parity of the large-token path of the verify step (more than 8 tokens
in one step, and several sequences with their own caches in one step,
ftx_verify_batch) against the CPU oracle run on each sequence alone.

Logits: per row max|gpu - oracle| / max|oracle| <= 1e-3 (LOGIT_TOL).
Acceptance: on the device's logits, the device and the oracle accept the
same nodes, draw the same bonus token and leave the same rng state.
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


def random_tree(rng, n, max_depth, max_branch):
    """Parents of an n-node draft tree in breadth-first order: each node of a
    level below max_depth gets 1 .. max_branch children until n nodes."""
    parents, level, depth = [], [-1], 0
    while len(parents) < n and depth < max_depth:
        nxt = []
        for par in level:
            for _ in range(int(rng.integers(1, max_branch + 1))):
                if len(parents) == n:
                    break
                parents.append(par)
                nxt.append(len(parents) - 1)
        level, depth = nxt, depth + 1
    assert len(parents) == n, "tree too small for n"
    return parents


def upload(gctx, model):
    return {n: gctx.upload(t["raw"], t["dtype"], (t["ne0"], t["ne1"]))
            for n, t in model.items() if n != "cfg"}


def run_batch(gctx, orc, model, seqs, max_tokens, kv_seed=40):
    """seqs: [(tokens, parents or None, npast, cap)].  Returns per sequence
    (device logits, oracle logits, device K / V, oracle K / V)."""
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
        kg, vg = kv.read()
        kc, vc = k0.copy(), v0.copy()
        want = orc.forward(model, kc, vc, npast, toks, parents=parents)
        out.append((got, want, (kg, vg), (kc, vc)))
    for o in bufs + kvs:
        o.free()
    gm.free()
    for t in tensors.values():
        t.free()
    return out


SMALL = P.model_cfg(2, 512, 8, 4, 64, 1024, 1000, rope_theta=10000.0)


@pytest.mark.parametrize("dts", [
    # Q4_K everywhere (one-pass GEMMs and the column-axpy down) with a Q6_K
    # head (the generic head, once per sequence)
    dict(tok_embd=P.Q4_K, output=P.Q6_K, q=P.Q4_K, k=P.Q4_K, v=P.Q4_K, o=P.Q4_K,
         gate=P.Q4_K, up=P.Q4_K, down=P.Q4_K),
    # Q8_0 attention projections, Q4_K FFN, a Q4_0 head (one pass over the
    # rows of every sequence)
    dict(tok_embd=P.F32, output=P.Q4_0, q=P.Q8_0, k=P.Q8_0, v=P.Q8_0, o=P.Q8_0,
         gate=P.Q4_K, up=P.Q4_K, down=P.Q4_K),
    # Q4_0 everywhere (the generic down kernel)
    dict(tok_embd=P.F32, output=P.Q4_0, q=P.Q4_0, k=P.Q4_0, v=P.Q4_0, o=P.Q4_0,
         gate=P.Q4_0, up=P.Q4_0, down=P.Q4_0),
])
def test_batch_three_sequences(gctx, orc, dts):
    """Three sequences in one step -- a 5-token chain at context 20, a
    7-node tree at context 33 and a 3-token chain with no context -- each
    equal to the oracle's forward of that sequence alone, with its cache rows
    written at its own slots."""
    model = P.make_model(orc, SMALL, dts, seed=61)
    rng = np.random.default_rng(62)
    seqs = [(rng.integers(0, 1000, 5).tolist(), None, 20, 40),
            (rng.integers(0, 1000, 7).tolist(), [-1, 0, 0, 1, 1, 2, -1], 33, 48),
            (rng.integers(0, 1000, 3).tolist(), None, 0, 16)]
    for (got, want, (kg, vg), (kc, vc)), (toks, par, npast, cap) in zip(
            run_batch(gctx, orc, model, seqs, 16), seqs):
        assert rel_err_rows(got, want) < LOGIT_TOL, (npast, par)
        np.testing.assert_allclose(kg.astype(np.float32), kc.astype(np.float32), rtol=3e-3,
                                   atol=3e-3)
        assert np.array_equal(kg[:, :npast], kc[:, :npast])


@pytest.mark.parametrize("M", [9, 30, 64, 200])
def test_large_chain_one_pass(gctx, orc, M):
    """A single sequence of 9, 30, 64 and 200 tokens (one 16-, 32- and
    64-token tile, and four 64-token tiles) through the one-pass GEMMs, Q4_K
    projections and down, Q8_0 head."""
    dts = dict(tok_embd=P.Q8_0, output=P.Q8_0, q=P.Q4_K, k=P.Q4_K, v=P.Q4_K, o=P.Q4_K,
               gate=P.Q4_K, up=P.Q4_K, down=P.Q4_K)
    cfg = P.model_cfg(1, 1024, 8, 2, 128, 2048, 700, rope_theta=500000.0)
    model = P.make_model(orc, cfg, dts, seed=70 + M)
    toks = np.random.default_rng(M).integers(0, 700, M).tolist()
    (got, want, _, _), = run_batch(gctx, orc, model, [(toks, None, 77, 77 + M + 3)], 256)
    assert rel_err_rows(got, want) < LOGIT_TOL


@pytest.mark.parametrize("d,M", [(12288, 9), (16384, 20)])
def test_wide_rows_one_pass(gctx, orc, d, M):
    """Model widths of 12288 and 16384 (three and four 4096-element chunks
    per thread in the one-row operand prep), 2 layers of Q4_K, chains of 9
    and 20 tokens: the plain prep of the embeddings, the fold of the o
    projection's split partials into the residual rows before the FFN and
    of ffn_down's before the second layer."""
    orc.set_threads(16)
    V = 300
    cfg = P.model_cfg(2, d, d // 128, 8, 128, 1024, V, rope_theta=500000.0)
    rng = np.random.default_rng(d + M)
    model = {"cfg": dict(cfg)}

    def q(rows, cols):
        return q_rows(orc, rng, rows, cols, P.Q4_K, unique=1024)

    model["tok_embd"] = q(V, d)
    model["output"] = q(V, d)
    model["out_norm"] = norm_raw(rng, d)
    for l in range(2):
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, d)
        model[p + "ffn_norm"] = norm_raw(rng, d)
        for nm, rows, cols in (("q", d, d), ("k", 1024, d), ("v", 1024, d), ("o", d, d),
                               ("gate", 1024, d), ("up", 1024, d), ("down", 1024, d)):
            model[p + nm] = q(rows, cols)
    toks = rng.integers(0, V, M).tolist()
    (got, want, _, _), = run_batch(gctx, orc, model, [(toks, None, 33, 33 + M + 3)], 64)
    assert rel_err_rows(got, want) < LOGIT_TOL


@pytest.mark.parametrize("M", [12, 20, 130])
def test_large_chain_q6k_one_pass(gctx, orc, M):
    """Q6_K projections (q / k / v, o, gate / up with SwiGLU) and a Q6_K head
    through the one-pass GEMM's Q6_K operand (scale split 16 sh + sl), one
    16- and one 32-token tile, and three 64-token tiles; ffn_down Q4_K."""
    dts = dict(tok_embd=P.Q8_0, output=P.Q6_K, q=P.Q6_K, k=P.Q6_K, v=P.Q6_K, o=P.Q6_K,
               gate=P.Q6_K, up=P.Q6_K, down=P.Q4_K)
    cfg = P.model_cfg(2, 1024, 8, 2, 128, 2048, 700, rope_theta=500000.0)
    model = P.make_model(orc, cfg, dts, seed=90 + M)
    toks = np.random.default_rng(M + 1).integers(0, 700, M).tolist()
    (got, want, _, _), = run_batch(gctx, orc, model, [(toks, None, 40, 40 + M + 3)], 256)
    assert rel_err_rows(got, want) < LOGIT_TOL


def test_long_context_tree_chunk_groups(gctx, orc):
    """A 64-node tree over context 4030 with 64 query heads of 64 on 8 kv
    heads: the one-chunk attention grid would hold 8320 workgroups, so each
    workgroup walks two chunks with a running maximum and sum (one partial
    per pair)."""
    cfg = P.model_cfg(1, 4096, 64, 8, 64, 1024, 300, rope_theta=500000.0)
    dts = dict(tok_embd=P.Q8_0, output=P.Q8_0, q=P.Q8_0, k=P.Q8_0, v=P.Q8_0, o=P.Q8_0,
               gate=P.Q8_0, up=P.Q8_0, down=P.Q8_0)
    model = P.make_model(orc, cfg, dts, seed=97)
    rng = np.random.default_rng(98)
    par = [-1] + [int(rng.integers(max(-1, i - 6), i)) for i in range(1, 64)]
    seqs = [(rng.integers(0, 300, 64).tolist(), par, 4030, 4030 + 64 + 2)]
    (got, want, _, _), = run_batch(gctx, orc, model, seqs, 64)
    assert rel_err_rows(got, want) < LOGIT_TOL


def test_batch_errors(gctx, orc):
    model = P.make_model(orc, SMALL, dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q8_0, k=P.Q8_0,
                                          v=P.Q8_0, o=P.Q8_0, gate=P.Q8_0, up=P.Q8_0,
                                          down=P.Q8_0), seed=5)
    tensors = upload(gctx, model)
    gm = gctx.model(SMALL, tensors, max_tokens=16)
    a, b = gm.kv(64), gm.kv(64)
    buf = gctx.buffer(16 * 1000 * 4)
    cases = [
        [(a, [1, 2], buf.ptr, None, False), (a, [3], buf.ptr, None, False)],   # shared cache
        [(a, [1, 2], buf.ptr, None, False), (b, [3], None, None, False)],      # mixed logits
        [(a, list(range(10)), None, None, False), (b, list(range(10)), None, None, False)],
    ]
    for c in cases:
        with pytest.raises(ftx.FtxError) as e:
            gm.verify_batch(c)
        assert e.value.code == -1  # FTX_E_INVALID
    for o in (buf, a, b, gm):
        o.free()
    for t in tensors.values():
        t.free()


def test_batch_70b_layer_shape_trees(gctx, orc):
    """The 70B layer shape (d 8192, 64 / 8 heads x 128, FFN 28672, vocab
    128256, all Q4_K), 2 layers, four sequences each verifying a 64-node
    draft tree (depth <= 6, branching <= 4) at context 8192 in one step (256
    tokens), then residual acceptance of each sequence's device logits,
    identical on the device and in the oracle."""
    orc.set_threads(16)
    V, d, ff = 128256, 8192, 28672
    cfg = P.model_cfg(2, d, 64, 8, 128, ff, V, rope_theta=500000.0)
    rng = np.random.default_rng(701)
    model = {"cfg": dict(cfg)}

    def q(rows, cols):
        return q_rows(orc, rng, rows, cols, P.Q4_K, unique=1024)

    model["tok_embd"] = q(V, d)
    model["output"] = q(V, d)
    model["out_norm"] = norm_raw(rng, d)
    for l in range(2):
        p = "blk.%d." % l
        model[p + "attn_norm"] = norm_raw(rng, d)
        model[p + "ffn_norm"] = norm_raw(rng, d)
        for nm, rows, cols in (("q", d, d), ("k", 1024, d), ("v", 1024, d), ("o", d, d),
                               ("gate", ff, d), ("up", ff, d), ("down", ff, d)):
            model[p + nm] = q(rows, cols)
    seqs = []
    for s in range(4):
        par = random_tree(rng, 64, 6, 4)
        seqs.append((rng.integers(0, V, 64).tolist(), par, 8192 - 64 - 8 * s, 8192))
    res = run_batch(gctx, orc, model, seqs, 256)
    for s, ((got, want, _, _), (toks, par, npast, cap)) in enumerate(zip(res, seqs)):
        assert rel_err_rows(got, want) < LOGIT_TOL, s
        base = (rng.standard_normal(V) * 2).astype(np.float32)
        qd = rng.dirichlet(np.ones(V), size=64).astype(np.float32)
        bb, rb, qb = gctx.buffer(V * 4), gctx.buffer(64 * V * 4), gctx.buffer(64 * V * 4)
        bb.write(base)
        rb.write(got)
        qb.write(qd)
        props = np.array(toks, np.int32)
        g = gctx.accept(bb.ptr, rb.ptr, 64, V, props, ftx.ACCEPT_RESIDUAL, temp=0.8, rng=900 + s,
                        parents=par, q_ptr=qb.ptr)
        o = orc.verify_accept(base, got, props, P.ACCEPT_RESIDUAL, temp=0.8, seed=900 + s,
                              parents=par, q=qd)
        assert (g["accepted"], g["bonus"], g["rng"]) == (o["accepted"], o["bonus"], o["rng"]), s
        for b_ in (bb, rb, qb):
            b_.free()
