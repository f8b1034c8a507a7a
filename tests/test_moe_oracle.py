"""The oracle's MoE FFN and attention extras (bias on q / k / v, per-head
q / k RMSNorm) pinned three ways:
  - routing against a brute-force restatement (float32 sums, stable
    descending order) and hand-made cases (ties, zero weights, bias);
  - one expert's FFN against the reference's ExpertStreamer at several
    window sizes (bit-exact) and against the direct loop of the reference's
    chunker test (src/tests/test_core.cpp:307-346);
  - whole models written as GGUF and stepped token by token through the
    reference Engine (src/engine.cpp:179-258, 519-551): bit-exact logits.
"""
import numpy as np
import pytest

import pyoracle as P
from xwfes_amd import gguf as G

DT = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q8_0, k=P.Q4_0, v=P.Q8_0, o=P.Q8_0,
          gate=P.Q4_0, up=P.Q4_0, down=P.Q8_0, gate_inp=P.F32, gate_exps=P.Q4_0,
          up_exps=P.Q4_0, down_exps=P.Q4_0, gate_sh=P.Q8_0, up_sh=P.Q8_0, down_sh=P.Q8_0)


def brute_route(orc, router, U, bias=None):
    """Selection and renormalisation by brute force over the probabilities
    of the oracle's softmax (itself pinned against the reference's)."""
    r = np.array(router, np.float32)
    M, E = r.shape
    te = np.empty((M, U), np.int32)
    tw = np.empty((M, U), np.float32)
    used = []
    for m in range(M):
        row = (r[m] + (0 if bias is None else np.asarray(bias, np.float32))).astype(np.float32)
        p = orc.softmax(row)
        order = sorted(range(E), key=lambda j: (-p[j], j))[:U]
        wsum = np.float32(0)
        for j in order:
            wsum = np.float32(wsum + p[j])
        inv = np.float32(1) / wsum if wsum > 0 else np.float32(0)
        te[m] = order
        tw[m] = [np.float32(p[j] * inv) for j in order]
        for j in order:
            if j not in used:
                used.append(j)
    return te, tw, used


def test_route_matches_brute_force(orc):
    rng = np.random.default_rng(3)
    for E, U, M in ((8, 2, 16), (64, 6, 9), (4, 4, 5), (16, 1, 7)):
        r = rng.standard_normal((M, E)).astype(np.float32) * 3
        bias = rng.standard_normal(E).astype(np.float32) if E == 64 else None
        _, te, tw, used = orc.moe_route(r, U, bias)
        bte, btw, bused = brute_route(orc, r, U, bias)
        assert np.array_equal(te, bte) and np.array_equal(tw, btw), (E, U)
        assert used.tolist() == bused
        np.testing.assert_allclose(tw.sum(1), 1.0, rtol=1e-6)


def test_route_ties_and_order(orc):
    # equal logits: the lower expert index first; first-use order over
    # (token, rank); a -inf logit never wins over a finite one
    r = np.array([[1, 1, 1, 1], [0, 5, 5, -np.inf], [2, 0, 0, 3]], np.float32)
    _, te, tw, used = orc.moe_route(r, 2)
    assert te.tolist() == [[0, 1], [1, 2], [3, 0]]
    assert tw[0].tolist() == [0.5, 0.5] and tw[1].tolist() == [0.5, 0.5]
    assert used.tolist() == [0, 1, 2, 3]
    # a bias moves the choice; the weights are the biased probabilities
    _, te, tw, _ = orc.moe_route(r[:1], 1, np.array([0, 0, 1, 0], np.float32))
    assert te.tolist() == [[2]] and tw.tolist() == [[1.0]]


def rand_q(orc, rng, rows, cols, dt, std=0.3):
    return orc.quantize((rng.standard_normal((rows, cols)) * std).astype(np.float32), dt)


def test_expert_ffn_equals_direct_loop(orc):
    """The reference chunker test's direct loop, restated: h_i = silu(g_i) u_i,
    out += sum_i h_i down_i (F32 weights so the loop is exact float math)."""
    rng = np.random.default_rng(5)
    K, FF, M = 16, 48, 3
    g, u, d = (rng.standard_normal((FF, K)).astype(np.float32) * 0.5 for _ in range(3))
    x = rng.standard_normal((M, K)).astype(np.float32)
    got = orc.expert_ffn(x, g, u, P.F32, d, P.F32, FF)
    want = np.zeros((M, K), np.float64)
    for m in range(M):
        for i in range(FF):
            gg, uu = float(x[m] @ g[i]), float(x[m] @ u[i])
            want[m] += (gg / (1 + np.exp(-gg))) * uu * d[i]
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5


@pytest.mark.parametrize("dt", [P.Q4_0, P.Q4_1, P.Q8_0, P.F16, P.BF16])
def test_expert_ffn_equals_reference_streamer(orc, ref, dt):
    """Windows of 32, 64 and all neurons through ExpertStreamer::run give
    exactly the oracle's one pass (the down rows add in ascending order).
    The reference sizes its rows for 32-element block types only
    (include/ft/types.h:42-52), so K-quant experts are not among them."""
    rng = np.random.default_rng(dt)
    K, F, M = 256, 192, 5
    g, u, d = (rand_q(orc, rng, F, K, dt, 0.05) for _ in range(3))
    x = rng.standard_normal((M, K)).astype(np.float32)
    y0 = rng.standard_normal((M, K)).astype(np.float32)
    want = orc.expert_ffn(x, g, u, dt, d, dt, F, out=y0)
    for chunk in (32, 64, F):
        got = ref.expert_stream(x, g, u, d, dt, F, chunk, out=y0)
        assert np.array_equal(got, want), chunk


CASES = [
    # Mixtral-like: 8 experts, top-2
    ("llama", P.model_cfg(2, 64, 4, 2, 16, 96, 50, n_expert=8, n_expert_used=2), ()),
    # top-3 of 4 with a router bias and a shared expert
    ("llama", P.model_cfg(2, 64, 4, 2, 16, 64, 50, n_expert=4, n_expert_used=3),
     ("router_bias", "gate_sh", "up_sh", "down_sh")),
    # qwen2-style q / k / v bias (neox rope by the arch name)
    ("qwen2", P.model_cfg(2, 64, 4, 2, 16, 96, 50, rope_neox=1), ("q_bias", "k_bias", "v_bias")),
    # qwen3-style per-head q / k norms
    ("qwen3", P.model_cfg(2, 64, 4, 2, 16, 96, 50, rope_neox=1), ("q_norm", "k_norm")),
    # both, on a MoE model
    ("qwen3moe", P.model_cfg(2, 64, 4, 2, 16, 64, 50, rope_neox=1, n_expert=6, n_expert_used=2),
     ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm")),
]


def oracle_steps(orc, model, toks, cap=64):
    cfg = model["cfg"]
    shape = (cfg["n_layer"], cap, cfg["n_head_kv"] * cfg["head_dim"])
    kc, vc = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    return np.array([orc.forward(model, kc, vc, i, [t])[0] for i, t in enumerate(toks)])


@pytest.mark.parametrize("case", range(len(CASES)))
def test_reference_engine_steps_equal_oracle(tmp_path, orc, ref, case):
    arch, cfg, extras = CASES[case]
    model = P.make_model(orc, cfg, DT, seed=5 + case, extras=extras)
    p = str(tmp_path / "m.gguf")
    G.write_gguf(p, G.model_kv(cfg, arch=arch), G.model_tensor_list(model))
    toks = [3, 17, 42, 0, 9, 49, 5, 33]
    h = ref.engine_load(p, 1, 64)
    try:
        rows = np.array([ref.engine_step(h, t) for t in toks])
    finally:
        ref.engine_free(h)
    want = oracle_steps(orc, model, toks)
    assert np.array_equal(rows, want)


def test_moe_block_forward_equals_steps(orc):
    """An M-token block routes every token alone; only the order in which a
    token's experts add up (first use over the block) differs from steps."""
    arch, cfg, extras = CASES[1]
    model = P.make_model(orc, cfg, DT, seed=44, extras=extras)
    toks = [3, 17, 42, 0, 9, 49, 5, 33]
    shape = (cfg["n_layer"], 64, cfg["n_head_kv"] * cfg["head_dim"])
    blk = orc.forward(model, np.zeros(shape, np.float32), np.zeros(shape, np.float32), 0, toks)
    st = oracle_steps(orc, model, toks)
    assert np.abs(blk - st).max() / np.abs(st).max() < 1e-6
    # the extras change the result: the same model without them differs
    plain = {k: v for k, v in model.items() if not k.endswith(extras)}
    pb = orc.forward(plain, np.zeros(shape, np.float32), np.zeros(shape, np.float32), 0, toks)
    assert np.abs(pb - blk).max() > 1e-3
