"""Pins of the oracle's linear algebra, host ops and forward.

matmul/down_axpy: bit-exact against the reference's CpuBackend::matmul
(M = 1, and the documented M-sum behaviour for M > 1) and matmul_down_axpy;
fp64 brute force on dequantised weights.  Norm / RoPE / softmax: closed forms.
Forward: M-token == M single-token steps (exact), tree == chain of each
root-to-node path (exact), and against the reference Engine where built.
"""
import numpy as np
import pytest

import pyoracle as P


def rand_w(orc, rng, rows, cols, dtype):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    return orc.quantize(w, dtype)


@pytest.mark.parametrize("dtype", [P.F32, P.Q8_0, P.Q4_0, P.F16])
def test_matmul_vs_reference(orc, ref, dtype):
    rng = np.random.default_rng(11)
    K, N = 256, 48
    raw = rand_w(orc, rng, N, K, dtype)
    x = rng.standard_normal((3, K)).astype(np.float32)
    y = orc.matmul(x, raw, dtype, N)
    # M = 1: the reference is correct and must agree bit-for-bit
    y1 = ref.cpu_matmul(x[:1], raw, dtype, N, threads=2)
    assert np.array_equal(y[0].view(np.uint32), y1.view(np.uint32))
    # M = 3: the reference returns sum_m x_m . W_r in y[r] (M-sum bug)
    y3 = ref.cpu_matmul(x, raw, dtype, N)
    acc = y[0].copy()
    for m in (1, 2):
        acc = (acc + y[m]).astype(np.float32)
    assert np.array_equal(acc.view(np.uint32), y3.view(np.uint32))


@pytest.mark.parametrize("dtype", [P.Q4_K, P.Q6_K, P.Q8_0, P.Q4_0])
def test_matmul_brute_force(orc, dtype):
    rng = np.random.default_rng(12)
    K, N, M = 512, 40, 5
    raw = rand_w(orc, rng, N, K, dtype)
    W = orc.dequant(raw, dtype, K, rows=N).astype(np.float64)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = orc.matmul(x, raw, dtype, N)
    want = x.astype(np.float64) @ W.T
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()
    for m in range(M):   # M rows == M independent single-row products
        assert np.array_equal(orc.matmul(x[m:m + 1], raw, dtype, N)[0], y[m])


@pytest.mark.parametrize("dtype", [P.F32, P.Q8_0, P.Q4_0])
@pytest.mark.parametrize("threads", [1, 4])
def test_down_axpy_vs_reference(orc, ref, dtype, threads):
    rng = np.random.default_rng(13)
    n_in, N, M = 96, 512, 3
    raw = rand_w(orc, rng, n_in, N, dtype)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    x[1, ::7] = 0.0
    orc.set_threads(threads)
    try:
        y = orc.down_axpy(x, raw, dtype, N)
    finally:
        orc.set_threads(1)
    assert np.array_equal(y.view(np.uint32), ref.down_axpy(x, raw, dtype, N).view(np.uint32))


def test_down_axpy_brute_force_kquant(orc):
    rng = np.random.default_rng(14)
    n_in, N, M = 64, 512, 4
    for dtype in (P.Q4_K, P.Q6_K):
        raw = rand_w(orc, rng, n_in, N, dtype)
        W = orc.dequant(raw, dtype, N, rows=n_in).astype(np.float64)
        x = rng.standard_normal((M, n_in)).astype(np.float32)
        y = orc.down_axpy(x, raw, dtype, N)
        want = x.astype(np.float64) @ W
        assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()


def test_rms_norm_closed_form(orc):
    x = np.full(64, 3.0, np.float32)
    w = np.arange(64, dtype=np.float32)
    out = orc.rms_norm(x, w, 1e-5)
    inv = 1.0 / np.sqrt(9.0 + 1e-5)
    assert np.allclose(out, 3.0 * inv * w, rtol=1e-6)
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4096).astype(np.float32)
    out = orc.rms_norm(x, None, 1e-5)
    assert abs(np.mean(out.astype(np.float64) ** 2) - 1.0) < 1e-4


def test_rope_closed_forms(orc):
    rng = np.random.default_rng(1)
    v = rng.standard_normal(128).astype(np.float32)
    for neox in (0, 1):
        assert np.array_equal(orc.rope(v, 0, 10000.0, neox), v)   # pos 0: identity
    # interleaved pair 0 rotates by angle pos (frequency 1)
    r = orc.rope(v, 3, 10000.0, 0)
    c, s = np.float32(np.cos(3.0)), np.float32(np.sin(3.0))
    assert r[0] == np.float32(v[0] * c - v[1] * s)
    assert r[1] == np.float32(v[0] * s + v[1] * c)
    # pair norms preserved; neox == interleaved under the pair permutation
    perm = np.concatenate([np.arange(0, 128, 2), np.arange(1, 128, 2)])
    a = orc.rope(v, 1234, 500000.0, 0)
    b = orc.rope(v[perm], 1234, 500000.0, 1)
    assert np.array_equal(a[perm], b)
    n0 = v[0::2].astype(np.float64) ** 2 + v[1::2].astype(np.float64) ** 2
    n1 = a[0::2].astype(np.float64) ** 2 + a[1::2].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-5)


def test_softmax(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(1000).astype(np.float32) * 5
    p = orc.softmax(x)
    want = np.exp(x.astype(np.float64) - x.max())
    want /= want.sum()
    assert np.allclose(p, want, rtol=1e-5, atol=1e-9)
    assert np.array_equal(orc.softmax(x + 7.0), orc.softmax(x)) or \
        np.allclose(orc.softmax(x + 7.0), p, rtol=1e-6)


TINY = P.model_cfg(2, 64, 4, 2, 16, 96, 50, rope_theta=10000.0)
TINY_DT = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q4_0, k=P.Q8_0, v=P.Q4_0, o=P.Q8_0,
               gate=P.Q4_0, up=P.Q4_0, down=P.Q8_0)


def kv_for(cfg, cap, dtype=np.float16, seed=5, npast=0):
    rng = np.random.default_rng(seed)
    shape = (cfg["n_layer"], cap, cfg["n_head_kv"] * cfg["head_dim"])
    k = np.zeros(shape, dtype)
    v = np.zeros(shape, dtype)
    k[:, :npast] = rng.standard_normal((shape[0], npast, shape[2]))
    v[:, :npast] = rng.standard_normal((shape[0], npast, shape[2]))
    return k, v


def test_forward_block_equals_steps(orc):
    model = P.make_model(orc, TINY, TINY_DT, seed=3)
    toks = [3, 17, 42, 0, 9]
    k1, v1 = kv_for(TINY, 32, npast=7)
    k2, v2 = k1.copy(), v1.copy()
    blk = orc.forward(model, k1, v1, 7, toks)
    for i, t in enumerate(toks):
        row = orc.forward(model, k2, v2, 7 + i, [t])
        assert np.array_equal(row[0], blk[i])
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


def test_forward_tree_equals_paths(orc):
    model = P.make_model(orc, TINY, TINY_DT, seed=4)
    # root children 0,1; node 0 -> 2,3; node 3 -> 4
    parents = [-1, -1, 0, 0, 3]
    toks = [5, 6, 7, 8, 9]
    kt, vt = kv_for(TINY, 32, npast=6)
    tree = orc.forward(model, kt.copy(), vt.copy(), 6, toks, parents=parents)
    paths = {0: [0], 1: [1], 2: [0, 2], 3: [0, 3], 4: [0, 3, 4]}
    for node, path in paths.items():
        kc, vc = kt.copy(), vt.copy()
        chain = orc.forward(model, kc, vc, 6, [toks[i] for i in path])
        assert np.array_equal(chain[-1], tree[node]), node
    # a chain given as explicit parents is the reference causal forward
    a = orc.forward(model, kt.copy(), vt.copy(), 6, toks, parents=[-1, 0, 1, 2, 3])
    b = orc.forward(model, kt.copy(), vt.copy(), 6, toks)
    assert np.array_equal(a, b)


def test_kv_commit_tree_path_equals_chain(orc):
    """Committing an accepted tree path leaves the cache exactly as a chain
    forward of that path would, so the next step's logits are the chain's."""
    model = P.make_model(orc, TINY, TINY_DT, seed=5)
    parents = [-1, -1, 0, 0, 3, 1]
    toks = [5, 6, 7, 8, 9, 10]
    path = [0, 3, 4]  # root -> node 3 -> node 4
    kt, vt = kv_for(TINY, 32, npast=6)
    k1, v1 = kt.copy(), vt.copy()
    orc.forward(model, k1, v1, 6, toks, parents=parents)
    npast = P.Oracle.kv_commit(k1, v1, 6, path)
    assert npast == 9
    nxt = orc.forward(model, k1, v1, npast, [11])
    k2, v2 = kt.copy(), vt.copy()
    chain = orc.forward(model, k2, v2, 6, [toks[i] for i in path] + [11])
    assert np.array_equal(nxt[0], chain[-1])
    assert np.array_equal(k1[:, :10], k2[:, :10]) and np.array_equal(v1[:, :10], v2[:, :10])


def test_kv_commit_chain_and_errors(orc):
    k, v = kv_for(TINY, 16, npast=4)
    k[:, 4:9] = 1.0 + np.arange(5)[None, :, None]
    v[:, 4:9] = -1.0 - np.arange(5)[None, :, None]
    k0, v0 = k.copy(), v.copy()
    # a chain moves nothing
    assert P.Oracle.kv_commit(k, v, 4, [0, 1, 2]) == 7
    assert np.array_equal(k, k0) and np.array_equal(v, v0)
    # a path overlapping its own destinations: nodes 1, 2, 4 -> slots 4, 5, 6
    assert P.Oracle.kv_commit(k, v, 4, [1, 2, 4]) == 7
    assert np.array_equal(k[:, 4:7], k0[:, [5, 6, 8]]) and np.array_equal(v[:, 4:7], v0[:, [5, 6, 8]])
    for bad in ([1, 1], [2, 1], [0, 0], [20]):
        with pytest.raises(ValueError):
            P.Oracle.kv_commit(k.copy(), v.copy(), 4, bad)
