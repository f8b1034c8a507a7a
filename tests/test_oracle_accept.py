"""Pins of the oracle's acceptance sampling.

Reference KAT (src/tests/test_core.cpp:348-356), published SplitMix64
outputs, bit-exact agreement with the reference's accept_chain_* and
softmax_prob where built, reductions between modes, and a chi-square test
that multi-candidate residual sampling reproduces the target distribution.
"""
import numpy as np
import pytest

import pyoracle as P


def test_reference_kat_accept_chain(orc):
    base = np.array([9, 1, 1, 1], np.float32)
    rows = np.array([1, 9, 1, 1, 1, 1, 9, 1], np.float32)
    assert orc.accept_chain_greedy(base, rows, [0, 1, 2]) == 3
    assert orc.accept_chain_greedy(base, rows, [0, 3, 2]) == 1


def test_splitmix64_published_outputs(orc):
    # SplitMix64 from state 0: first outputs of the published generator
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    s = 0
    for w in want:
        v, s = orc.rng_next(s)
        assert v == w
    u = orc.rng_floats(0, 1)[0]
    assert u == np.float32((0xE220A8397B1DCDAF >> 40) / 16777216.0)


def test_argmax_first_max(orc):
    assert orc.argmax(np.array([1, 3, 3, 2], np.float32)) == 1


def rand_case(rng, k, V, spread=3.0):
    base = (rng.standard_normal(V) * spread).astype(np.float32)
    rows = (rng.standard_normal((k, V)) * spread).astype(np.float32)
    props = rng.integers(0, V, k).astype(np.int32)
    return base, rows, props


def test_accept_sampling_matches_reference(orc, ref):
    rng = np.random.default_rng(21)
    for trial in range(200):
        k, V = 6, 64
        base, rows, props = rand_case(rng, k, V, spread=1.0)
        # make acceptance likely: drafts near the target argmax
        for a in range(k):
            pred = base if a == 0 else rows[a - 1]
            if rng.random() < 0.7:
                props[a] = int(np.argmax(pred))
        pd = rng.random(k).astype(np.float32) * 0.5
        pd[rng.random(k) < 0.15] = 0.0        # greedy positions
        seed = int(rng.integers(1, 2**63))
        a1, s1 = orc.accept_chain_sampling(base, rows, pd, props, 1.0, seed)
        a2, s2 = ref.accept_chain_sampling(base, rows, pd, props, 1.0, seed)
        assert (a1, s1) == (a2, s2)
        assert orc.accept_chain_greedy(base, rows, props) == ref.accept_chain_greedy(base, rows, props)
        for a in range(k):
            pred = base if a == 0 else rows[a - 1]
            assert orc.softmax_prob(pred, props[a]) == ref.softmax_prob(pred, props[a])


def test_softmax_prob_temperature(orc):
    rng = np.random.default_rng(22)
    lg = rng.standard_normal(100).astype(np.float32) * 3
    for T in (0.5, 0.8, 2.0):
        z = (lg - lg.max()).astype(np.float32) / np.float32(T)
        p = np.exp(z.astype(np.float64))
        p /= p.sum()
        assert abs(orc.softmax_prob(lg, 7, T) - p[7]) <= 1e-7 * max(p[7], 1e-30) + 1e-12


def test_verify_greedy_chain(orc):
    rng = np.random.default_rng(23)
    for _ in range(100):
        base, rows, props = rand_case(rng, 5, 16)
        for a in range(5):
            if rng.random() < 0.8:
                props[a] = int(np.argmax(base if a == 0 else rows[a - 1]))
        r = orc.verify_accept(base, rows, props, P.ACCEPT_GREEDY)
        n = orc.accept_chain_greedy(base, rows, props)
        assert r["accepted"] == list(range(n))
        after = base if n == 0 else rows[n - 1]
        assert r["bonus"] == int(np.argmax(after))


def test_verify_ratio_equals_chain_sampling(orc):
    rng = np.random.default_rng(24)
    for _ in range(100):
        base, rows, props = rand_case(rng, 6, 32, spread=1.0)
        pd = (rng.random(6) * 0.3).astype(np.float32)
        seed = int(rng.integers(1, 2**63))
        a, s_after = orc.accept_chain_sampling(base, rows, pd, props, 0.8, seed)
        ss = int(rng.integers(1, 2**63))
        r = orc.verify_accept(base, rows, props, P.ACCEPT_RATIO, temp=0.8, seed=seed, pd=pd,
                              sampler_state=ss)
        assert r["accepted"] == list(range(a))
        # the acceptance stream stops at the decisions (src/spec.cpp:214-238);
        # the bonus is Sampler::sample of the row after the last accepted
        # node, from the sampler's own state
        assert r["rng"] == s_after
        after = base if a == 0 else rows[a - 1]
        assert (r["bonus"], r["sampler_state"]) == orc.sampler_sample(after, 0.8, 40, 0.95, ss)


def test_residual_single_child_equals_ratio(orc):
    """One child per level: RESIDUAL takes the same decisions as RATIO."""
    rng = np.random.default_rng(25)
    V, k = 24, 5
    for _ in range(100):
        base, rows, props = rand_case(rng, k, V, spread=1.0)
        q = rng.dirichlet(np.ones(V), size=k).astype(np.float32)
        for a in range(k):
            qq = q[a].astype(np.float64)
            props[a] = int(rng.choice(V, p=qq / qq.sum()))
        pd = q[np.arange(k), props]
        seed = int(rng.integers(1, 2**63))
        r1 = orc.verify_accept(base, rows, props, P.ACCEPT_RATIO, temp=0.8, seed=seed, pd=pd)
        r2 = orc.verify_accept(base, rows, props, P.ACCEPT_RESIDUAL, temp=0.8, seed=seed, q=q,
                               parents=list(range(-1, k - 1)))
        assert r1["accepted"] == r2["accepted"]


def tree_children(parents):
    ch = {}
    for i, p in enumerate(parents):
        ch.setdefault(p, []).append(i)
    return ch


def test_greedy_tree_brute_force(orc):
    rng = np.random.default_rng(26)
    parents = [-1, -1, -1, 0, 0, 1, 3, 3]
    ch = tree_children(parents)
    for _ in range(100):
        V = 6
        base, rows, props = rand_case(rng, len(parents), V)
        r = orc.verify_accept(base, rows, props, P.ACCEPT_GREEDY, parents=parents)
        cur, path = -1, []
        while True:
            row = base if cur < 0 else rows[cur]
            g = int(np.argmax(row))
            nxt = [c for c in ch.get(cur, []) if props[c] == g]
            if not nxt:
                break
            cur = nxt[0]
            path.append(cur)
        assert r["accepted"] == path
        assert r["bonus"] == int(np.argmax(base if cur < 0 else rows[cur]))


def test_residual_tree_reproduces_target(orc):
    """Speculative sampling is distribution-preserving: the first emitted
    token (first accepted node's token, else the bonus) is distributed as the
    target p_T(base_row), whatever the draft q (chi-square, V = 6)."""
    rng = np.random.default_rng(27)
    V, T = 6, 0.8
    parents = [-1, -1, -1, 0, 0, 1]
    base = np.array([2.0, 0.5, -1.0, 1.0, 0.0, -0.5], np.float32)
    rows = (rng.standard_normal((len(parents), V))).astype(np.float32)
    qroot = np.array([0.05, 0.4, 0.3, 0.05, 0.1, 0.1], np.float32)
    qs = rng.dirichlet(np.ones(V), size=len(parents)).astype(np.float32)
    ch = tree_children(parents)
    counts = np.zeros(V)
    n = 6000
    for trial in range(n):
        q = qs.copy()
        props = np.zeros(len(parents), np.int32)
        for c in ch[-1]:
            q[c] = qroot
        for par, kids in ch.items():
            for c in kids:
                qq = q[c].astype(np.float64)
                props[c] = rng.choice(V, p=qq / qq.sum())
        r = orc.verify_accept(base, rows, props, P.ACCEPT_RESIDUAL, temp=T,
                              seed=trial * 7919 + 1, q=q, parents=parents)
        first = props[r["accepted"][0]] if r["accepted"] else r["bonus"]
        counts[first] += 1
    z = (base - base.max()) / np.float32(T)
    p = np.exp(z.astype(np.float64))
    p /= p.sum()
    chi2 = (((counts - n * p) ** 2) / (n * p)).sum()
    assert chi2 < 20.5, (chi2, counts / n, p)     # 5 dof, p ~ 0.001


def test_sample_weights(orc):
    w = np.array([0.0, 1.0, 0.0, 3.0], np.float64)
    assert orc.sample_weights(w, 0.0) == 1
    assert orc.sample_weights(w, 0.2499) == 1
    assert orc.sample_weights(w, 0.25) == 3
    assert orc.sample_weights(w, 0.9999999) == 3


@pytest.mark.parametrize("V", [7, 64, 1001, 32000])
def test_sampler_sample_matches_reference(orc, ref, V):
    """Sampler::sample (include/ft/sampler.h:30-94): the oracle's restatement
    against the reference's own, on the same rows and states: temperature,
    top-k, top-p (each on and off), the state carried from draw to draw."""
    rng = np.random.default_rng(V)
    state_o = state_r = P.SAMPLER_SEED
    for trial in range(40):
        lg = (rng.standard_normal(V) * rng.choice([0.5, 2.0, 6.0])).astype(np.float32)
        temp = float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.7]))
        top_k = int(rng.choice([0, 1, 5, 40, V, V + 3]))
        top_p = float(rng.choice([0.5, 0.9, 0.95, 1.0]))
        to, state_o = orc.sampler_sample(lg, temp, top_k, top_p, state_o)
        tr, state_r = ref.sampler_sample(lg, temp, top_k, top_p, state_r)
        assert (to, state_o) == (tr, state_r), (trial, temp, top_k, top_p)


def test_sampler_sample_distribution(orc):
    """The draws follow the top-k / top-p renormalised softmax (chi-square on a
    6-token row): p = softmax(l / T) restricted to the 3 largest, then to the
    smallest prefix whose mass reaches top_p."""
    lg = np.array([2.0, 0.5, 1.0, -1.0, 1.5, 0.0], np.float32)
    T, k, p = 0.8, 3, 0.9
    e = np.exp((lg - lg.max()) / T)
    q = e / e.sum()
    order = np.argsort(-q)[:k]
    kept = np.zeros_like(q)
    kept[order] = q[order] / q[order].sum()
    cum = np.cumsum(kept[order])
    cut = int(np.searchsorted(cum, p) + 1)
    final = np.zeros_like(q)
    final[order[:cut]] = kept[order[:cut]] / kept[order[:cut]].sum()
    n = 20000
    counts = np.zeros(6)
    s = P.SAMPLER_SEED
    for _ in range(n):
        t, s = orc.sampler_sample(lg, T, k, p, s)
        counts[t] += 1
    assert counts[final == 0].sum() == 0
    nz = final > 0
    chi2 = ((counts[nz] - n * final[nz]) ** 2 / (n * final[nz])).sum()
    assert chi2 < 15.0, (counts, final)
