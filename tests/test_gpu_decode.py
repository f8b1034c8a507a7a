"""Decode (Engine::step, src/engine.cpp:650-658) and prefill
(Engine::prefill, src/engine.cpp:598-648, without the prefix cache) through
the verify-step kernels, on the GPU: a prompt prefilled in advancing chains
(the LM head on the last chain only) and then stepped token by token gives
the logits and KV rows of the oracle's forward of the whole sequence from an
empty cache (logits within 1e-3 relative per row; fp16 KV rows within fp16
rounding)."""
import numpy as np
import pytest

import pyoracle as P
from xwfes_amd import ftx

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3

MODELS = {
    "tiny": (P.model_cfg(2, 64, 4, 2, 16, 96, 50, rope_theta=10000.0),
             dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q4_0, k=P.Q8_0, v=P.Q4_0, o=P.Q8_0,
                  gate=P.Q4_0, up=P.Q4_0, down=P.Q8_0)),
    "hd128_kquant": (P.model_cfg(2, 1024, 8, 2, 128, 1024, 1000, rope_theta=500000.0),
                     dict(tok_embd=P.Q4_K, output=P.Q6_K, q=P.Q4_K, k=P.Q4_K, v=P.Q6_K,
                          o=P.Q4_K, gate=P.Q4_K, up=P.Q4_K, down=P.Q6_K)),
}


def rel_err_rows(a, b):
    a = np.atleast_2d(a).astype(np.float64)
    b = np.atleast_2d(b).astype(np.float64)
    return (np.abs(a - b).max(axis=1) / np.maximum(np.abs(b).max(axis=1), 1e-30)).max()


@pytest.mark.parametrize("name", sorted(MODELS))
@pytest.mark.parametrize("chunk", [8, 3])
def test_prefill_then_steps(gctx, orc, name, chunk):
    cfg, dts = MODELS[name]
    model = P.make_model(orc, cfg, dts, seed=21)
    tensors = {n: gctx.upload(t["raw"], t["dtype"], (t["ne0"], t["ne1"]))
               for n, t in model.items() if n != "cfg"}
    gm = gctx.model(cfg, tensors, max_tokens=8)
    cap = 128
    kv = gm.kv(cap)
    V = cfg["vocab"]
    rng = np.random.default_rng(5)
    prompt = [int(t) for t in rng.integers(0, V, 21)]
    steps = [int(t) for t in rng.integers(0, V, 3)]
    seq = prompt + steps
    shape = kv.shape
    kc = np.zeros(shape, np.float16)
    vc = np.zeros(shape, np.float16)
    want = orc.forward(model, kc, vc, 0, seq)
    buf = gctx.buffer(8 * V * 4)
    kv.truncate(0)
    rows = gm.prefill(kv, prompt, buf.ptr, chunk=chunk)
    gctx.sync()
    got = buf.read(np.float32, rows * V).reshape(rows, V)
    assert rows == len(prompt) - (len(prompt) - 1) // chunk * chunk
    assert rel_err_rows(got, want[len(prompt) - rows:len(prompt)]) < LOGIT_TOL
    assert kv.pointers()[2] == len(prompt)
    for i, t in enumerate(steps):
        gm.step(kv, t, buf.ptr)
        gctx.sync()
        got = buf.read(np.float32, V)
        assert rel_err_rows(got, want[len(prompt) + i]) < LOGIT_TOL, i
    assert kv.pointers()[2] == len(seq)
    kg, vg = kv.read()
    n = len(seq)
    assert np.abs(kg[:, :n].astype(np.float32) - kc[:, :n].astype(np.float32)).max() < 2e-2
    assert np.abs(vg[:, :n].astype(np.float32) - vc[:, :n].astype(np.float32)).max() < 2e-2
    # a prefill without logits leaves the same cache
    kv.truncate(0)
    assert gm.prefill(kv, prompt, None, chunk=chunk) == rows
    gctx.sync()
    k2, v2 = kv.read()
    m = len(prompt)
    assert np.array_equal(k2[:, :m], kg[:, :m]) and np.array_equal(v2[:, :m], vg[:, :m])
    buf.free()
    kv.free()
    gm.free()
    for t in tensors.values():
        t.free()
