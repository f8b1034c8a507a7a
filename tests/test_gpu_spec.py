"""Speculative generation on the GPU (xwfes_amd/spec.py: DraftModelDrafter,
generate) against the oracle's restatement (pyoracle.Oracle.generate, itself
pinned against the reference's generate in tests/test_spec.py): the same
emitted tokens with up to four draft tokens per round, greedy (temperature 0)
and sampled (temperatures 0.7 and 1, the reference's sampler defaults), with
the draft equal to the target and a different draft, with and without an
end-of-sequence token; plus the drafter's per-token pick (ftx_argmax_prob)
against Sampler::argmax and softmax_prob."""
import numpy as np
import pytest

import pyoracle as P
from xwfes_amd import ftx, spec

pytestmark = pytest.mark.gpu

CFG = P.model_cfg(2, 64, 4, 2, 16, 96, 48, rope_theta=10000.0)
DT = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q8_0, k=P.Q8_0, v=P.Q8_0, o=P.Q8_0,
          gate=P.Q8_0, up=P.Q8_0, down=P.Q8_0)


def peaked(orc, seed, gain):
    m = P.make_model(orc, CFG, DT, seed=seed)
    m["out_norm"]["raw"] = np.full(CFG["n_embd"], gain, np.float32).view(np.uint8).copy()
    return m


def upload(gctx, model):
    tensors = {n: gctx.upload(t["raw"], t["dtype"], (t["ne0"], t["ne1"]))
               for n, t in model.items() if n != "cfg"}
    gm = gctx.model(model["cfg"], tensors, max_tokens=8)
    gm.owned = list(tensors.values())
    return gm


@pytest.mark.parametrize("eos_at", [None, 5])
@pytest.mark.parametrize("temp", [0.0, 0.7, 1.0])
@pytest.mark.parametrize("same_draft", [True, False])
def test_generate_equals_oracle(gctx, orc, temp, same_draft, eos_at):
    """eos_at: the end-of-sequence id is the token the run without one
    emits at that position; both loops then stop as the reference's does."""
    target = peaked(orc, 31, 30.0)
    draft = target if same_draft else peaked(orc, 32, 25.0)
    tm = upload(gctx, target)
    dm = tm if same_draft else upload(gctx, draft)
    cap = 128
    tkv, dkv = tm.kv(cap), dm.kv(cap)
    drafter = spec.DraftModelDrafter(gctx, dm, dkv)
    prompt = [3, 17, 5, 40, 11, 9, 30, 2, 21]  # two prefill chains
    eos = -1
    if eos_at is not None:
        full, _ = orc.generate(target, draft, prompt, 30, spec_k=4, temp=temp, cap=cap)
        eos = full[eos_at]
    try:
        got, st = spec.generate(gctx, tm, tkv, drafter, prompt, 30, spec_k=4, temp=temp, eos=eos)
    finally:
        drafter.free()
    want, sto = orc.generate(target, draft, prompt, 30, spec_k=4, temp=temp, cap=cap, eos=eos)
    assert got == want, (st, sto, got, want)
    assert st == sto
    assert st["drafted"] > 0 and (st["accepted"] > 0 or not same_draft)
    if eos_at is not None:
        assert st["hit_eos"] and eos in got and len(got) <= eos_at + 5
    tkv.free()
    dkv.free()
    tm.free()
    if not same_draft:
        dm.free()


@pytest.mark.parametrize("V", [48, 1001, 128256])
def test_argmax_prob(gctx, orc, V):
    rng = np.random.default_rng(V)
    b = gctx.buffer(V * 4)
    for trial in range(6):
        row = (rng.standard_normal(V) * rng.choice([0.3, 3.0, 20.0])).astype(np.float32)
        if trial == 5:
            row[[7, V - 2]] = row.max() + 1.0  # equal maxima: the first wins
        b.write(row)
        t, p = gctx.argmax_prob(b.ptr, V)
        assert t == orc.argmax(row)
        assert p == np.float32(orc.softmax_prob(row, t, 1.0))
    b.free()


def test_generate_tiny_llama_q4_0(gctx, orc):
    """The reference's own CPU-runnable case on the device: a 4-layer Q4_0
    target (d 512, 8 x 64 heads, FFN 1408, vocab 32000, F32 embedding) with a
    1-layer draft of the same shape, a 128-token prompt, 4 draft tokens a
    round, greedy: the oracle's tokens and statistics exactly."""
    cfg = P.model_cfg(4, 512, 8, 8, 64, 1408, 32000, rope_theta=10000.0)
    dts = dict(tok_embd=P.F32, output=P.Q4_0, q=P.Q4_0, k=P.Q4_0, v=P.Q4_0, o=P.Q4_0,
               gate=P.Q4_0, up=P.Q4_0, down=P.Q4_0)
    target = P.make_model(orc, cfg, dts, seed=41)
    target["out_norm"]["raw"] = np.full(512, 30.0, np.float32).view(np.uint8).copy()
    draft = P.make_model(orc, dict(cfg, n_layer=1), dts, seed=42)
    # the draft shares the target's embedding and (peaked) head, so its
    # tokens pass the draft cut and are sometimes accepted
    for nm in ("tok_embd", "output", "out_norm"):
        draft[nm] = target[nm]
    tm, dm = upload(gctx, target), upload(gctx, draft)
    cap = 256
    tkv, dkv = tm.kv(cap), dm.kv(cap)
    drafter = spec.DraftModelDrafter(gctx, dm, dkv)
    prompt = [int(t) for t in np.random.default_rng(43).integers(0, 32000, 128)]
    try:
        got, st = spec.generate(gctx, tm, tkv, drafter, prompt, 24, spec_k=4, temp=0.0)
    finally:
        drafter.free()
    want, sto = orc.generate(target, draft, prompt, 24, spec_k=4, temp=0.0, cap=cap)
    assert got == want, (st, sto, got, want)
    assert st == sto and st["drafted"] > 0
    for x in (tkv, dkv, tm, dm):
        x.free()
