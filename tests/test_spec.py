"""Speculative generation (generate with a DraftModelDrafter, src/spec.cpp:
72-119, 245-333) in the oracle, pinned against the reference's own generate
loading the same GGUF files (oracle/_ref), on the CPU: identical emitted
tokens with the draft equal to the target (every draft accepted) and with a
different draft (rejections: the oracle then takes the bonus from the
reference's row, rows[min(acc, k - 1)], with ref_bonus_row), at temperature 0
(argmax bonus), 0.7 (the reference's default) and 1 -- the ratio test at T = 1
in both, the temperature shaping the bonus only -- with the reference's
sampler defaults, and with an end-of-sequence id in the target file that the
run reaches (the loops stop alike).

The reference's CPU matmul sums the M rows of a block into the first output
row (src/cpu_backend.cpp:95-103), so its forwards are right only at M = 1:
the comparison runs both of its engines with prefill in chains of one token
and one draft token per round, which keeps every reference forward at M = 1
while the draft / cut / verify / accept / bonus / truncate / step / commit
sequence runs as in any round.  Its Engine::prefill also forwards the
engine's whole history again before new tokens when no prefix snapshot
matches (src/engine.cpp:614-621), which its drafter's sync does every round:
the oracle reproduces that drafter behaviour with ref_draft_prefill for this
comparison only.  Rounds of more draft tokens are covered by the oracle's own
invariants (tests of verify, acceptance and the drafter) and on the GPU
against this oracle."""
import numpy as np
import pytest

import pyoracle as P
from xwfes_amd import gguf as G

CFG = P.model_cfg(2, 64, 4, 2, 16, 96, 48, rope_theta=10000.0)
DT = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q8_0, k=P.Q8_0, v=P.Q8_0, o=P.Q8_0,
          gate=P.Q8_0, up=P.Q8_0, down=P.Q8_0)


def peaked(orc, seed, gain=30.0):
    """A random model whose logits are scaled by `gain` (the output norm),
    so that draft probabilities pass the 0.02 / 0.05 cut."""
    m = P.make_model(orc, CFG, DT, seed=seed)
    m["out_norm"]["raw"] = np.full(CFG["n_embd"], gain, np.float32).view(np.uint8).copy()
    return m


def write(tmp_path, name, model, eos=None):
    p = str(tmp_path / name)
    G.write_gguf(p, G.model_kv(CFG, eos=eos), G.model_tensor_list(model))
    return p


@pytest.mark.parametrize("eos_at", [None, 4, 9])
@pytest.mark.parametrize("temp", [0.0, 0.7, 1.0])
@pytest.mark.parametrize("same_draft", [True, False])
def test_oracle_generate_equals_reference(orc, ref, tmp_path, temp, same_draft, eos_at):
    """eos_at: the target file's tokenizer.ggml.eos_token_id is the token
    the run without one emits at that position (the reference reads it from
    the file, src/tokenizer.cpp:68); both loops stop as the reference's does
    (src/spec.cpp:316-328)."""
    target = peaked(orc, 31)
    draft = target if same_draft else peaked(orc, 32, gain=25.0)
    prompt = [3, 17, 5, 40, 11]
    kw = dict(spec_k=1, temp=temp, seed=0, cap=2304, kv_dtype=np.float32, ref_bonus_row=True,
              ref_draft_prefill=True)
    eos = -1
    if eos_at is not None:
        eos = orc.generate(target, draft, prompt, 24, **kw)[0][eos_at]
    tp = write(tmp_path, "t.gguf", target, eos=eos if eos >= 0 else None)
    dp = tp if same_draft else write(tmp_path, "d.gguf", draft)
    # seed 0: a non-zero seed makes the reference's Sampler restart from it
    # on every draw (include/ft/sampler.h:31), which the oracle does not copy
    want = ref.generate(tp, dp, prompt, max_new=24, spec_k=1, temp=temp, seed=0, ctx_len=2048,
                        prefill_batch=1)
    got, st = orc.generate(target, draft, prompt, 24, eos=eos, **kw)
    assert got == want, (st, got, want)
    if eos_at is not None:
        assert st["hit_eos"] and eos in got
        assert len(got) <= eos_at + 2
        return
    # drafts were verified; with the draft equal to the target some were
    # accepted (its duplicated context makes others wrong)
    assert st["drafted"] > 0 and st["accepted"] < st["drafted"]
    assert st["accepted"] > 0 or not same_draft
    assert len(got) >= 24


def test_cut_draft_float_thresholds():
    """The cut compares with the float constants 0.02f and 0.05f
    (src/spec.cpp:279-281): a probability equal to 0.02f is kept, one just
    below it cuts; a running product in [0.05, 0.05f) is above the reference's
    threshold 0.05f only when it is not below it."""
    from xwfes_amd.spec import cut_draft
    f02 = float(np.float32(0.02))
    below = float(np.nextafter(np.float32(0.02), np.float32(0)))
    # (a kept token is the last one: the running product then falls below 0.05f)
    assert cut_draft([1, 2], [f02, 0.9])[0] == [1]
    assert cut_draft([1, 2], [below, 0.9])[0] == []
    assert cut_draft([1, 2, 3], [0.9, below, 0.9])[0] == [1]
    # 0.05f is slightly above 0.05: a product equal to 0.05 is below it
    assert float(np.float32(0.05)) > 0.05
    assert cut_draft([1, 2, 3], [0.5, 0.1, 0.9])[0] == [1, 2]
    # the oracle applies the same constants
    assert (P.CUT_MIN_PROB, P.CUT_MIN_CUM) == (f02, float(np.float32(0.05)))
