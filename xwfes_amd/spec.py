"""Speculative decoding on the device: the draft-model drafter and the
generate loop around the verify step.

DraftModelDrafter mirrors the reference's (src/spec.cpp:72-119): its own
resident model and KV cache, synced to the committed history by prefill,
k greedy draft tokens each with its T = 1 softmax probability (one device
step per token after the first), truncation to the accepted prefix on
commit.  generate mirrors generate's speculative block (src/spec.cpp:245-333):
draft, the probability cut heuristic, one verify step of the draft on the
target, acceptance (the ratio test with the draft probabilities), the bonus
token, truncation of the target cache, one target step on the bonus token.
The bonus is drawn from the row after the last accepted token (the reference
uses rows[min(acc, k - 1)], the next token's row only when every draft token
is accepted) by the reference's Sampler (temperature, top-k, top-p, its
state carried over); temp <= 0 takes the argmax, as Sampler::sample does.
The acceptance test takes the target at T = 1 whatever temp is, as
accept_chain_sampling does (src/spec.cpp:216).  An end-of-sequence token
(the GGUF's tokenizer.ggml.eos_token_id) ends the loop as the reference's
does (src/spec.cpp:316-328).
"""
import numpy as np

from . import ftx

# generate's cut heuristic (src/spec.cpp:276-285)
# the reference compares against the float constants 0.02f and 0.05f
# (src/spec.cpp:279-281): their exact values as doubles
CUT_MIN_PROB = float(np.float32(0.02))
CUT_MIN_CUM = float(np.float32(0.05))


class DraftModelDrafter:
    """A drafter over a resident draft model (ftx.Model) and its cache."""

    def __init__(self, ctx, model, kv):
        self.ctx, self.model, self.kv = ctx, model, kv
        self.V = model.cfg["vocab"]
        self.logits = ctx.buffer(8 * self.V * 4)  # the last prefill chain's rows
        self.row = 0            # row of self.logits holding the current logits
        self.pending_base = 0
        self.synced = 0

    def npast(self):
        return self.kv.pointers()[2]

    def sync(self, history):
        """src/spec.cpp:77-85: reset when ahead of the history, prefill the
        tokens it lacks; the logits of the history's last token are then
        current."""
        if self.npast() > len(history):
            self.kv.truncate(0)
        have = self.npast()
        if have < len(history):
            n = self.model.prefill(self.kv, list(history[have:]), self.logits.ptr)
            self.row = n - 1
        self.synced = len(history)

    def draft(self, history, k):
        """k greedy draft tokens and each one's T = 1 probability
        (src/spec.cpp:97-112)."""
        self.sync(history)
        self.pending_base = len(history)
        props, probs = [], []
        for j in range(k):
            t, p = self.ctx.argmax_prob(self.logits.ptr + self.row * self.V * 4, self.V)
            props.append(t)
            probs.append(p)
            if j + 1 < k:
                self.model.step(self.kv, t, self.logits.ptr)
                self.row = 0
        return props, probs

    def on_commit(self, accepted):
        """src/spec.cpp:114-117; Engine::truncate_to clamps to the history it
        holds (src/engine.cpp:423-428), so after a fully accepted draft the
        cache keeps the k - 1 tokens it stepped and the next sync prefills
        the last draft token with the bonus."""
        self.kv.truncate(min(self.pending_base + accepted, self.npast()))
        self.synced = self.pending_base + accepted

    def free(self):
        self.logits.free()


def cut_draft(props, probs):
    """src/spec.cpp:276-285: stop at the first probability below 0.02, or
    after the token that takes the running product below 0.05."""
    cut = len(props)
    cum = 1.0
    for i, p in enumerate(probs):
        if 0 <= p < CUT_MIN_PROB:
            cut = i
            break
        cum *= p if p > 0 else 1.0
        if cum < CUT_MIN_CUM:
            cut = i + 1
            break
    return props[:cut], probs[:cut]


def generate(ctx, target, kv, drafter, prompt, max_new, spec_k=8, temp=0.0, top_k=40,
             top_p=0.95, seed=0, eos=-1):
    """Speculative generation after `prompt` (the target cache starts
    empty) until at least max_new tokens are out or eos (-1: none) ends it;
    a round's accepted tokens and bonus are emitted together, so the last
    round may go past max_new (as the reference's does).  eos: an accepted
    draft token equal to it ends the loop once every accepted token is out
    (no bonus), a bonus equal to it is emitted and stepped, the sampled
    token of an empty draft is emitted (src/spec.cpp:287-295, 316-328).
    Returns (tokens, stats)."""
    V = target.cfg["vocab"]
    kv.truncate(0)
    if not 1 <= spec_k <= 8:
        raise ValueError("spec_k must be in 1..8 (the verify step's fast width)")
    PREFILL_CHUNK = 8
    base = ctx.buffer(V * 4)      # the logits row of the last committed token
    # the draft's rows, and the prompt's last prefill chain (up to 8 rows)
    rows = ctx.buffer(max(spec_k, PREFILL_CHUNK) * V * 4)
    n = target.prefill(kv, list(prompt), rows.ptr, chunk=PREFILL_CHUNK)
    ctx.copy(base.ptr, rows.ptr + (n - 1) * V * 4, V * 4)
    history = list(prompt)
    out = []
    rsamp = seed if seed else 88172645463325252  # src/spec.cpp:259
    sstate = seed if seed else ftx.SAMPLER_SEED
    # the ratio test at T = 1 (src/spec.cpp:216); temp <= 0: a top-1 bonus
    # (the argmax)
    acc_temp = 1.0
    bk, bp = (top_k, top_p) if temp > 0 else (1, 1.0)
    stats = dict(rounds=0, drafted=0, accepted=0, hit_eos=False)
    try:
        while len(out) < max_new:
            props, probs = drafter.draft(history, spec_k)
            props, probs = cut_draft(props, probs)
            np_before = kv.pointers()[2]
            M = len(props)
            if M:
                target.verify(kv, props, rows.ptr)
            r = ctx.accept(base.ptr, rows.ptr if M else None, M, V, props, ftx.ACCEPT_RATIO,
                           temp=acc_temp, rng=rsamp, pd=np.asarray(probs, np.float32),
                           sampler_state=sstate, top_k=bk, top_p=bp)
            rsamp, sstate = r["rng"], r["sampler_state"]
            acc = len(r["accepted"])
            bonus = r["bonus"]
            kv.truncate(np_before + acc)
            stats["rounds"] += 1
            stats["drafted"] += M
            stats["accepted"] += acc
            if M == 0 and bonus == eos:  # an empty draft's sampled token
                out.append(bonus)
                stats["hit_eos"] = True
                break
            # a round is emitted whole (src/spec.cpp:314-322)
            out += list(props[:acc])
            history += list(props[:acc])
            if eos >= 0 and eos in props[:acc]:
                drafter.on_commit(acc)
                stats["hit_eos"] = True
                break
            out.append(bonus)
            history.append(bonus)
            # one target step on the bonus token: the next round's base row
            target.step(kv, bonus, base.ptr)
            drafter.on_commit(acc)
            if bonus == eos:
                stats["hit_eos"] = True
                break
    finally:
        base.free()
        rows.free()
    return out, stats
