#!/usr/bin/env python3
"""Verify-step benchmark on one MI355X.

A step is one speculative-decoding verification of an 8-token linear draft
against a Llama-3-8B-shaped random-init Q4_K_M model at context 2048: the
device-resident forward of the 8 draft tokens (ftx_verify_step) followed by
stochastic acceptance at T = 0.8 with the reference's ratio test and seeded
SplitMix64 uniforms plus the bonus token (ftx_accept).  Inputs (weights, KV
context, draft) are resident in HBM before the timed region.

Prints one JSON line.  `value` = verified tokens per second (M / t_step).
"""
import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16 MFMA (no sparsity)
REPLAY = 20  # back-to-back issues of each dominant-class launch when timing it
LLAMA3_8B = dict(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=14336,
                vocab=128256, rope_theta=500000.0, rope_neox=0, rms_eps=1e-5)
TINY_LLAMA = dict(n_layer=4, n_embd=512, n_head=8, n_head_kv=8, head_dim=64, n_ff=1408,
                  vocab=32000, rope_theta=10000.0, rope_neox=0, rms_eps=1e-5)
LLAMA32_1B = dict(n_layer=16, n_embd=2048, n_head=32, n_head_kv=8, head_dim=64, n_ff=8192,
                  vocab=128256, rope_theta=500000.0, rope_neox=0, rms_eps=1e-5)
MIXTRAL_8X7B = dict(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=14336,
                    vocab=32000, rope_theta=1e6, rope_neox=0, rms_eps=1e-5, n_expert=8,
                    n_expert_used=2)
LLAMA3_70B = dict(n_layer=80, n_embd=8192, n_head=64, n_head_kv=8, head_dim=128, n_ff=28672,
                  vocab=128256, rope_theta=500000.0, rope_neox=0, rms_eps=1e-5)
WORKLOADS = {
    # kind verify: one verify step (M draft tokens at context ctx) plus ratio
    # acceptance; decode: one Engine::step at context ctx; prefill: P prompt
    # tokens from an empty cache in advancing chains of M
    "llama3-8b-q4km-k8-ctx2048": dict(kind="verify", cfg=LLAMA3_8B, mix="q4_k_m", ctx=2048, M=8,
                                      temp=0.8),
    "llama3-8b-q4km-decode-ctx2048": dict(kind="decode", cfg=LLAMA3_8B, mix="q4_k_m", ctx=2048,
                                          M=1, temp=0.8),
    "llama3-8b-q4km-prefill-512": dict(kind="prefill", cfg=LLAMA3_8B, mix="q4_k_m", ctx=0, M=8,
                                       P=512, temp=0.8),
    # generate: N tokens after a P-token prompt, a draft model proposing M
    # tokens a round (greedy); random weights, so the draft is rarely accepted
    "llama3-8b-q4km+1b-draft-spec4": dict(kind="generate", cfg=LLAMA3_8B, draft_cfg=LLAMA32_1B,
                                          mix="q4_k_m", ctx=0, M=4, P=8, N=32, temp=0.0),
    # the reference's own CPU-runnable case: a 4-layer Q4_0 target (d 512,
    # 8 x 64 heads, FFN 1408, vocab 32000, F32 embedding) and a 1-layer draft
    # of the same shape, a 128-token prompt, 4 draft tokens a round, greedy
    "tinyllama-q4_0+1l-draft-spec4": dict(kind="generate", cfg=TINY_LLAMA,
                                          draft_cfg=dict(TINY_LLAMA, n_layer=1), mix="q4_0",
                                          ctx=0, M=4, P=128, N=32, temp=0.0),
    # tree: a 52-node draft tree (branching 4, 4, 2 from the root) at context
    # 4096, ancestor-only attention, residual (SpecInfer) acceptance at T 0.8
    # with Dirichlet(1) draft distributions; Q8_0 attention projections and a
    # Q4_K FFN
    "llama3-8b-q8attn-tree52-ctx4096": dict(kind="tree", cfg=LLAMA3_8B, mix="q8_0_attn", ctx=4096,
                                            M=52, branching=(4, 4, 2), temp=0.8),
    # the same tree pruned to its first 32 nodes in breadth-first order (4 +
    # 16 + the children of the first 6 second-level nodes): the 32-node draft
    # tree of branching (4, 4, 2)
    "llama3-8b-q8attn-tree32-ctx4096": dict(kind="tree", cfg=LLAMA3_8B, mix="q8_0_attn", ctx=4096,
                                            M=32, branching=(4, 4, 2), temp=0.8),
    # batch: `seqs` sequences verified in one step (ftx_verify_batch), each
    # against its own cache at context ctx, then accepted one by one.
    # Mixtral-8x7B-shaped Q4_0 MoE (8 experts top-2, all resident), 8-token
    # linear drafts for 4 sequences at context 1024, ratio acceptance at T 0.8
    "mixtral-8x7b-q4_0-k8x4-ctx1024": dict(kind="batch", cfg=MIXTRAL_8X7B, mix="q4_0_moe",
                                           ctx=1024, M=8, seqs=4, tree=None, temp=0.8),
    # Llama-3-70B-shaped Q4_K, a 64-node draft tree (depth <= 6, branching
    # <= 4) for each of 4 sequences at context 8192, residual acceptance
    "llama3-70b-q4k-tree64x4-ctx8192": dict(kind="batch", cfg=LLAMA3_70B, mix="q4_k", ctx=8192,
                                            M=64, seqs=4, tree=(6, 4), temp=0.8),
}
# the arithmetic the step's projections compute in (weights enter the
# MFMAs as their exact quantised integers; block scales on the accumulators)
DTYPES = {"q4_k_m": "q4_k/q6_k weights x int8x2-limb activations (MFMA i8), int32/fp32 accumulate; "
                    "f16 KV",
          "q4_0": "q4_0 weights (f32 embedding) x fp32 activations, fp32 accumulate; f16 KV",
          "q8_0_attn": "q8_0 / q4_k / q6_k weights x fp16 hi+lo activations (MFMA f16), fp32 "
                       "accumulate; f16 KV",
          "q4_0_moe": "q4_0 weights x fp16 hi+lo activations (MFMA f16), fp32 accumulate; f16 KV",
          "q4_k": "q4_k weights x fp16 hi+lo activations (MFMA f16), fp32 accumulate; f16 KV"}


def mix_of(name, cfg):
    from xwfes_amd import synth
    return {"q4_k_m": lambda: synth.q4_k_m_mix(cfg),
            "q4_0": lambda: synth.uniform_mix(synth.Q4_0, embd=synth.F32),
            "q8_0_attn": lambda: synth.q8_attn_mix(cfg),
            "q4_0_moe": lambda: synth.uniform_mix(synth.Q4_0),
            "q4_k": lambda: synth.uniform_mix(synth.Q4_K)}[name]()


def draft_tree(V, branching, seed, nodes=None):
    """A full draft tree (nodes in breadth-first order, parents[i] < i): each
    node's children are drawn from one Dirichlet(1) distribution over the
    vocab, which is every child's q row.  nodes: keep the first `nodes`
    nodes (a pruned tree: every kept node's parent is kept)."""
    rng = np.random.default_rng(seed)
    parents, props, q = [], [], []
    level = [-1]
    for b in branching:
        nxt = []
        for par in level:
            e = -np.log(rng.random(V))
            dist = (e / e.sum()).astype(np.float32)
            cdf = np.cumsum(dist.astype(np.float64))
            for _ in range(b):
                parents.append(par)
                props.append(min(int(np.searchsorted(cdf, rng.random() * cdf[-1])), V - 1))
                q.append(dist)
                nxt.append(len(parents) - 1)
        level = nxt
    n = len(parents) if nodes is None else nodes
    return (np.array(parents[:n], np.int32), np.array(props[:n], np.int32),
            np.ascontiguousarray(np.stack(q[:n])))


def random_tree(V, n, max_depth, max_branch, seed):
    """An n-node draft tree in breadth-first order: each node of a level
    below max_depth gets 1 .. max_branch children until n nodes; a node's
    children share one Dirichlet(1) draft distribution (their q rows) and are
    drawn from it.  A draw that stays below n nodes is redrawn from the next
    seed."""
    for attempt in range(100):
        t = _random_tree(V, n, max_depth, max_branch, seed + 1000 * attempt)
        if t is not None:
            return t
    raise ValueError("no %d-node tree of depth <= %d" % (n, max_depth))


def _random_tree(V, n, max_depth, max_branch, seed):
    rng = np.random.default_rng(seed)
    shape = []
    level, depth, count = [-1], 0, 0
    while count < n and depth < max_depth:
        nxt = []
        for par in level:
            for _ in range(int(rng.integers(1, max_branch + 1))):
                if count == n:
                    break
                shape.append(par)
                nxt.append(count)
                count += 1
        level, depth = nxt, depth + 1
    if count < n:
        return None
    parents, props, q = [], [], []
    level, depth = [-1], 0
    rng = np.random.default_rng(seed + 1)
    kids = {}
    for i, par in enumerate(shape):
        kids.setdefault(par, []).append(i)
    while len(parents) < n and depth < max_depth:
        nxt = []
        for par in level:
            if par not in kids:
                continue
            e = -np.log(rng.random(V))
            dist = (e / e.sum()).astype(np.float32)
            cdf = np.cumsum(dist.astype(np.float64))
            for _ in kids[par]:
                parents.append(par)
                props.append(min(int(np.searchsorted(cdf, rng.random() * cdf[-1])), V - 1))
                q.append(dist)
                nxt.append(len(parents) - 1)
        level, depth = nxt, depth + 1
    return (np.array(parents, np.int32), np.array(props, np.int32),
            np.ascontiguousarray(np.stack(q)))


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def draft(V, M, seed):
    """q_a ~ Dirichlet(1) over the vocab (normalised -log u); props[a] drawn
    from q_a by inverse CDF; pd[a] = q_a(props[a])."""
    rng = np.random.default_rng(seed)
    props = np.zeros(M, np.int32)
    pd = np.zeros(M, np.float32)
    for a in range(M):
        e = -np.log(rng.random(V))
        q = e / e.sum()
        props[a] = min(int(np.searchsorted(np.cumsum(q), rng.random())), V - 1)
        pd[a] = np.float32(q[props[a]])
    return props, pd


def step_bytes(tensors, cfg, ctx_len, M):
    """Algorithmic HBM bytes of one verify step: every weight tensor at its
    stored size (the LM head counted once), the KV read 2*L*(ctx+M)*kvdim*2 B,
    M embedding rows and the M*V*4 B logits write."""
    L, d, V = cfg["n_layer"], cfg["n_embd"], cfg["vocab"]
    kdim = cfg["n_head_kv"] * cfg["head_dim"]
    w = sum(t.nbytes for n, t in tensors.items() if n != "tok_embd")
    emb = M * tensors["tok_embd"].nbytes // V
    kv = 2 * L * (ctx_len + M) * kdim * 2
    logits = M * V * 4
    return w + emb + kv + logits


def prefill_bytes(tensors, cfg, P, chunk):
    """Algorithmic HBM bytes of a P-token prefill in chains of `chunk`: each
    chain a verify step at its context, the LM head and its logits only on
    the last chain."""
    head = tensors["output"].nbytes if "output" in tensors else tensors["tok_embd"].nbytes
    total, n = 0, 0
    for s0 in range(0, P, chunk):
        m = min(chunk, P - s0)
        total += step_bytes(tensors, cfg, s0, m)
        n += 1
        if s0 + chunk < P:
            total -= head + m * cfg["vocab"] * 4
    return total


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo, as lscpu shows it)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    """Threads for the CPU baseline: the process's CPU share (OMP_NUM_THREADS
    where the host sets it, else the CPUs this process may run on)."""
    n = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return n if n > 0 else len(os.sched_getaffinity(0))


def host_model(ctx, tensors, cfg, n_layer):
    """Host copies of tok_embd, out_norm, output and layer 0's tensors (any
    roles, dense or MoE), with every one of n_layer layers taking layer 0's
    tensors: the oracle's model dict of a bounded sample of the step."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))

    def host(t):
        raw = np.empty(t.nbytes, np.uint8)
        ctx.copy(raw.ctypes.data, t.ptr, t.nbytes)
        return dict(raw=raw, dtype=t.dtype, ne0=t.ne[0], ne1=int(np.prod(t.ne[1:])))

    base = {k: host(tensors[k]) for k in ("tok_embd", "output", "out_norm") if k in tensors}
    layer0 = {n[len("blk.0."):]: host(t) for n, t in tensors.items() if n.startswith("blk.0.")}
    model = dict(base)
    model["cfg"] = dict(cfg, n_layer=n_layer)
    for l in range(n_layer):
        for nm, t in layer0.items():
            model["blk.%d.%s" % (l, nm)] = t
    return model


def cpu_baseline(ctx, tensors, cfg, ctx_len, M, props, threads, layers=(1, 2), parents=None):
    """The oracle's reference loop nest (CpuBackend::matmul, matmul_down_axpy,
    Impl::attn, moe_ffn) timed on this host on a bounded sample: 1-layer and
    2-layer forwards of the same weights (layer 0, tok_embd, output) at the
    same tokens (a tree through its parent array) and context, one
    sequence; the caller extrapolates to all layers (and sequences)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as P
    orc = P.Oracle()
    orc.set_threads(threads)
    kdim = cfg["n_head_kv"] * cfg["head_dim"]
    rng = np.random.default_rng(4)
    times = {}
    for nl in layers:
        model = host_model(ctx, tensors, cfg, nl)
        cap = ctx_len + M
        k = rng.standard_normal((nl, cap, kdim)).astype(np.float16)
        v = rng.standard_normal((nl, cap, kdim)).astype(np.float16)
        orc.forward(model, k, v, ctx_len, props[:1])  # warm caches and threads
        t0 = time.perf_counter()
        orc.forward(model, k, v, ctx_len, props, parents=parents)
        times[nl] = time.perf_counter() - t0
        del model
    return times


def cpu_summary(times, cfg, M, ctx_len, threads, nseq=1):
    t_layer = max(times[2] - times[1], 0.0)
    t_step = (times[1] + (cfg["n_layer"] - 1) * t_layer) * nseq
    return t_step, t_layer, ("oracle forward of M=%d tokens at ctx %d over 1 and 2 layers of the "
                             "same weights (%.2f s, %.2f s) on %d threads, extrapolated to %d "
                             "layers%s: %.3f s/step" % (
                                 M, ctx_len, times[1], times[2], threads, cfg["n_layer"],
                                 (" and x %d sequences (one Engine each, run one after another)"
                                  % nseq) if nseq > 1 else "", t_step))


def cpu_generate_baseline(ctx, tensors, dtensors, cfg, dcfg, prompt, N, M, threads):
    """The oracle's generate (src/spec.cpp:245-333 with a DraftModelDrafter)
    over host copies of the same target and draft models, run whole on this
    host: generated tokens per second."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as P
    orc = P.Oracle()
    orc.set_threads(threads)

    def full(ts, c):
        m = {}
        for n, t in ts.items():
            raw = np.empty(t.nbytes, np.uint8)
            ctx.copy(raw.ctypes.data, t.ptr, t.nbytes)
            m[n] = dict(raw=raw, dtype=t.dtype, ne0=t.ne[0], ne1=int(np.prod(t.ne[1:])))
        m["cfg"] = dict(c)
        return m

    target, draft = full(tensors, cfg), full(dtensors, dcfg)
    cap = len(prompt) + N + 32
    t0 = time.perf_counter()
    out, st = orc.generate(target, draft, prompt, N, spec_k=M, temp=0.0, cap=cap)
    dt = time.perf_counter() - t0
    return len(out) / dt, ("oracle generate of %d tokens after a %d-token prompt, %d draft tokens "
                           "a round, greedy, whole run %.2f s on %d threads (%d rounds)" % (
                               len(out), len(prompt), M, dt, threads, st["rounds"]))


def class_flops(kernel_class, cfg, tokens):
    """Algorithmic flops of one launch of a GEMM kernel class (one layer's
    projection, or the LM head) over `tokens` tokens: 2 x tokens x the
    weight elements it contracts; None for other classes."""
    d, F, V = cfg["n_embd"], cfg["n_ff"], cfg["vocab"]
    qd, kd = cfg["n_head"] * cfg["head_dim"], cfg["n_head_kv"] * cfg["head_dim"]
    w = {"gemv_qkv": (qd + 2 * kd) * d, "gemv_o": d * qd, "gemv_swiglu": 2 * F * d,
         "down": F * d, "head": V * d}.get(kernel_class)
    return None if w is None else 2.0 * tokens * w


def step_flops(cfg, M, nseq, ctx_len):
    """Algorithmic flops of a verify step: 2 x tokens x every weight element
    the step contracts (the projections of every layer and the LM head; the
    embedding is a lookup) plus attention's 4 x rows x head_dim x slots per
    head and sequence."""
    d, F, V, L = cfg["n_embd"], cfg["n_ff"], cfg["vocab"], cfg["n_layer"]
    qd, kd = cfg["n_head"] * cfg["head_dim"], cfg["n_head_kv"] * cfg["head_dim"]
    ffn = 3 * F * d * (cfg.get("n_expert_used", 0) or 1)
    w = L * ((qd + 2 * kd) * d + d * qd + ffn) + V * d
    attn = 4.0 * M * cfg["n_head"] * cfg["head_dim"] * (ctx_len + M) * L
    return 2.0 * M * nseq * w + attn * nseq


def measured_traffic(workload, kernel_class):
    """HBM bytes per launch of `kernel_class` as measured by the FETCH_SIZE /
    WRITE_SIZE counter passes recorded in profiles/traffic_<workload>.json
    (copy-calibrated; the commands are in the file), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_%s.json" % workload)
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    c = t.get("classes", {}).get(kernel_class)
    return c.get("bytes_per_launch") if c else None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="llama3-8b-q4km-k8-ctx2048", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--trace-steps", type=int, default=10)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="before the timed steps, copy MIB MiB device-to-device three times "
                         "(a copy of known size for scaling hardware byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the verify step runs on a single MI355X and this "
              "build has no multi-GPU path (asked for --gpus %d)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    from xwfes_amd import ftx, spec, synth
    W = WORKLOADS[args.workload]
    cfg, ctx_len, M, temp = W["cfg"], W["ctx"], W["M"], W["temp"]
    V = cfg["vocab"]
    ctx = ftx.Context(0)
    if args.copy_calibration > 0:
        nb = args.copy_calibration << 20
        src, dst = ctx.buffer(nb), ctx.buffer(nb)
        ctx.fill_normal(src.ptr, nb // 4, seed=9, std=1.0)
        for _ in range(3):
            ctx.copy(dst.ptr, src.ptr, nb)
        log("copy calibration: 3 device copies of %d bytes" % nb)
        src.free()
        dst.free()
    t0 = time.perf_counter()
    tensors = synth.build(ctx, cfg, mix_of(W["mix"], cfg), seed=1)
    log("model built in %.1f s (%.3f GB of weights)" % (time.perf_counter() - t0,
                                                        synth.weight_bytes(tensors) / 1e9))
    kind = W["kind"]
    P_tok = W.get("P", 0)
    nseq = W.get("seqs", 1)
    model = ctx.model(cfg, tensors, max_tokens=max(M * nseq, 8))
    kv = model.kv(max(ctx_len, P_tok + W.get("N", 0) + 16) + M + 8)
    # batch: one cache, logits, base row and draft per sequence
    bkv, blog, bbase, bdraft = [], [], [], []
    if kind == "batch":
        bkv = [kv] + [model.kv(ctx_len + M + 8) for _ in range(nseq - 1)]
    drafter = dtensors = dmodel = dkv = None
    gen_stats = []
    if kind == "generate":
        dcfg = W["draft_cfg"]
        dtensors = synth.build(ctx, dcfg, mix_of(W["mix"], dcfg), seed=2)
        dmodel = ctx.model(dcfg, dtensors, max_tokens=8)
        dkv = dmodel.kv(P_tok + W["N"] + 32)
        drafter = spec.DraftModelDrafter(ctx, dmodel, dkv)
        log("draft model built (%.3f GB of weights)" % (synth.weight_bytes(dtensors) / 1e9))
    for i, c in enumerate(bkv or [kv]):
        kp, vp, _ = c.pointers()
        n_kv = cfg["n_layer"] * c.cap_alloc * cfg["n_head_kv"] * cfg["head_dim"]
        ctx.fill_normal(kp, n_kv, seed=4 + 2 * i, std=1.0, dtype=ftx.F16)
        ctx.fill_normal(vp, n_kv, seed=5 + 2 * i, std=1.0, dtype=ftx.F16)
    logits = ctx.buffer(M * V * 4)
    base = ctx.buffer(V * 4)
    if kind in ("verify", "tree"):
        # the base row: logits of the last committed token (position ctx - 1)
        kv.truncate(ctx_len - 1)
        model.verify(kv, [int(np.random.default_rng(3).integers(V))], base.ptr, advance=True)
        ctx.sync()
    props, pd = draft(V, M, seed=6)
    parents = qbuf = None
    if kind == "tree":
        parents, props, qrows = draft_tree(V, W["branching"], seed=6, nodes=M)
        assert len(props) == M
        qbuf = ctx.buffer(qrows.nbytes)
        qbuf.write(qrows)
        del qrows
    if kind == "batch":
        for i in range(nseq):
            blog.append(ctx.buffer(M * V * 4))
            bbase.append(ctx.buffer(V * 4))
            if W["tree"]:
                par, pr, qrows = random_tree(V, M, W["tree"][0], W["tree"][1], seed=60 + i)
                qb = ctx.buffer(qrows.nbytes)
                qb.write(qrows)
                del qrows
                bdraft.append(dict(parents=par, props=pr, q=qb, pd=None))
            else:
                pr, pdv = draft(V, M, seed=60 + i)
                bdraft.append(dict(parents=None, props=pr, q=None, pd=pdv))
        # base rows: the logits of each sequence's last committed token
        for c in bkv:
            c.truncate(ctx_len - 1)
        first = np.random.default_rng(3).integers(V, size=nseq)
        model.verify_batch([(c, [int(t)], b.ptr, None, True)
                            for c, t, b in zip(bkv, first, bbase)])
        ctx.sync()
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, V, P_tok)]
    rng_state = [5, ftx.SAMPLER_SEED]
    seq_rng = [[5 + i, ftx.SAMPLER_SEED] for i in range(max(nseq, 1))]
    accepted = []

    def step():
        if kind == "verify":
            kv.truncate(ctx_len)
            model.verify(kv, props, logits.ptr)
            r = ctx.accept(base.ptr, logits.ptr, M, V, props, ftx.ACCEPT_RATIO, temp=temp,
                           rng=rng_state[0], pd=pd, sampler_state=rng_state[1])
            rng_state[0], rng_state[1] = r["rng"], r["sampler_state"]
            accepted.append(len(r["accepted"]))
        elif kind == "tree":
            kv.truncate(ctx_len)
            model.verify(kv, props, logits.ptr, parents=parents)
            r = ctx.accept(base.ptr, logits.ptr, M, V, props, ftx.ACCEPT_RESIDUAL, temp=temp,
                           rng=rng_state[0], parents=parents, q_ptr=qbuf.ptr)
            rng_state[0] = r["rng"]
            accepted.append(len(r["accepted"]))
        elif kind == "batch":
            for c in bkv:
                c.truncate(ctx_len)
            model.verify_batch([(c, dr["props"], lg.ptr, dr["parents"], False)
                                for c, dr, lg in zip(bkv, bdraft, blog)])
            # every sequence's acceptance (its own streams, as one engine per
            # sequence has) in one call
            items = []
            for i, (dr, lg, bs) in enumerate(zip(bdraft, blog, bbase)):
                it = dict(base_ptr=bs.ptr, rows_ptr=lg.ptr, M=M, V=V, props=dr["props"], temp=temp,
                          rng=seq_rng[i][0], sampler_state=seq_rng[i][1])
                if dr["q"] is not None:
                    it.update(mode=ftx.ACCEPT_RESIDUAL, parents=dr["parents"], q_ptr=dr["q"].ptr)
                else:
                    it.update(mode=ftx.ACCEPT_RATIO, pd=dr["pd"])
                items.append(it)
            for i, r in enumerate(ctx.accept_batch(items)):
                seq_rng[i] = [r["rng"], r["sampler_state"]]
                accepted.append(len(r["accepted"]))
        elif kind == "decode":
            kv.truncate(ctx_len)
            model.step(kv, int(props[0]), logits.ptr)
            # the token's logits are complete when the step returns, as the
            # caller samples from them before the next step
            ctx.sync()
        elif kind == "generate":
            out, st = spec.generate(ctx, model, kv, drafter, prompt, W["N"], spec_k=M, temp=temp)
            gen_stats.append((len(out), st))
        else:
            kv.truncate(0)
            model.prefill(kv, prompt, logits.ptr, chunk=M)
            ctx.sync()

    for _ in range(args.warmup):
        step()
    ctx.sync()
    accepted.clear()
    gen_stats.clear()
    per = []
    ctx.sync()
    t_start = time.perf_counter()
    for _ in range(args.steps):
        ts = time.perf_counter()
        step()
        per.append(time.perf_counter() - ts)
    ctx.sync()
    elapsed = time.perf_counter() - t_start
    ms_step = elapsed / args.steps * 1e3
    med_ms = statistics.median(per) * 1e3
    log("timed %d steps: mean %.3f ms, median %.3f ms" % (args.steps, ms_step, med_ms))

    # per-kernel-class device time from HIP events on the launch stream
    args.trace_steps = max(args.trace_steps, 1)
    ctx.trace(True)
    for _ in range(args.trace_steps):
        step()
    tr = ctx.trace_read()
    ctx.trace(False)
    pair = tr.pop("event_pair", None)
    pair_ms = pair["ms"] / pair["launches"] if pair else 0.0
    traced_ms = sum(e["ms"] for e in tr.values()) / max(args.trace_steps, 1)
    dom_name, dom = max(tr.items(), key=lambda kv_: kv_[1]["ms"])
    per_launch_b = dom["bytes"] / dom["launches"]
    # the dominant class's launch time inside the step (the steps' own
    # order and cache state): its main kernel timed by HIP events carried on
    # the kernel's own dispatch, start to end of the kernel -- the figure
    # rocprofv3's kernel trace gives (a split-sum kernel that follows it is
    # not part of it)
    bracket_ms = dom["ms"] / dom["launches"]
    if dom.get("kernel_launches"):
        kern_ms = dom["kernel_ms"] / dom["kernel_launches"]
        per_launch_ms = kern_ms
    else:
        kern_ms = None
        per_launch_ms = bracket_ms - pair_ms
    achieved = per_launch_b / (per_launch_ms * 1e-3) / 1e9
    # for comparison: the same launches replayed back to back (their weights
    # then partly cache-resident), which spreads the events' overhead
    ctx.trace_replay(dom_name, REPLAY)
    ctx.trace(True)
    step()
    rep = ctx.trace_read()[dom_name]
    ctx.trace(False)
    ctx.trace_replay(dom_name, 1)
    replay_ms = rep["ms"] / rep["launches"]
    log("dominant class %s: %.2f us per launch (main kernel on its own dispatch; bracket %.2f us, "
        "empty bracket %.2f us), %.2f us replayed x%d" % (dom_name, per_launch_ms * 1e3,
                                                         bracket_ms * 1e3, pair_ms * 1e3,
                                                         replay_ms * 1e3, REPLAY))
    for name, e in sorted(tr.items(), key=lambda kv_: -kv_[1]["ms"]):
        log("  %-12s %5d launches %8.3f ms/step  %7.1f GB/s" % (
            name, e["launches"] // args.trace_steps, e["ms"] / args.trace_steps,
            e["bytes"] / (e["ms"] * 1e-3) / 1e9 if e["ms"] > 0 else 0.0))

    if kind == "prefill":
        sb = prefill_bytes(tensors, cfg, P_tok, M)
        tokens = P_tok
    elif kind == "generate":
        tokens = statistics.mean(n for n, _ in gen_stats)
        sb = 0
    elif kind == "batch":
        # the weights once, each sequence's KV, embedding rows and logits
        sb = step_bytes(tensors, cfg, ctx_len, M)
        sb += (nseq - 1) * (step_bytes(tensors, cfg, ctx_len, M) - synth.weight_bytes(
            {n: t for n, t in tensors.items() if n != "tok_embd"}))
        tokens = M * nseq
    else:
        sb = step_bytes(tensors, cfg, ctx_len, M)
        tokens = M
    gbs = sb / (ms_step * 1e-3) / 1e9
    metric = {"verify": "verify-step tokens/s + HBM GB/s (% of peak), 8B-shape Q4_K, K=8 draft, "
                        "1 GPU",
              "tree": "tree verify-step tokens/s + HBM GB/s (%% of peak), 8B-shape Q8_0 attention "
                      "/ Q4_K FFN, %d-node draft tree, ctx 4096, 1 GPU" % M,
              "decode": "decode tokens/s (Engine::step, M=1, ctx 2048), 8B-shape Q4_K, 1 GPU",
              "batch": "batched verify-step tokens/s + HBM GB/s (%% of peak), %s, %d sequences x "
                       "%s, ctx %d, 1 GPU" % (
                           args.workload.split("-")[0] + "-shape " + W["mix"], nseq,
                           ("%d-node draft trees" % M) if W.get("tree") else
                           ("%d-token drafts" % M), ctx_len),
              "prefill": "prefill tokens/s (512-token prompt, chains of 8), 8B-shape Q4_K, "
                         "1 GPU",
              "generate": "generated tokens/s (speculative: %s target, %s draft, %d draft "
                          "tokens a round, greedy), 1 GPU" % (
                              W["mix"] + " %d-layer d%d" % (cfg["n_layer"], cfg["n_embd"]),
                              "%d-layer d%d" % (W["draft_cfg"]["n_layer"],
                                                W["draft_cfg"]["n_embd"]) if "draft_cfg" in W
                              else "", M)}[kind]
    unit = {"verify": "verified tokens/s", "tree": "verified tokens/s",
            "batch": "verified tokens/s", "decode": "decoded tokens/s",
            "prefill": "prefilled tokens/s", "generate": "generated tokens/s"}[kind]
    out = {
        "metric": metric,
        "value": round(tokens / (ms_step * 1e-3), 2),
        "unit": unit,
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": round(med_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": DTYPES[W["mix"]],
        "data": "synthetic: random-init N(0,0.02) weights quantised on device, N(0,1) fp16 KV, "
                "Dirichlet(1) draft",
        "config": {"workload": args.workload, "kind": kind, "M": M, "ctx": ctx_len,
                   "prompt": P_tok, "layers": cfg["n_layer"], "d_model": cfg["n_embd"],
                   "vocab": V, "mix": W["mix"],
                   "accept": {"verify": "ratio", "tree": "residual",
                              "batch": "residual" if W.get("tree") else "ratio"}.get(kind),
                   "temperature": temp, "batch": nseq,
                   "experts": cfg.get("n_expert", 0), "experts_used": cfg.get("n_expert_used", 0)},
        "step_bytes": sb,
        "hbm_gbs": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "committed_tokens_per_s": (round((statistics.mean(accepted) + 1) / (ms_step * 1e-3), 2)
                                   if accepted else None),
        "generate_rounds": (statistics.mean(st["rounds"] for _, st in gen_stats)
                            if gen_stats else None),
        "draft_acceptance": (round(sum(st["accepted"] for _, st in gen_stats) /
                                   max(1, sum(st["drafted"] for _, st in gen_stats)), 4)
                             if gen_stats else None),
        "mean_accepted": round(statistics.mean(accepted), 3) if accepted else None,
        "traced_device_ms_per_step": round(traced_ms, 4),
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "bytes_per_launch": per_launch_b, "us_per_launch": round(per_launch_ms * 1e3, 2),
                     "source": "in-step HIP events on the main kernel's own dispatch",
                     "bracket_us": round(bracket_ms * 1e3, 2), "empty_bracket_us": round(pair_ms * 1e3, 2),
                     "replay_us_per_launch": round(replay_ms * 1e3, 2), "replays": REPLAY,
                     "traffic": measured_traffic(args.workload, dom_name)},
        "cpu_baseline": None,
    }
    if kind in ("verify", "tree", "batch"):
        sf = step_flops(cfg, M, nseq, ctx_len)
        out["step_tflops"] = round(sf / (ms_step * 1e-3) / 1e12, 2)
        out["step_mfma_frac"] = round(sf / (ms_step * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4)
    # the 70B batch of trees is MFMA-bound (256 tokens: ~910 flop per weight
    # byte against the fp16 ridge of 2.5 PF / 8 TB/s = 312): its roofline is
    # the dominant GEMM's algorithmic flops per launch over its in-step
    # launch time against the dense fp16 MFMA peak (the one-pass GEMMs run
    # v_mfma_f32_16x16x32_f16)
    cf = class_flops(dom_name, cfg, tokens)
    if kind == "batch" and W.get("tree") and cf:
        tf = cf / (per_launch_ms * 1e-3) / 1e12
        hbm = out["roofline"]
        out["roofline"] = {"bound": "mfma", "kernel": dom_name, "achieved": round(tf, 1),
                           "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": round(tf / MFMA_PEAK_TFLOPS, 4), "flops_per_launch": cf,
                           "us_per_launch": hbm["us_per_launch"], "source": hbm["source"],
                           "hbm_gbs_of_that_launch": hbm["achieved"],
                           "bytes_per_launch": per_launch_b, "traffic": hbm["traffic"]}
    if not args.no_cpu_baseline and kind in ("verify", "tree", "batch"):
        threads = cpu_threads()
        t0 = time.perf_counter()
        par = parents
        pr = props
        if kind == "batch":
            pr, par = bdraft[0]["props"], bdraft[0]["parents"]
        times = cpu_baseline(ctx, tensors, cfg, ctx_len, M, pr, threads, parents=par)
        t_step, t_layer, sample = cpu_summary(times, cfg, M, ctx_len, threads, nseq=nseq)
        # one thread: the 1-layer forward, the per-layer time scaled by the
        # multi-thread run's layer / 1-layer ratio (the layer work splits
        # over threads the same way as the head's)
        t1 = cpu_baseline(ctx, tensors, cfg, ctx_len, M, pr, 1, layers=(1,), parents=par)[1]
        t_step1 = t1 * t_step / times[1]
        out["cpu_baseline"] = dict(
            value=round(tokens / t_step, 3), unit=unit, cores=threads, kind="port",
            sample=sample, single_thread_value=round(tokens / t_step1, 4),
            single_thread_sample="1-layer forward on 1 thread %.2f s, scaled by the %d-thread "
                                 "step / 1-layer ratio" % (t1, threads),
            nproc=os.cpu_count(), cpu_model=cpu_model())
        log("cpu baseline in %.1f s" % (time.perf_counter() - t0))
    elif not args.no_cpu_baseline and kind == "generate" and cfg["n_layer"] * cfg["n_embd"] <= 8192:
        # the reference's own CPU-runnable case: the whole generate on the host
        threads = cpu_threads()
        t0 = time.perf_counter()
        tps, sample = cpu_generate_baseline(ctx, tensors, dtensors, cfg, W["draft_cfg"], prompt,
                                            W["N"], M, threads)
        out["cpu_baseline"] = dict(value=round(tps, 3), unit=unit, cores=threads, kind="port",
                                   sample=sample, nproc=os.cpu_count(), cpu_model=cpu_model())
        log("cpu baseline in %.1f s" % (time.perf_counter() - t0))
    print(json.dumps(out), flush=True)
    if drafter is not None:
        drafter.free()
        dkv.free()
        dmodel.free()
        synth.free(dtensors)
    if qbuf is not None:
        qbuf.free()
    for b in blog + bbase + [dr["q"] for dr in bdraft if dr["q"] is not None] + bkv[1:]:
        b.free()
    logits.free()
    base.free()
    kv.free()
    model.free()
    synth.free(tensors)
    ctx.close()


if __name__ == "__main__":
    main()
