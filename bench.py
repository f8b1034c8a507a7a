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
REPLAY = 20  # back-to-back issues of each dominant-class launch when timing it
LLAMA3_8B = dict(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=14336,
                vocab=128256, rope_theta=500000.0, rope_neox=0, rms_eps=1e-5)
TINY_LLAMA = dict(n_layer=4, n_embd=512, n_head=8, n_head_kv=8, head_dim=64, n_ff=1408,
                  vocab=32000, rope_theta=10000.0, rope_neox=0, rms_eps=1e-5)
LLAMA32_1B = dict(n_layer=16, n_embd=2048, n_head=32, n_head_kv=8, head_dim=64, n_ff=8192,
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
}
DTYPES = {"q4_k_m": "q4_k/q6_k weights, f16 KV, fp32 accumulate",
          "q4_0": "q4_0 weights (f32 embedding), f16 KV, fp32 accumulate",
          "q8_0_attn": "q8_0 attention / q4_k FFN / q6_k head weights, f16 KV, fp32 accumulate"}


def mix_of(name, cfg):
    from xwfes_amd import synth
    return {"q4_k_m": lambda: synth.q4_k_m_mix(cfg),
            "q4_0": lambda: synth.uniform_mix(synth.Q4_0, embd=synth.F32),
            "q8_0_attn": lambda: synth.q8_attn_mix(cfg)}[name]()


def draft_tree(V, branching, seed):
    """A full draft tree (nodes in breadth-first order, parents[i] < i): each
    node's children are drawn from one Dirichlet(1) distribution over the
    vocab, which is every child's q row."""
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


def cpu_baseline(ctx, tensors, cfg, ctx_len, M, props, threads):
    """The oracle's reference loop nest (CpuBackend::matmul, matmul_down_axpy,
    Impl::attn) timed on this host on a bounded sample: 1-layer and 2-layer
    forwards of the same weights (layer 0, tok_embd, output) at the same M and
    context, extrapolated linearly to all layers."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as P
    orc = P.Oracle()
    orc.set_threads(threads)

    def host(t):
        raw = np.empty(t.nbytes, np.uint8)
        ctx.copy(raw.ctypes.data, t.ptr, t.nbytes)
        return dict(raw=raw, dtype=t.dtype, ne0=t.ne[0], ne1=t.ne[1])

    base = {k: host(tensors[k]) for k in ("tok_embd", "output", "out_norm")}
    layer0 = {nm: host(tensors["blk.0." + nm]) for nm in P.LAYER_TENSORS}
    kdim = cfg["n_head_kv"] * cfg["head_dim"]
    rng = np.random.default_rng(4)
    times = {}
    for nl in (1, 2):
        model = dict(base)
        model["cfg"] = dict(cfg, n_layer=nl)
        for l in range(nl):
            for nm in P.LAYER_TENSORS:
                model["blk.%d.%s" % (l, nm)] = layer0[nm]
        cap = ctx_len + M
        k = rng.standard_normal((nl, cap, kdim)).astype(np.float16)
        v = rng.standard_normal((nl, cap, kdim)).astype(np.float16)
        orc.forward(model, k, v, ctx_len, props[:1])  # warm caches and threads
        t0 = time.perf_counter()
        orc.forward(model, k, v, ctx_len, props)
        times[nl] = time.perf_counter() - t0
    t_layer = max(times[2] - times[1], 0.0)
    t_step = times[1] + (cfg["n_layer"] - 1) * t_layer
    return dict(value=M / t_step, unit="verified tokens/s", cores=threads, kind="port",
                sample="oracle forward of M=%d tokens at ctx %d over 1 and 2 layers of the same "
                       "weights (%.2f s, %.2f s), extrapolated to %d layers: %.3f s/step"
                       % (M, ctx_len, times[1], times[2], cfg["n_layer"], t_step))


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
    model = ctx.model(cfg, tensors, max_tokens=max(M, 8))
    kv = model.kv(max(ctx_len, P_tok + W.get("N", 0) + 16) + M + 8)
    drafter = dtensors = dmodel = dkv = None
    gen_stats = []
    if kind == "generate":
        dcfg = W["draft_cfg"]
        dtensors = synth.build(ctx, dcfg, mix_of(W["mix"], dcfg), seed=2)
        dmodel = ctx.model(dcfg, dtensors, max_tokens=8)
        dkv = dmodel.kv(P_tok + W["N"] + 32)
        drafter = spec.DraftModelDrafter(ctx, dmodel, dkv)
        log("draft model built (%.3f GB of weights)" % (synth.weight_bytes(dtensors) / 1e9))
    kp, vp, _ = kv.pointers()
    n_kv = cfg["n_layer"] * kv.cap_alloc * cfg["n_head_kv"] * cfg["head_dim"]
    ctx.fill_normal(kp, n_kv, seed=4, std=1.0, dtype=ftx.F16)
    ctx.fill_normal(vp, n_kv, seed=5, std=1.0, dtype=ftx.F16)
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
        parents, props, qrows = draft_tree(V, W["branching"], seed=6)
        assert len(props) == M
        qbuf = ctx.buffer(qrows.nbytes)
        qbuf.write(qrows)
        del qrows
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, V, P_tok)]
    rng_state = [5, ftx.SAMPLER_SEED]
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
        elif kind == "decode":
            kv.truncate(ctx_len)
            model.step(kv, int(props[0]), logits.ptr)
        elif kind == "generate":
            out, st = spec.generate(ctx, model, kv, drafter, prompt, W["N"], spec_k=M, temp=temp)
            gen_stats.append((len(out), st))
        else:
            kv.truncate(0)
            model.prefill(kv, prompt, logits.ptr, chunk=M)

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
    traced_ms = sum(e["ms"] for e in tr.values()) / max(args.trace_steps, 1)
    dom_name, dom = max(tr.items(), key=lambda kv_: kv_[1]["ms"])
    per_launch_b = dom["bytes"] / dom["launches"]
    # the dominant class's launch time: each of its launches replayed
    # REPLAY times back to back between the two events, so the events' own
    # overhead (a few microseconds per bracket) is spread over the replays
    ctx.trace_replay(dom_name, REPLAY)
    ctx.trace(True)
    step()
    rep = ctx.trace_read()[dom_name]
    ctx.trace(False)
    ctx.trace_replay(dom_name, 1)
    per_launch_ms = rep["ms"] / rep["launches"]
    achieved = per_launch_b / (per_launch_ms * 1e-3) / 1e9
    log("dominant class %s: %.2f us per launch (events, %d replays), %.2f us in the step trace" % (
        dom_name, per_launch_ms * 1e3, REPLAY, dom["ms"] / dom["launches"] * 1e3))
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
    else:
        sb = step_bytes(tensors, cfg, ctx_len, M)
        tokens = M
    gbs = sb / (ms_step * 1e-3) / 1e9
    metric = {"verify": "verify-step tokens/s + HBM GB/s (% of peak), 8B-shape Q4_K, K=8 draft, "
                        "1 GPU",
              "tree": "tree verify-step tokens/s + HBM GB/s (% of peak), 8B-shape Q8_0 attention "
                      "/ Q4_K FFN, 52-node draft tree, ctx 4096, 1 GPU",
              "decode": "decode tokens/s (Engine::step, M=1, ctx 2048), 8B-shape Q4_K, 1 GPU",
              "prefill": "prefill tokens/s (512-token prompt, chains of 8), 8B-shape Q4_K, "
                         "1 GPU",
              "generate": "generated tokens/s (speculative: %s target, %s draft, %d draft "
                          "tokens a round, greedy), 1 GPU" % (
                              W["mix"] + " %d-layer d%d" % (cfg["n_layer"], cfg["n_embd"]),
                              "%d-layer d%d" % (W["draft_cfg"]["n_layer"],
                                                W["draft_cfg"]["n_embd"]) if "draft_cfg" in W
                              else "", M)}[kind]
    unit = {"verify": "verified tokens/s", "tree": "verified tokens/s", "decode": "decoded tokens/s",
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
                   "vocab": V, "mix": W["mix"], "accept": {"verify": "ratio", "tree": "residual"}.get(kind),
                   "temperature": temp, "batch": 1},
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
                     "replays": REPLAY,
                     "traffic": measured_traffic(args.workload, dom_name)},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline and kind == "verify":
        threads = min(16, os.cpu_count() or 1)
        t0 = time.perf_counter()
        out["cpu_baseline"] = cpu_baseline(ctx, tensors, cfg, ctx_len, M, props, threads)
        log("cpu baseline in %.1f s" % (time.perf_counter() - t0))
    print(json.dumps(out), flush=True)
    if drafter is not None:
        drafter.free()
        dkv.free()
        dmodel.free()
        synth.free(dtensors)
    if qbuf is not None:
        qbuf.free()
    logits.free()
    base.free()
    kv.free()
    model.free()
    synth.free(tensors)
    ctx.close()


if __name__ == "__main__":
    main()
