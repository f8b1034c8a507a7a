"""Synthetic random-init models built directly on the device.

Weights are N(0, std) drawn by ftx_fill_normal and quantised by ftx_quantize
into resident tensors, so a 4.6 GB model is built without host traffic.
Tensor names and orientations follow the reference's GGUF layout
(src/engine.cpp:318-394): linear weights are rows of ne0 input columns, and
ffn_down is n_ff rows of n_embd columns (the reference's down orientation,
src/cpu_backend.cpp:60-75).
"""
import numpy as np

from . import ftx

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = ftx.F32, ftx.F16, ftx.Q4_0, ftx.Q8_0, ftx.Q4_K, ftx.Q6_K


def model_cfg(n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, vocab, rope_theta=10000.0,
              rope_neox=0, rms_eps=1e-5, n_expert=0, n_expert_used=0):
    return dict(n_layer=n_layer, n_embd=n_embd, n_head=n_head, n_head_kv=n_head_kv,
                head_dim=head_dim, n_ff=n_ff, vocab=vocab, rope_theta=rope_theta,
                rope_neox=rope_neox, rms_eps=rms_eps, n_expert=n_expert,
                n_expert_used=n_expert_used)


def tensor_shapes(cfg):
    """(name, ne) of every tensor of the llama layout: ne = (cols, rows), or
    (cols, rows, n_expert) for expert planes.  A MoE config (n_expert > 0)
    has the router (n_expert rows) and the experts' gate / up / down planes
    in place of the dense FFN."""
    d, hd, F = cfg["n_embd"], cfg["head_dim"], cfg["n_ff"]
    qd, kd = cfg["n_head"] * hd, cfg["n_head_kv"] * hd
    E = cfg.get("n_expert", 0)
    out = [("tok_embd", (d, cfg["vocab"])), ("out_norm", (d, 1)), ("output", (d, cfg["vocab"]))]
    for l in range(cfg["n_layer"]):
        p = "blk.%d." % l
        out += [(p + "attn_norm", (d, 1)), (p + "q", (d, qd)), (p + "k", (d, kd)),
                (p + "v", (d, kd)), (p + "o", (qd, d)), (p + "ffn_norm", (d, 1))]
        if E:
            out += [(p + "gate_inp", (d, E)), (p + "gate_exps", (d, F, E)),
                    (p + "up_exps", (d, F, E)), (p + "down_exps", (d, F, E))]
        else:
            out += [(p + "gate", (d, F)), (p + "up", (d, F)), (p + "down", (d, F))]
    return out


def q4_k_m_mix(cfg):
    """llama.cpp's Q4_K_M choice: Q6_K for output.weight and for attn_v /
    ffn_down on the 'more bits' layers (i < L/8, i >= 7L/8, or
    (i - L/8) % 3 == 2), Q4_K elsewhere."""
    L = cfg["n_layer"]

    def dtype(name):
        key = name.split(".")[-1]
        if key == "output":
            return Q6_K
        if name.startswith("blk.") and key in ("v", "down"):
            i = int(name.split(".")[1])
            if i < L // 8 or i >= 7 * L // 8 or (i - L // 8) % 3 == 2:
                return Q6_K
        return Q4_K
    return dtype


def q8_attn_mix(cfg):
    """Q8_0 attention projections (q, k, v, o), Q6_K output, Q4_K FFN."""
    def dtype(name):
        key = name.split(".")[-1]
        if key == "output":
            return Q6_K
        return Q8_0 if key in ("q", "k", "v", "o") else Q4_K
    return dtype


def uniform_mix(dt, embd=None):
    """Every matrix in dt (the MoE router stays F32, as GGUF converters keep
    ffn_gate_inp), the embedding in `embd` if given."""
    def dtype(name):
        if name == "tok_embd" and embd is not None:
            return embd
        if name.endswith("gate_inp"):
            return F32
        return dt
    return dtype


def build(ctx, cfg, dtype_of, seed=1, std=0.02, tied=False):
    """Returns {name: ftx.Tensor}.  Norm weights are F32 vectors of
    1 + 0.1 N(0, 1), one per layer and role; the MoE router is F32
    N(0, 4 / n_embd) (router logits of a few units, so that routing varies
    from token to token)."""
    shapes = [s for s in tensor_shapes(cfg) if not (tied and s[0] == "output")]
    big = max(int(np.prod(ne)) for name, ne in shapes)
    scratch = ctx.buffer(big * 4)
    tensors = {}
    nrng = np.random.default_rng(seed)
    try:
        for i, (name, ne) in enumerate(shapes):
            key = name.split(".")[-1]
            if key in ("attn_norm", "ffn_norm", "out_norm"):
                w = (1.0 + 0.1 * nrng.standard_normal(ne[0])).astype(np.float32)
                tensors[name] = ctx.upload(w.view(np.uint8), F32, (ne[0], 1))
                continue
            dt = dtype_of(name)
            t = ctx.alloc(dt, ne)
            n = int(np.prod(ne))
            sd = 2.0 / np.sqrt(ne[0]) if key == "gate_inp" else std
            if dt == F32:
                ctx.fill_normal(t.ptr, n, seed * 1000003 + i, sd)
            else:
                ctx.fill_normal(scratch.ptr, n, seed * 1000003 + i, sd)
                ctx.quantize(scratch.ptr, t)
            tensors[name] = t
    finally:
        scratch.free()
    return tensors


def weight_bytes(tensors):
    return sum(t.nbytes for t in tensors.values())


def free(tensors):
    for t in tensors.values():
        t.free()
