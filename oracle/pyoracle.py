"""ctypes view of the CPU oracle (liboracle.so) and of the library built
from the reference's own sources (_ref/libftref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The product (xwfes_amd/) never imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libftref.so")

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 30
# the Sampler's state for seed 0 (include/ft/sampler.h:19)
SAMPLER_SEED = 0x9E3779B97F4A7C15
# generate()'s draft cut compares float probabilities with 0.02f and the
# double running product with 0.05f (src/spec.cpp:279-281)
CUT_MIN_PROB = float(np.float32(0.02))
CUT_MIN_CUM = float(np.float32(0.05))
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20),
         Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
ACCEPT_GREEDY, ACCEPT_RATIO, ACCEPT_RESIDUAL = 0, 1, 2
KV_F32, KV_F16 = 0, 1
LAYER_TENSORS = ("attn_norm", "q", "k", "v", "o", "ffn_norm", "gate", "up", "down")
# optional per-layer roles, in the order of orc_model.ext (ftx_oracle.h):
# attention bias and per-head q / k norms, the MoE router, the experts'
# planes (ne1 = n_expert * rows of one plane), router bias, shared expert
LAYER_EXT = ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm", "gate_inp", "gate_exps",
             "up_exps", "down_exps", "router_bias", "gate_sh", "up_sh", "down_sh")

_fp = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_i32p = C.POINTER(C.c_int32)
_u64p = C.POINTER(C.c_uint64)
_dp = C.POINTER(C.c_double)


def build():
    subprocess.check_call(["make", "-s", "-C", HERE, "liboracle.so"])


def build_ref(ref_root="/root/reference/ft-igpu-src"):
    """Compile the reference's own build where the reference tree exists."""
    if not os.path.isdir(ref_root):
        return False
    subprocess.check_call(["make", "-s", "-C", HERE, "-f", "Makefile.ref",
                           "REF_ROOT=" + ref_root])
    return True


def row_bytes(dtype, n):
    be, bb = BLOCK[dtype]
    return (n + be - 1) // be * bb


def _ptr(a, t):
    return a.ctypes.data_as(t)


class _TensorC(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int32), ("pad_", C.c_int32),
                ("ne0", C.c_int64), ("ne1", C.c_int64)]


class _ModelC(C.Structure):
    _fields_ = [("n_layer", C.c_int64), ("n_embd", C.c_int64), ("n_head", C.c_int64),
                ("n_head_kv", C.c_int64), ("head_dim", C.c_int64), ("n_ff", C.c_int64),
                ("vocab", C.c_int64), ("rms_eps", C.c_float), ("rope_neox", C.c_int32),
                ("rope_theta", C.c_double), ("tok_embd", _TensorC), ("out_norm", _TensorC),
                ("output", _TensorC), ("layers", C.POINTER(_TensorC)),
                ("ext", C.POINTER(_TensorC)), ("n_expert", C.c_int64),
                ("n_expert_used", C.c_int64)]


class Oracle:
    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            build()
        L = self.lib = C.CDLL(path)
        L.orc_half_to_float.restype = C.c_float
        L.orc_half_to_float.argtypes = [C.c_uint16]
        L.orc_float_to_half.restype = C.c_uint16
        L.orc_float_to_half.argtypes = [C.c_float]
        L.orc_bf16_to_float.restype = C.c_float
        L.orc_bf16_to_float.argtypes = [C.c_uint16]
        L.orc_dequant_row.argtypes = [_fp, C.c_void_p, C.c_int, C.c_int64]
        L.orc_dot_row_f32.restype = C.c_float
        L.orc_dot_row_f32.argtypes = [_fp, C.c_void_p, C.c_int, C.c_int64]
        L.orc_quantize_row.argtypes = [C.c_void_p, _fp, C.c_int, C.c_int64]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_matmul.argtypes = [_fp, C.c_int64, C.c_int64, C.c_void_p, C.c_int, C.c_int64, _fp]
        L.orc_down_axpy.argtypes = [_fp, C.c_int64, C.c_int64, C.c_void_p, C.c_int, C.c_int64, _fp]
        L.orc_rms_norm.argtypes = [_fp, _fp, _fp, C.c_int64, C.c_float]
        L.orc_rope_vec.argtypes = [_fp, C.c_int64, C.c_int64, C.c_double, C.c_int]
        L.orc_softmax_inplace.argtypes = [_fp, C.c_int64]
        L.orc_expert_ffn.argtypes = [_fp, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_int,
                                     C.c_void_p, C.c_int, C.c_int64, _fp, _fp, _fp]
        L.orc_moe_route.argtypes = [_fp, C.c_int64, C.c_int64, C.c_int64, _fp, _i32p, _fp, _i32p,
                                    _i32p]
        L.orc_forward.argtypes = [C.POINTER(_ModelC), C.c_void_p, C.c_void_p, C.c_int, C.c_int64,
                                  C.c_int64, _i32p, C.c_int64, _i32p, C.c_int, _fp]
        L.orc_rng_next.restype = C.c_uint64
        L.orc_rng_next.argtypes = [_u64p]
        L.orc_rng_float.restype = C.c_float
        L.orc_rng_float.argtypes = [_u64p]
        L.orc_argmax.restype = C.c_int32
        L.orc_argmax.argtypes = [_fp, C.c_int64]
        L.orc_softmax_prob.restype = C.c_float
        L.orc_softmax_prob.argtypes = [_fp, C.c_int64, C.c_int32, C.c_float]
        L.orc_accept_chain_greedy.argtypes = [_fp, _fp, C.c_int64, _i32p, C.c_int64]
        L.orc_accept_chain_sampling.argtypes = [_fp, _fp, _fp, C.c_int64, _i32p, C.c_int64,
                                                C.c_float, _u64p]
        L.orc_sample_weights.restype = C.c_int32
        L.orc_sample_weights.argtypes = [_dp, C.c_int64, C.c_float]
        L.orc_verify_accept.argtypes = [_fp, _fp, C.c_int64, C.c_int64, _i32p, _i32p, _fp, _fp,
                                        C.c_int, C.c_float, C.POINTER(C.c_uint64),
                                        C.POINTER(C.c_uint64), C.c_int32, C.c_float, _i32p,
                                        _i32p, _i32p, _fp]
        L.orc_sampler_sample.restype = C.c_int32
        L.orc_sampler_sample.argtypes = [_fp, C.c_int64, C.c_float, C.c_int32, C.c_float,
                                         C.POINTER(C.c_uint64)]

    # ---- formats ----
    def half_to_float(self, h):
        return self.lib.orc_half_to_float(int(h))

    def float_to_half(self, f):
        return self.lib.orc_float_to_half(float(f))

    def bf16_to_float(self, b):
        return self.lib.orc_bf16_to_float(int(b))

    def dequant(self, raw, dtype, n, rows=1):
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        rb = row_bytes(dtype, n)
        assert raw.size >= rb * rows
        out = np.empty((rows, n), np.float32)
        for r in range(rows):
            rc = self.lib.orc_dequant_row(_ptr(out[r], _fp), raw.ctypes.data + r * rb, dtype, n)
            assert rc == 0, "unsupported dtype %d" % dtype
        return out if rows > 1 else out[0]

    def quantize(self, x, dtype):
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        rows, n = x.shape
        rb = row_bytes(dtype, n)
        out = np.zeros(rows * rb, np.uint8)
        for r in range(rows):
            rc = self.lib.orc_quantize_row(out.ctypes.data + r * rb, _ptr(x[r], _fp), dtype, n)
            assert rc == 0
        return out

    def dot(self, x, raw, dtype, n):
        x = np.ascontiguousarray(x, dtype=np.float32)
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        return self.lib.orc_dot_row_f32(_ptr(x, _fp), raw.ctypes.data, dtype, n)

    # ---- ops ----
    def set_threads(self, n):
        self.lib.orc_set_threads(int(n))

    def matmul(self, x, raw, dtype, N):
        x = np.ascontiguousarray(x, dtype=np.float32)
        M, K = x.shape
        y = np.empty((M, N), np.float32)
        self.lib.orc_matmul(_ptr(x, _fp), M, K, raw.ctypes.data, dtype, N, _ptr(y, _fp))
        return y

    def down_axpy(self, x, raw, dtype, N, y=None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        M, n_in = x.shape
        y = np.zeros((M, N), np.float32) if y is None else np.ascontiguousarray(y, np.float32).copy()
        self.lib.orc_down_axpy(_ptr(x, _fp), M, n_in, raw.ctypes.data, dtype, N, _ptr(y, _fp))
        return y

    def rms_norm(self, x, w, eps=1e-5):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        wp = _ptr(np.ascontiguousarray(w, np.float32), _fp) if w is not None else None
        self.lib.orc_rms_norm(_ptr(out, _fp), _ptr(x, _fp), wp, x.size, eps)
        return out

    def rope(self, v, pos, theta, neox):
        v = np.ascontiguousarray(v, np.float32).copy()
        self.lib.orc_rope_vec(_ptr(v, _fp), v.size, pos, theta, int(neox))
        return v

    def expert_ffn(self, x, gate, up, gu_dt, down, down_dt, F, out=None):
        """One expert's SwiGLU FFN over the rows of x: out [S][K] + the FFN."""
        x = np.ascontiguousarray(x, np.float32)
        S, K = x.shape
        y = np.zeros((S, K), np.float32) if out is None else np.array(out, np.float32)
        self.lib.orc_expert_ffn(_ptr(x, _fp), S, K, gate.ctypes.data, up.ctypes.data, gu_dt,
                                down.ctypes.data, down_dt, F, _ptr(y, _fp), None, None)
        return y

    def moe_route(self, router, U, bias=None):
        """Routing of router rows [M][E]: (probabilities [M][E], experts
        [M][U], weights [M][U], experts in first-use order)."""
        r = np.ascontiguousarray(router, np.float32).copy()
        M, E = r.shape
        te = np.empty((M, U), np.int32)
        tw = np.empty((M, U), np.float32)
        used = np.empty(E, np.int32)
        n = C.c_int32(0)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.lib.orc_moe_route(_ptr(r, _fp), M, E, U, None if b is None else _ptr(b, _fp),
                               _ptr(te, _i32p), _ptr(tw, _fp), _ptr(used, _i32p), C.byref(n))
        return r, te, tw, used[:n.value].copy()

    def softmax(self, p):
        p = np.ascontiguousarray(p, np.float32).copy()
        self.lib.orc_softmax_inplace(_ptr(p, _fp), p.size)
        return p

    def generate(self, target, draft, prompt, max_new, spec_k=8, temp=0.0, top_k=40, top_p=0.95,
                 seed=0, cap=256, kv_dtype=np.float16, ref_bonus_row=False,
                 ref_draft_prefill=False, eos=-1):
        """generate's speculative block (src/spec.cpp:245-333) with a
        DraftModelDrafter (72-119) over two models of this module's form, on
        caches of kv_dtype: draft k greedy tokens with their T = 1
        probabilities (the drafter syncs to the history by prefill and
        truncates to the accepted prefix, clamped to what it holds, as
        Engine::truncate_to is, engine.cpp:423-428), cut them (276-285),
        verify them on the target, accept by the ratio test, draw the bonus
        from the row after the last accepted token by Sampler::sample (temp
        <= 0: the argmax, the test at T = 1), truncate, step the target on
        the bonus.  A round is emitted whole.  ref_bonus_row draws the bonus
        from rows[min(acc, M - 1)] as the reference does (309-311: the wrong
        row after a rejection), to compare with it.  ref_draft_prefill makes
        the drafter's sync forward its whole held history again before the
        new tokens, as the reference's Engine::prefill does on a non-empty
        engine without a prefix-cache hit (src/engine.cpp:614-621: the loop
        starts at the hit length, 0, not at the history length), again only
        to compare with it.  The ratio test runs at T = 1 whatever temp is
        (accept_chain_sampling ignores the temperature, spec.cpp:216); temp
        shapes the bonus draw only.  eos (the tokenizer's
        tokenizer.ggml.eos_token_id, -1 for none) ends the loop as the
        reference's does (316-328): an accepted draft token equal to it ends
        the round after every accepted token is out (no bonus), a bonus equal
        to it is emitted and stepped, a sampled token of an empty draft is
        emitted and not stepped.  Returns (tokens, stats)."""
        def state(model):
            c = model["cfg"]
            shape = (c["n_layer"], cap, c["n_head_kv"] * c["head_dim"])
            return dict(m=model, k=np.zeros(shape, kv_dtype), v=np.zeros(shape, kv_dtype), n=0,
                        lg=None)

        def fwd(st, toks):
            rows = self.forward(st["m"], st["k"], st["v"], st["n"], list(toks))
            return rows

        T, D = state(target), state(draft)
        D["hist"] = []  # the tokens in the drafter's cache, in order
        V = target["cfg"]["vocab"]
        rows = fwd(T, prompt)
        T["n"] = len(prompt)
        base = rows[-1]
        history = list(prompt)
        out = []
        rsamp = seed if seed else 88172645463325252
        sstate = seed if seed else SAMPLER_SEED
        acc_temp = 1.0
        bk, bp = (top_k, top_p) if temp > 0 else (1, 1.0)
        stats = dict(rounds=0, drafted=0, accepted=0, hit_eos=False)
        while len(out) < max_new:
            # DraftModelDrafter::sync + draft
            if D["n"] > len(history):
                D["n"] = 0
                D["hist"] = []
            if D["n"] < len(history):
                tail = history[D["n"]:]
                toks = (D["hist"] + tail) if ref_draft_prefill else tail
                r = fwd(D, toks)
                D["lg"] = r[-1]
                D["n"] += len(toks)
                D["hist"] = D["hist"] + toks
            pending_base = len(history)
            props, probs = [], []
            for j in range(spec_k):
                t = self.argmax(D["lg"])
                props.append(t)
                probs.append(self.softmax_prob(D["lg"], t, 1.0))
                if j + 1 < spec_k:
                    D["lg"] = fwd(D, [t])[0]
                    D["n"] += 1
                    D["hist"] = D["hist"] + [t]
            # the cut heuristic
            cut, cum = len(props), 1.0
            for i, p in enumerate(probs):
                if 0 <= p < CUT_MIN_PROB:
                    cut = i
                    break
                cum *= p if p > 0 else 1.0
                if cum < CUT_MIN_CUM:
                    cut = i + 1
                    break
            props, probs = props[:cut], probs[:cut]
            M = len(props)
            rows = fwd(T, props) if M else np.zeros((0, V), np.float32)
            r = self.verify_accept(base, rows, np.asarray(props, np.int32), ACCEPT_RATIO,
                                   temp=acc_temp, seed=rsamp, pd=np.asarray(probs, np.float32),
                                   sampler_state=sstate, top_k=bk, top_p=bp)
            acc = len(r["accepted"])
            bonus = r["bonus"]
            if ref_bonus_row and M:
                # the same one draw from the same state, from the reference's row
                bonus, _ = self.sampler_sample(rows[min(acc, M - 1)], temp if temp > 0 else 0.0,
                                               top_k, top_p, sstate)
            rsamp, sstate = r["rng"], r["sampler_state"]
            T["n"] += acc
            stats["rounds"] += 1
            stats["drafted"] += M
            stats["accepted"] += acc

            def commit():
                D["n"] = min(pending_base + acc, D["n"])
                D["hist"] = D["hist"][:D["n"]]

            if M == 0 and bonus == eos:  # an empty draft's sampled token
                out.append(bonus)
                stats["hit_eos"] = True
                break
            out += props[:acc]  # every accepted token is out, past an eos too
            history += props[:acc]
            if eos >= 0 and eos in props[:acc]:
                commit()
                stats["hit_eos"] = True
                break
            out.append(bonus)
            history.append(bonus)
            base = fwd(T, [bonus])[0]
            T["n"] += 1
            commit()
            if bonus == eos:
                stats["hit_eos"] = True
                break
        return out, stats

    @staticmethod
    def kv_commit(kcache, vcache, npast, nodes):
        """Keep the accepted draft path `nodes` (node indices of the verify
        step whose rows were written at npast + j) at slots npast + i; returns
        the new npast.  A chain (nodes[i] == i) is Engine::truncate_to(npast +
        n) / KvCache::set_npast (src/engine.cpp:423-428, include/ft/
        kv_cache.h:31); a tree path gathers its rows.  kcache / vcache are
        [L][cap][dk] arrays in the reference layout, modified in place."""
        nodes = [int(j) for j in nodes]
        for i, j in enumerate(nodes):
            if j < i or (i and j <= nodes[i - 1]):
                raise ValueError("nodes must be strictly increasing with nodes[i] >= i")
            if npast + j >= kcache.shape[1]:
                raise ValueError("node out of range")
        for i, j in enumerate(nodes):
            kcache[:, npast + i] = kcache[:, npast + j]
            vcache[:, npast + i] = vcache[:, npast + j]
        return npast + len(nodes)

    def forward(self, model, kcache, vcache, npast, toks, parents=None, layer_limit=0):
        """model: dict from make_model(); kcache/vcache: numpy [L][cap][dk]
        (float32 or float16, modified in place).  Returns logits [M][V]."""
        cfg = model["cfg"]
        keep = []

        def tc(name):
            t = model[name]
            keep.append(t["raw"])
            return _TensorC(t["raw"].ctypes.data, t["dtype"], 0, t["ne0"], t["ne1"])

        def opt(name):
            return tc(name) if name in model else _TensorC(None, 0, 0, 0, 0)

        nl, nt, nx = cfg["n_layer"], len(LAYER_TENSORS), len(LAYER_EXT)
        lay = (_TensorC * (nl * nt))()
        ext = (_TensorC * (nl * nx))()
        has_ext = False
        for l in range(nl):
            for i, nm in enumerate(LAYER_TENSORS):
                lay[l * nt + i] = opt("blk.%d.%s" % (l, nm))
            for i, nm in enumerate(LAYER_EXT):
                ext[l * nx + i] = opt("blk.%d.%s" % (l, nm))
                has_ext |= ("blk.%d.%s" % (l, nm)) in model
        md = _ModelC(cfg["n_layer"], cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"],
                     cfg["head_dim"], cfg["n_ff"], cfg["vocab"], cfg.get("rms_eps", 1e-5),
                     int(cfg.get("rope_neox", 0)), cfg.get("rope_theta", 10000.0),
                     tc("tok_embd"), tc("out_norm"), opt("output"), lay,
                     ext if has_ext else None, cfg.get("n_expert", 0),
                     cfg.get("n_expert_used", 0))
        toks = np.ascontiguousarray(toks, np.int32)
        M = toks.size
        par = None if parents is None else np.ascontiguousarray(parents, np.int32)
        kv_dt = KV_F16 if kcache.dtype == np.float16 else KV_F32
        assert kcache.flags.c_contiguous and vcache.flags.c_contiguous
        cap = kcache.shape[1]
        logits = np.empty((M, cfg["vocab"]), np.float32)
        rc = self.lib.orc_forward(C.byref(md), kcache.ctypes.data, vcache.ctypes.data, kv_dt, cap,
                                  npast, _ptr(toks, _i32p), M,
                                  None if par is None else _ptr(par, _i32p), layer_limit,
                                  _ptr(logits, _fp))
        assert rc == 0, "orc_forward failed"
        return logits

    # ---- acceptance ----
    def rng_next(self, state):
        s = C.c_uint64(state)
        v = self.lib.orc_rng_next(C.byref(s))
        return v, s.value

    def rng_floats(self, seed, n):
        s = C.c_uint64(seed)
        return np.array([self.lib.orc_rng_float(C.byref(s)) for _ in range(n)], np.float32)

    def argmax(self, row):
        row = np.ascontiguousarray(row, np.float32)
        return self.lib.orc_argmax(_ptr(row, _fp), row.size)

    def softmax_prob(self, row, t, temp=1.0):
        row = np.ascontiguousarray(row, np.float32)
        return self.lib.orc_softmax_prob(_ptr(row, _fp), row.size, int(t), temp)

    def accept_chain_greedy(self, base, rows, props):
        base = np.ascontiguousarray(base, np.float32)
        rows = np.ascontiguousarray(rows, np.float32)
        props = np.ascontiguousarray(props, np.int32)
        return self.lib.orc_accept_chain_greedy(_ptr(base, _fp), _ptr(rows, _fp), base.size,
                                                _ptr(props, _i32p), props.size)

    def accept_chain_sampling(self, base, rows, pd, props, temp, seed):
        base = np.ascontiguousarray(base, np.float32)
        rows = np.ascontiguousarray(rows, np.float32)
        pd = np.ascontiguousarray(pd, np.float32)
        props = np.ascontiguousarray(props, np.int32)
        s = C.c_uint64(seed)
        a = self.lib.orc_accept_chain_sampling(_ptr(base, _fp), _ptr(rows, _fp), _ptr(pd, _fp),
                                               base.size, _ptr(props, _i32p), props.size, temp,
                                               C.byref(s))
        return a, s.value

    def sample_weights(self, w, u):
        w = np.ascontiguousarray(w, np.float64)
        return self.lib.orc_sample_weights(_ptr(w, _dp), w.size, float(u))

    def sampler_sample(self, logits, temp=0.7, top_k=40, top_p=0.95, state=SAMPLER_SEED):
        """Sampler::sample (include/ft/sampler.h:30-94); returns (token, state)."""
        lg = np.ascontiguousarray(logits, np.float32)
        s = C.c_uint64(state)
        t = self.lib.orc_sampler_sample(_ptr(lg, _fp), lg.size, temp, top_k, top_p, C.byref(s))
        return t, s.value

    def verify_accept(self, base, rows, props, mode, temp=1.0, seed=0, parents=None, pd=None,
                      q=None, sampler_state=None, top_k=40, top_p=0.95):
        base = np.ascontiguousarray(base, np.float32)
        rows = np.ascontiguousarray(rows, np.float32)
        props = np.ascontiguousarray(props, np.int32)
        M, V = props.size, base.size
        par = None if parents is None else np.ascontiguousarray(parents, np.int32)
        pdv = None if pd is None else np.ascontiguousarray(pd, np.float32)
        qv = None if q is None else np.ascontiguousarray(q, np.float32)
        acc = np.zeros(max(M, 1), np.int32)
        na = C.c_int32(0)
        bonus = C.c_int32(0)
        mg = C.c_float(0)
        s = C.c_uint64(seed)
        ss = C.c_uint64(SAMPLER_SEED if sampler_state is None else sampler_state)
        rc = self.lib.orc_verify_accept(
            _ptr(base, _fp), _ptr(rows, _fp), M, V, _ptr(props, _i32p),
            None if par is None else _ptr(par, _i32p),
            None if pdv is None else _ptr(pdv, _fp),
            None if qv is None else _ptr(qv, _fp), mode, temp, C.byref(s), C.byref(ss), top_k,
            top_p, _ptr(acc, _i32p), C.byref(na), C.byref(bonus), C.byref(mg))
        assert rc == 0, "orc_verify_accept failed"
        return dict(accepted=acc[:na.value].tolist(), bonus=bonus.value, rng=s.value,
                    sampler_state=ss.value, margin=mg.value)


class Ref:
    """The reference's own functions (compiled from its sources by
    Makefile.ref).  Available only where the reference tree was present when
    the library was built."""

    def __init__(self, path=REF_PATH):
        L = self.lib = C.CDLL(path)
        L.ref_half_to_float.restype = C.c_float
        L.ref_half_to_float.argtypes = [C.c_uint16]
        L.ref_float_to_half.restype = C.c_uint16
        L.ref_float_to_half.argtypes = [C.c_float]
        L.ref_bf16_to_float.restype = C.c_float
        L.ref_bf16_to_float.argtypes = [C.c_uint16]
        L.ref_dequant_row.argtypes = [_fp, C.c_void_p, C.c_int, C.c_int64]
        L.ref_dot_row_f32.restype = C.c_float
        L.ref_dot_row_f32.argtypes = [_fp, C.c_void_p, C.c_int, C.c_int64]
        L.ref_cpu_matmul.argtypes = [_fp, C.c_int64, C.c_int64, C.c_void_p, C.c_int, C.c_int64,
                                     _fp, C.c_int]
        L.ref_down_axpy.argtypes = [_fp, C.c_int64, C.c_int64, C.c_void_p, C.c_int, C.c_int64, _fp]
        L.ref_argmax.argtypes = [_fp, C.c_int64]
        L.ref_softmax_prob.restype = C.c_float
        L.ref_softmax_prob.argtypes = [_fp, C.c_int64, C.c_int32]
        L.ref_accept_chain_greedy.argtypes = [_fp, _fp, C.c_int64, _i32p, C.c_int64]
        L.ref_accept_chain_sampling.argtypes = [_fp, _fp, _fp, C.c_int64, _i32p, C.c_int64,
                                                C.c_float, _u64p]
        L.ref_expert_stream.argtypes = [_fp, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_int, C.c_int64, C.c_int64, _fp]
        L.ref_engine_load.restype = C.c_void_p
        L.ref_engine_load.argtypes = [C.c_char_p, C.c_int, C.c_int64]
        L.ref_engine_free.argtypes = [C.c_void_p]
        L.ref_engine_vocab.restype = C.c_int64
        L.ref_engine_vocab.argtypes = [C.c_void_p]
        L.ref_engine_step.argtypes = [C.c_void_p, C.c_int32, _fp]
        L.ref_sampler_sample.restype = C.c_int32
        L.ref_sampler_sample.argtypes = [_fp, C.c_int64, C.c_float, C.c_int32, C.c_float,
                                         C.POINTER(C.c_uint64)]
        L.ref_generate.restype = C.c_int64
        L.ref_generate.argtypes = [C.c_char_p, C.c_char_p, _i32p, C.c_int64, C.c_int, C.c_int,
                                   C.c_float, C.c_int, C.c_float, C.c_uint64, C.c_int64,
                                   C.c_int64, _i32p, C.c_int64]
        L.ref_gguf_summary.restype = C.c_int64
        L.ref_gguf_summary.argtypes = [C.c_char_p, C.c_char_p, C.c_char_p, C.c_int64]

    @staticmethod
    def available():
        return os.path.exists(REF_PATH)

    def dequant(self, raw, dtype, n):
        raw = np.ascontiguousarray(raw, np.uint8)
        out = np.empty(n, np.float32)
        self.lib.ref_dequant_row(_ptr(out, _fp), raw.ctypes.data, dtype, n)
        return out

    def dot(self, x, raw, dtype, n):
        x = np.ascontiguousarray(x, np.float32)
        raw = np.ascontiguousarray(raw, np.uint8)
        return self.lib.ref_dot_row_f32(_ptr(x, _fp), raw.ctypes.data, dtype, n)

    def cpu_matmul(self, x, raw, dtype, N, threads=1):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        y = np.zeros(N, np.float32)
        self.lib.ref_cpu_matmul(_ptr(x, _fp), M, K, raw.ctypes.data, dtype, N, _ptr(y, _fp),
                                threads)
        return y

    def down_axpy(self, x, raw, dtype, N):
        x = np.ascontiguousarray(x, np.float32)
        M, n_in = x.shape
        y = np.zeros((M, N), np.float32)
        self.lib.ref_down_axpy(_ptr(x, _fp), M, n_in, raw.ctypes.data, dtype, N, _ptr(y, _fp))
        return y

    def softmax_prob(self, row, t):
        row = np.ascontiguousarray(row, np.float32)
        return self.lib.ref_softmax_prob(_ptr(row, _fp), row.size, int(t))

    def argmax(self, row):
        row = np.ascontiguousarray(row, np.float32)
        return self.lib.ref_argmax(_ptr(row, _fp), row.size)

    def accept_chain_greedy(self, base, rows, props):
        base = np.ascontiguousarray(base, np.float32)
        rows = np.ascontiguousarray(rows, np.float32)
        props = np.ascontiguousarray(props, np.int32)
        return self.lib.ref_accept_chain_greedy(_ptr(base, _fp), _ptr(rows, _fp), base.size,
                                                _ptr(props, _i32p), props.size)

    def accept_chain_sampling(self, base, rows, pd, props, temp, seed):
        base = np.ascontiguousarray(base, np.float32)
        rows = np.ascontiguousarray(rows, np.float32)
        pd = np.ascontiguousarray(pd, np.float32)
        props = np.ascontiguousarray(props, np.int32)
        s = C.c_uint64(seed)
        a = self.lib.ref_accept_chain_sampling(_ptr(base, _fp), _ptr(rows, _fp), _ptr(pd, _fp),
                                               base.size, _ptr(props, _i32p), props.size, temp,
                                               C.byref(s))
        return a, s.value

    def expert_stream(self, x, gate, up, down, dtype, F, chunk, out=None):
        """ExpertStreamer::run of one expert (F rows of K each) in windows of
        `chunk` neurons; returns out [M][K] + the FFN."""
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        y = np.zeros((M, K), np.float32) if out is None else np.array(out, np.float32)
        self.lib.ref_expert_stream(_ptr(x, _fp), M, K, gate.ctypes.data, up.ctypes.data,
                                   down.ctypes.data, dtype, F, chunk, _ptr(y, _fp))
        return y

    def engine_load(self, path, threads=1, ctx_len=0):
        h = self.lib.ref_engine_load(path.encode(), threads, ctx_len)
        assert h, "reference Engine failed to load " + path
        return h

    def engine_step(self, h, tok):
        V = self.lib.ref_engine_vocab(h)
        out = np.empty(V, np.float32)
        assert self.lib.ref_engine_step(h, tok, _ptr(out, _fp)) == 0
        return out

    def engine_free(self, h):
        self.lib.ref_engine_free(h)

    def sampler_sample(self, logits, temp, top_k, top_p, state):
        """The reference's Sampler::sample from `state` (seed 0 in the params,
        so the state is used as it is); returns (token, state after)."""
        lg = np.ascontiguousarray(logits, np.float32)
        s = C.c_uint64(state)
        t = self.lib.ref_sampler_sample(_ptr(lg, _fp), lg.size, temp, top_k, top_p, C.byref(s))
        return t, s.value

    def generate(self, target_path, draft_path, prompt, max_new, spec_k, temp, top_k=40,
                 top_p=0.95, seed=0, ctx_len=256, prefill_batch=256):
        """The reference's generate with a DraftModelDrafter (see
        ref_harness.cpp); returns the emitted tokens."""
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max_new + spec_k + 8, np.int32)
        n = self.lib.ref_generate(target_path.encode(), draft_path.encode(), _ptr(pr, _i32p),
                                  pr.size, max_new, spec_k, temp, top_k, top_p, seed, ctx_len,
                                  prefill_batch, _ptr(out, _i32p), out.size)
        assert n >= 0, "reference generate failed"
        return out[:n].tolist()

    def gguf_summary(self, path, keys):
        """The reference parser's summary of a GGUF (see ref_harness.cpp),
        or ("error", message) when it throws."""
        cap = 1 << 22
        buf = C.create_string_buffer(cap)
        n = self.lib.ref_gguf_summary(path.encode(), "\n".join(keys).encode(), buf, cap)
        text = buf.value.decode("utf-8", "surrogateescape")
        return ("error", text) if n < 0 else text


# ---------------- synthetic models (test data) ----------------

def model_cfg(n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, vocab, rope_theta=10000.0,
              rope_neox=0, rms_eps=1e-5, n_expert=0, n_expert_used=0):
    """n_expert > 0 makes every layer a MoE layer of n_expert experts of
    n_ff rows each, n_expert_used routed per token."""
    return dict(n_layer=n_layer, n_embd=n_embd, n_head=n_head, n_head_kv=n_head_kv,
                head_dim=head_dim, n_ff=n_ff, vocab=vocab, rope_theta=rope_theta,
                rope_neox=rope_neox, rms_eps=rms_eps, n_expert=n_expert,
                n_expert_used=n_expert_used)


def tensor_shapes(cfg, extras=()):
    """(name, ne0 cols, ne1 rows) of every tensor; down uses the reference
    orientation (n_ff rows of n_embd cols).  A MoE config (n_expert > 0)
    has the router and the experts' planes (ne1 = n_expert * n_ff) instead
    of the dense FFN; extras adds optional roles of LAYER_EXT (attention
    bias, q / k norms, router bias, a shared expert of n_ff rows)."""
    d, hd, F = cfg["n_embd"], cfg["head_dim"], cfg["n_ff"]
    qd, kd = cfg["n_head"] * hd, cfg["n_head_kv"] * hd
    E = cfg.get("n_expert", 0)
    ext = {"q_bias": (qd, 1), "k_bias": (kd, 1), "v_bias": (kd, 1), "q_norm": (hd, 1),
           "k_norm": (hd, 1), "router_bias": (E, 1), "gate_sh": (d, F), "up_sh": (d, F),
           "down_sh": (d, F)}
    out = [("tok_embd", d, cfg["vocab"]), ("out_norm", d, 1), ("output", d, cfg["vocab"])]
    for l in range(cfg["n_layer"]):
        p = "blk.%d." % l
        out += [(p + "attn_norm", d, 1), (p + "q", d, qd), (p + "k", d, kd), (p + "v", d, kd),
                (p + "o", qd, d), (p + "ffn_norm", d, 1)]
        if E:
            out += [(p + "gate_inp", d, E), (p + "gate_exps", d, E * F),
                    (p + "up_exps", d, E * F), (p + "down_exps", d, E * F)]
        else:
            out += [(p + "gate", d, F), (p + "up", d, F), (p + "down", d, F)]
        out += [(p + x, ext[x][0], ext[x][1]) for x in extras]
    return out


def make_model(orc, cfg, dtypes, seed=1, std=0.02, tied=False, extras=()):
    """Random-init model: weights N(0, std) quantised to dtypes[name-suffix]
    (keys: 'tok_embd', 'output', 'q', 'k', 'v', 'o', 'gate', 'up', 'down',
    and for MoE 'gate_inp', 'gate_exps', 'up_exps', 'down_exps', and the
    extras' matrices 'gate_sh', 'up_sh', 'down_sh'); norms (also q_norm /
    k_norm) are F32 vectors of 1 + 0.3 N(0, 1), different per layer and
    role; biases are F32 N(0, 0.5) (router bias N(0, 1)).  The router
    weights are N(0, 4 / n_embd), router logits of a few units, so that the
    routing differs from token to token and the second expert's weight is
    not negligible."""
    rng = np.random.default_rng(seed)
    model = {"cfg": dict(cfg)}
    for name, ne0, ne1 in tensor_shapes(cfg, extras):
        if name == "output" and tied:
            continue
        key = name.split(".")[-1]
        if key in ("attn_norm", "ffn_norm", "out_norm", "q_norm", "k_norm"):
            w = (1.0 + 0.3 * rng.standard_normal(ne0)).astype(np.float32)
            model[name] = dict(raw=w.view(np.uint8).copy(), dtype=F32, ne0=ne0, ne1=1)
            continue
        if key.endswith("bias"):
            sd = 1.0 if key == "router_bias" else 0.5
            w = (sd * rng.standard_normal(ne0)).astype(np.float32)
            model[name] = dict(raw=w.view(np.uint8).copy(), dtype=F32, ne0=ne0, ne1=1)
            continue
        dt = dtypes[key]
        sd = 2.0 / np.sqrt(ne0) if key == "gate_inp" else std
        w = (rng.standard_normal((ne1, ne0)) * sd).astype(np.float32)
        model[name] = dict(raw=orc.quantize(w, dt), dtype=dt, ne0=ne0, ne1=ne1)
    return model
