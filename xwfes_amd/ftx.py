"""ctypes binding of libftx.so (include/ftx.h).

The library is the product: HIP kernels for gfx950 behind a C ABI.  This
module only marshals arguments; there is no compute fallback.  If the shared
library is missing, importing the binding raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# FTX_LIB selects another build of the library (e.g. to compare two builds)
LIB_PATH = os.environ.get("FTX_LIB") or os.path.join(HERE, "libftx.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "ftx.h")

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20),
         Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
KV_F32, KV_F16 = 0, 1
# the sampler state of seed 0 (include/ft/sampler.h:19)
SAMPLER_SEED = 0x9E3779B97F4A7C15
ACCEPT_GREEDY, ACCEPT_RATIO, ACCEPT_RESIDUAL = 0, 1, 2
LAYER_TENSORS = ("attn_norm", "q", "k", "v", "o", "ffn_norm", "gate", "up", "down")
# optional per-layer tensors in the order of FTX_X_* (include/ftx.h)
LAYER_EXT = ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm", "gate_inp", "gate_exps",
             "up_exps", "down_exps", "router_bias", "gate_sh", "up_sh", "down_sh")
ERRORS = {-1: "invalid argument", -2: "unsupported", -3: "device error", -4: "out of memory",
          -5: "out of range"}

_vp = C.c_void_p
_i64 = C.c_int64
_fp = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)


class FtxError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("ftx error %d (%s): %s" % (code, ERRORS.get(code, "?"), msg))
        self.code = code


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("mem_bytes", C.c_int64), ("compute_units", C.c_int32),
                ("arch_major", C.c_int32), ("arch_minor", C.c_int32), ("pad_", C.c_int32)]


class ExpertJob(C.Structure):
    _fields_ = [("x", _vp), ("out", _vp), ("gate", _vp), ("up", _vp), ("down", _vp),
                ("dt", C.c_int32), ("pad_", C.c_int32), ("M", _i64), ("K", _i64), ("IC", _i64),
                ("gate_up_row_stride", _i64), ("down_row_stride", _i64)]


class ModelDesc(C.Structure):
    _fields_ = [("n_layer", _i64), ("n_embd", _i64), ("n_head", _i64), ("n_head_kv", _i64),
                ("head_dim", _i64), ("n_ff", _i64), ("vocab", _i64), ("rms_eps", C.c_float),
                ("rope_neox", C.c_int32), ("rope_theta", C.c_double), ("tok_embd", _vp),
                ("out_norm", _vp), ("output", _vp), ("layers", C.POINTER(_vp)),
                ("max_tokens", _i64), ("layer_ext", C.POINTER(_vp)), ("n_expert", _i64),
                ("n_expert_used", _i64)]


class VerifyArgs(C.Structure):
    _fields_ = [("M", _i64), ("tokens", _i32p), ("parents", _i32p), ("logits", _vp),
                ("advance", C.c_int32), ("pad_", C.c_int32)]


class SeqArgs(C.Structure):
    _fields_ = [("kv", _vp), ("M", _i64), ("tokens", _i32p), ("parents", _i32p),
                ("logits", _vp), ("advance", C.c_int32), ("pad_", C.c_int32)]


class AcceptArgs(C.Structure):
    _fields_ = [("base_row", _vp), ("rows", _vp), ("q", _vp), ("M", _i64), ("V", _i64),
                ("props", _i32p), ("parents", _i32p), ("pd", _fp), ("mode", C.c_int32),
                ("temp", C.c_float), ("rng", C.POINTER(C.c_uint64)), ("accepted", _i32p),
                ("n_acc", _i32p), ("bonus", _i32p), ("margin", _fp),
                ("sampler_rng", C.POINTER(C.c_uint64)), ("top_k", C.c_int32),
                ("top_p", C.c_float)]


class TraceEntry(C.Structure):
    _fields_ = [("name", C.c_char * 24), ("launches", C.c_int64), ("ms", C.c_double),
                ("bytes", C.c_double), ("kernel_launches", C.c_int64), ("kernel_ms", C.c_double)]


def header_functions(path=HEADER):
    """Names of the functions include/ftx.h declares."""
    import re
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ftx_[a-z_0-9]+)\s*\(", txt)))


def load(path=LIB_PATH):
    if not os.path.exists(path):
        raise FtxError(-3, "libftx.so is not built (%s); run __graft_entry__.build()" % path)
    L = C.CDLL(path)
    sig = {
        "ftx_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
        "ftx_destroy": (C.c_int, [_vp]),
        "ftx_device_info": (C.c_int, [_vp, C.POINTER(DeviceInfo)]),
        "ftx_last_error": (C.c_char_p, [_vp]),
        "ftx_set_stream": (C.c_int, [_vp, _vp]),
        "ftx_sync": (C.c_int, [_vp]),
        "ftx_row_bytes": (_i64, [C.c_int, _i64]),
        "ftx_tensor_upload": (C.c_int, [_vp, C.c_int, C.POINTER(_i64), _i64, _vp, C.POINTER(_vp)]),
        "ftx_tensor_alloc": (C.c_int, [_vp, C.c_int, C.POINTER(_i64), C.POINTER(_vp)]),
        "ftx_tensor_free": (C.c_int, [_vp]),
        "ftx_tensor_data": (_vp, [_vp]),
        "ftx_tensor_nbytes": (_i64, [_vp]),
        "ftx_quantize": (C.c_int, [_vp, _vp, _vp]),
        "ftx_dequant": (C.c_int, [_vp, _vp, _vp]),
        "ftx_matmul": (C.c_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
        "ftx_down_axpy": (C.c_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
        "ftx_down_axpy_noalloc": (C.c_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
        "ftx_expert_chunk": (C.c_int, [_vp, C.POINTER(ExpertJob)]),
        "ftx_alloc_staging": (_vp, [_vp, C.c_size_t]),
        "ftx_free_staging": (C.c_int, [_vp, _vp]),
        "ftx_stage": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
        "ftx_model_create": (C.c_int, [_vp, C.POINTER(ModelDesc), C.POINTER(_vp)]),
        "ftx_model_free": (C.c_int, [_vp]),
        "ftx_kv_create": (C.c_int, [_vp, _vp, _i64, C.c_int, C.POINTER(_vp)]),
        "ftx_kv_free": (C.c_int, [_vp]),
        "ftx_kv_pointers": (C.c_int, [_vp, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_i64)]),
        "ftx_kv_truncate": (C.c_int, [_vp, _i64]),
        "ftx_kv_commit": (C.c_int, [_vp, C.POINTER(C.c_int32), _i64]),
        "ftx_kv_write": (C.c_int, [_vp, _vp, _vp]),
        "ftx_kv_read": (C.c_int, [_vp, _vp, _vp]),
        "ftx_verify_step": (C.c_int, [_vp, _vp, _vp, C.POINTER(VerifyArgs)]),
        "ftx_verify_batch": (C.c_int, [_vp, _vp, C.POINTER(SeqArgs), _i64]),
        "ftx_accept": (C.c_int, [_vp, C.POINTER(AcceptArgs)]),
        "ftx_accept_batch": (C.c_int, [_vp, C.POINTER(AcceptArgs), C.c_int]),
        "ftx_argmax_prob": (C.c_int, [_vp, _vp, _i64, _i32p, _fp]),
        "ftx_fill_normal": (C.c_int, [_vp, _vp, C.c_int, _i64, C.c_uint64, C.c_float]),
        "ftx_trace": (C.c_int, [_vp, C.c_int]),
        "ftx_trace_read": (C.c_int, [_vp, C.POINTER(TraceEntry), C.c_int, C.POINTER(C.c_int)]),
        "ftx_trace_replay": (C.c_int, [_vp, C.c_char_p, C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


def row_bytes(dtype, n):
    be, bb = BLOCK[dtype]
    return (n + be - 1) // be * bb


def _ne(ne):
    ne = list(ne) + [1] * (4 - len(ne))
    return (_i64 * 4)(*ne)


class Tensor:
    def __init__(self, ctx, handle, dtype, ne):
        self.ctx, self.handle, self.dtype = ctx, handle, dtype
        self.ne = tuple(list(ne) + [1] * (4 - len(ne)))

    @property
    def ptr(self):
        return self.ctx.lib.ftx_tensor_data(self.handle)

    @property
    def nbytes(self):
        return self.ctx.lib.ftx_tensor_nbytes(self.handle)

    def free(self):
        if self.handle:
            self.ctx.lib.ftx_tensor_free(self.handle)
            self.handle = None


class DeviceBuffer:
    """Device memory from ftx_alloc_staging."""

    def __init__(self, ctx, nbytes):
        self.ctx, self.nbytes = ctx, int(nbytes)
        self.ptr = ctx.lib.ftx_alloc_staging(ctx.h, self.nbytes)
        if not self.ptr:
            raise FtxError(-4, ctx.error())

    def write(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        self.ctx.copy(self.ptr + offset, arr.ctypes.data, arr.nbytes)

    def read(self, dtype, count, offset=0):
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        self.ctx.copy(out.ctypes.data, self.ptr + offset, out.nbytes)
        return out

    def free(self):
        if self.ptr:
            self.ctx.lib.ftx_free_staging(self.ctx.h, self.ptr)
            self.ptr = None


class Context:
    def __init__(self, device=0, lib=None):
        self.lib = lib or load()
        h = _vp()
        rc = self.lib.ftx_create(device, C.byref(h))
        if rc:
            raise FtxError(rc, "ftx_create(%d) failed" % device)
        self.h = h.value

    def error(self):
        return self.lib.ftx_last_error(self.h).decode()

    def check(self, rc):
        if rc:
            raise FtxError(rc, self.error())

    def close(self):
        if self.h:
            self.lib.ftx_destroy(self.h)
            self.h = None

    def info(self):
        d = DeviceInfo()
        self.check(self.lib.ftx_device_info(self.h, C.byref(d)))
        return dict(name=d.name.decode(), mem_bytes=d.mem_bytes, compute_units=d.compute_units)

    def set_stream(self, stream_handle):
        self.check(self.lib.ftx_set_stream(self.h, stream_handle))

    def sync(self):
        self.check(self.lib.ftx_sync(self.h))

    def trace(self, enable):
        self.check(self.lib.ftx_trace(self.h, int(enable)))

    def trace_read(self):
        """{kernel class: dict(launches, ms, bytes)} since trace(True)."""
        buf = (TraceEntry * 32)()
        n = C.c_int(0)
        self.check(self.lib.ftx_trace_read(self.h, buf, 32, C.byref(n)))
        return {buf[i].name.decode(): dict(launches=buf[i].launches, ms=buf[i].ms,
                                           bytes=buf[i].bytes,
                                           kernel_launches=buf[i].kernel_launches,
                                           kernel_ms=buf[i].kernel_ms) for i in range(n.value)}

    def trace_replay(self, kind, times):
        """While tracing, issue each replayable launch of class `kind` `times`
        times back to back between its events (1 = off)."""
        self.check(self.lib.ftx_trace_replay(self.h, kind.encode(), int(times)))

    def copy(self, dst, src, nbytes):
        self.check(self.lib.ftx_stage(self.h, dst, src, nbytes))

    def buffer(self, nbytes):
        return DeviceBuffer(self, nbytes)

    # ---- tensors ----
    def upload(self, raw, dtype, ne):
        raw = np.ascontiguousarray(raw, np.uint8)
        h = _vp()
        self.check(self.lib.ftx_tensor_upload(self.h, dtype, _ne(ne), 0, raw.ctypes.data,
                                              C.byref(h)))
        return Tensor(self, h.value, dtype, ne)

    def alloc(self, dtype, ne):
        h = _vp()
        self.check(self.lib.ftx_tensor_alloc(self.h, dtype, _ne(ne), C.byref(h)))
        return Tensor(self, h.value, dtype, ne)

    def fill_normal(self, ptr, n, seed, std=1.0, dtype=F32):
        self.check(self.lib.ftx_fill_normal(self.h, ptr, dtype, n, seed, std))

    def quantize(self, src_ptr, t):
        self.check(self.lib.ftx_quantize(self.h, src_ptr, t.handle))

    def dequant(self, t):
        n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]
        out = np.empty(n, np.float32)
        self.check(self.lib.ftx_dequant(self.h, t.handle, out.ctypes.data))
        return out.reshape(-1, t.ne[0])

    # ---- IBackend-level ops on host arrays ----
    def matmul(self, x, t):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        N = t.ne[1] * t.ne[2] * t.ne[3]
        y = np.empty((M, N), np.float32)
        self.check(self.lib.ftx_matmul(self.h, x.ctypes.data, M, K, t.handle, y.ctypes.data))
        return y

    def down_axpy(self, x, t, y=None):
        x = np.ascontiguousarray(x, np.float32)
        M, n_in = x.shape
        N = t.ne[0]
        y = np.zeros((M, N), np.float32) if y is None else np.array(y, np.float32, copy=True)
        self.check(self.lib.ftx_down_axpy(self.h, x.ctypes.data, M, n_in, t.handle,
                                          y.ctypes.data))
        return y

    def expert_chunk(self, x, gate, up, down, out, dt, IC):
        x = np.ascontiguousarray(x, np.float32)
        out = np.array(out, np.float32, copy=True)
        M, K = x.shape
        rb = row_bytes(dt, K)
        j = ExpertJob(x.ctypes.data, out.ctypes.data, gate, up, down, dt, 0, M, K, IC, rb, rb)
        self.check(self.lib.ftx_expert_chunk(self.h, C.byref(j)))
        return out

    # ---- verify path ----
    def model(self, cfg, tensors, max_tokens=64):
        """cfg: dict of hyper-parameters (n_expert / n_expert_used for MoE);
        tensors: name -> Tensor with names tok_embd, out_norm, output
        (optional) and blk.<l>.<role> for the roles of LAYER_TENSORS (the
        dense FFN ones absent on MoE layers) and of LAYER_EXT (optional)."""
        L = cfg["n_layer"]
        nt, nx = len(LAYER_TENSORS), len(LAYER_EXT)
        lay = (_vp * (L * nt))()
        ext = (_vp * (L * nx))()
        has_ext = False
        for l in range(L):
            for i, nm in enumerate(LAYER_TENSORS):
                t = tensors.get("blk.%d.%s" % (l, nm))
                lay[l * nt + i] = t.handle if t is not None else None
            for i, nm in enumerate(LAYER_EXT):
                t = tensors.get("blk.%d.%s" % (l, nm))
                ext[l * nx + i] = t.handle if t is not None else None
                has_ext |= t is not None
        out_t = tensors.get("output")
        d = ModelDesc(cfg["n_layer"], cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"],
                      cfg["head_dim"], cfg["n_ff"], cfg["vocab"], cfg.get("rms_eps", 1e-5),
                      int(cfg.get("rope_neox", 0)), cfg.get("rope_theta", 10000.0),
                      tensors["tok_embd"].handle, tensors["out_norm"].handle,
                      out_t.handle if out_t is not None else None, lay, max_tokens,
                      ext if has_ext else None, cfg.get("n_expert", 0),
                      cfg.get("n_expert_used", 0))
        h = _vp()
        self.check(self.lib.ftx_model_create(self.h, C.byref(d), C.byref(h)))
        return Model(self, h.value, cfg, tensors)

    def argmax_prob(self, row_ptr, V):
        """(first-max token, its T = 1 softmax probability) of a device row."""
        t, p = C.c_int32(0), C.c_float(0)
        self.check(self.lib.ftx_argmax_prob(self.h, row_ptr, V, C.byref(t), C.byref(p)))
        return t.value, p.value

    def accept(self, base_ptr, rows_ptr, M, V, props, mode, temp=1.0, rng=0, parents=None,
               pd=None, q_ptr=None, sampler_state=SAMPLER_SEED, top_k=40, top_p=0.95):
        """ftx_accept; returns accepted node ids, bonus token, the advanced
        acceptance and sampler states and the decision margin.  The sampler
        defaults are the reference's SampleParams (include/ft/sampler.h:10-15)."""
        props = np.ascontiguousarray(props, np.int32)
        par = None if parents is None else np.ascontiguousarray(parents, np.int32)
        pdv = None if pd is None else np.ascontiguousarray(pd, np.float32)
        acc = np.zeros(max(M, 1), np.int32)
        na, bonus, mg = C.c_int32(0), C.c_int32(0), C.c_float(0)
        s = C.c_uint64(rng)
        ss = C.c_uint64(sampler_state)
        a = AcceptArgs(base_ptr, rows_ptr, q_ptr, M, V, props.ctypes.data_as(_i32p),
                       None if par is None else par.ctypes.data_as(_i32p),
                       None if pdv is None else pdv.ctypes.data_as(_fp), mode, temp,
                       C.pointer(s), acc.ctypes.data_as(_i32p), C.pointer(na), C.pointer(bonus),
                       C.pointer(mg), C.pointer(ss), top_k, top_p)
        self.check(self.lib.ftx_accept(self.h, C.byref(a)))
        return dict(accepted=acc[:na.value].tolist(), bonus=bonus.value, rng=s.value,
                    sampler_state=ss.value, margin=mg.value)

    def accept_batch(self, items):
        """ftx_accept_batch over several sequences: items are dicts of
        accept()'s arguments (base_ptr, rows_ptr, M, V, props, mode and the
        optional ones); returns accept()'s result for each, in order."""
        keep, outs = [], []
        args = (AcceptArgs * len(items))()
        for k, it in enumerate(items):
            M, V = it["M"], it["V"]
            props = np.ascontiguousarray(it["props"], np.int32)
            par = it.get("parents")
            par = None if par is None else np.ascontiguousarray(par, np.int32)
            pd = it.get("pd")
            pdv = None if pd is None else np.ascontiguousarray(pd, np.float32)
            acc = np.zeros(max(M, 1), np.int32)
            na, bonus, mg = C.c_int32(0), C.c_int32(0), C.c_float(0)
            s = C.c_uint64(it.get("rng", 0))
            ss = C.c_uint64(it.get("sampler_state", SAMPLER_SEED))
            args[k] = AcceptArgs(it["base_ptr"], it["rows_ptr"], it.get("q_ptr"), M, V,
                                 props.ctypes.data_as(_i32p),
                                 None if par is None else par.ctypes.data_as(_i32p),
                                 None if pdv is None else pdv.ctypes.data_as(_fp), it["mode"],
                                 it.get("temp", 1.0), C.pointer(s), acc.ctypes.data_as(_i32p),
                                 C.pointer(na), C.pointer(bonus), C.pointer(mg), C.pointer(ss),
                                 it.get("top_k", 40), it.get("top_p", 0.95))
            keep += [props, par, pdv]
            outs.append((acc, na, bonus, s, ss, mg))
        self.check(self.lib.ftx_accept_batch(self.h, args, len(items)))
        return [dict(accepted=acc[:na.value].tolist(), bonus=bonus.value, rng=s.value,
                     sampler_state=ss.value, margin=mg.value)
                for acc, na, bonus, s, ss, mg in outs]


class Model:
    def __init__(self, ctx, handle, cfg, tensors):
        self.ctx, self.handle, self.cfg, self.tensors = ctx, handle, cfg, tensors
        # tensors the model owns (freed with it); the device model reads its
        # tensors for its whole life, so the caller's stay alive until free()
        self.owned = []

    def kv(self, cap, kv_dtype=KV_F16):
        h = _vp()
        self.ctx.check(self.ctx.lib.ftx_kv_create(self.ctx.h, self.handle, cap, kv_dtype,
                                                  C.byref(h)))
        return KV(self.ctx, h.value, self.cfg, cap, kv_dtype)

    def verify(self, kv, tokens, logits_ptr, parents=None, advance=False):
        toks = np.ascontiguousarray(tokens, np.int32)
        par = None if parents is None else np.ascontiguousarray(parents, np.int32)
        a = VerifyArgs(toks.size, toks.ctypes.data_as(_i32p),
                       None if par is None else par.ctypes.data_as(_i32p), logits_ptr,
                       int(advance), 0)
        self.ctx.check(self.ctx.lib.ftx_verify_step(self.ctx.h, self.handle, kv.handle,
                                                    C.byref(a)))

    def verify_batch(self, seqs):
        """Several sequences in one step: seqs = [(kv, tokens, logits_ptr,
        parents or None, advance), ...]; each sequence verifies its draft
        against its own cache."""
        keep, arr = [], (SeqArgs * len(seqs))()
        for i, (kv, tokens, logits_ptr, parents, advance) in enumerate(seqs):
            toks = np.ascontiguousarray(tokens, np.int32)
            par = None if parents is None else np.ascontiguousarray(parents, np.int32)
            keep += [toks, par]
            arr[i] = SeqArgs(kv.handle, toks.size, toks.ctypes.data_as(_i32p),
                             None if par is None else par.ctypes.data_as(_i32p), logits_ptr,
                             int(advance), 0)
        self.ctx.check(self.ctx.lib.ftx_verify_batch(self.ctx.h, self.handle, arr, len(seqs)))

    def step(self, kv, token, logits_ptr):
        """Engine::step (src/engine.cpp:650-658): `token` at the committed
        position, its logits row (vocab floats) into logits_ptr, the cache
        one longer."""
        self.verify(kv, [token], logits_ptr, advance=True)

    def prefill(self, kv, tokens, logits_ptr=None, chunk=8):
        """Engine::prefill (src/engine.cpp:598-648, without its prefix
        cache): `tokens` through the model in advancing chains of at most
        `chunk` (the fast path's width); only the last chain runs the LM
        head, and logits_ptr (its len * vocab floats; None: no logits)
        receives its rows.  Returns the number of rows written there."""
        n = len(tokens)
        if n == 0:
            return 0
        for i in range(0, n, chunk):
            part = tokens[i:i + chunk]
            last = i + chunk >= n
            self.verify(kv, part, logits_ptr if last else None, advance=True)
        return len(tokens[(n - 1) // chunk * chunk:])

    def free(self):
        if self.handle:
            self.ctx.lib.ftx_model_free(self.handle)
            self.handle = None
        for t in self.owned:
            t.free()
        self.owned = []


class KV:
    def __init__(self, ctx, handle, cfg, cap, kv_dtype):
        self.ctx, self.handle, self.cap, self.kv_dtype = ctx, handle, cap, kv_dtype
        self.shape = (cfg["n_layer"], cap, cfg["n_head_kv"] * cfg["head_dim"])

    def pointers(self):
        k, v, n = _vp(), _vp(), _i64()
        self.ctx.check(self.ctx.lib.ftx_kv_pointers(self.handle, C.byref(k), C.byref(v),
                                                    C.byref(n)))
        return k.value, v.value, n.value

    def truncate(self, npast):
        self.ctx.check(self.ctx.lib.ftx_kv_truncate(self.handle, npast))

    def commit(self, nodes):
        """Keep the accepted draft path `nodes` (node indices of the last
        verify step) at the next committed slots."""
        arr = (C.c_int32 * max(len(nodes), 1))(*[int(j) for j in nodes])
        self.ctx.check(self.ctx.lib.ftx_kv_commit(self.handle, arr, len(nodes)))

    @property
    def cap_alloc(self):
        return (self.cap + 127) // 128 * 128  # ftx_kv_create's rounding

    def write(self, k, v):
        """Copy host arrays shaped like self.shape (the reference layout)
        into the cache."""
        dt = np.float16 if self.kv_dtype == KV_F16 else np.float32
        k = np.ascontiguousarray(k, dt)
        v = np.ascontiguousarray(v, dt)
        assert k.shape == self.shape and v.shape == self.shape
        self.ctx.check(self.ctx.lib.ftx_kv_write(self.handle, k.ctypes.data, v.ctypes.data))

    def read(self):
        dt = np.float16 if self.kv_dtype == KV_F16 else np.float32
        k = np.empty(self.shape, dt)
        v = np.empty(self.shape, dt)
        self.ctx.check(self.ctx.lib.ftx_kv_read(self.handle, k.ctypes.data, v.ctypes.data))
        return k, v

    def free(self):
        if self.handle:
            self.ctx.lib.ftx_kv_free(self.handle)
            self.handle = None
