"""GGUF on-disk boundary of the verify path: reader, writer, model config
and device upload.

Reader semantics follow the reference's parser (src/gguf.cpp:168-245):
little-endian GGUF v2 / v3, metadata values of the 13 GGUF kinds (arrays of
strings or numbers), tensor infos of 1-4 dims, data start aligned to
general.alignment (default 32; a value that is not a power of two falls back
to 32), tensor data at data_start + offset with bounds checks.  Its typed
accessors keep the reference's behaviour (src/gguf.cpp:247-345): get_i64 of
a float or bool key is 0, get_f64 of an integer key is its value, a missing
key returns the default.  The tensor dtypes are the reference's (F32, F16,
Q4_0, Q4_1, Q8_0, BF16, src/gguf.cpp:129-137) plus the public GGUF K-quants
Q4_K (12) and Q6_K (14), which the reference rejects at load.

config_from_gguf restates src/graph.cpp:24-80 (including its reading of the
RMSNorm epsilon through the integer accessor, so that a float-typed key
leaves the default 1e-5) and the n_ff / vocab fallbacks of Engine::load
(src/engine.cpp:282-396).  The file is memory-mapped; the loader hands the
mapped bytes to the device upload, so host memory holds one copy at most.
"""
import mmap
import os
import struct

import numpy as np

GGUF_MAGIC = 0x46554747
(T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64,
 T_F64) = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
           T_F32: "<f", T_BOOL: "<B", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
_NP = {T_U8: np.uint8, T_I8: np.int8, T_U16: np.uint16, T_I16: np.int16, T_U32: np.uint32,
       T_I32: np.int32, T_F32: np.float32, T_BOOL: np.uint8, T_U64: np.uint64,
       T_I64: np.int64, T_F64: np.float64}
_INT_KINDS = (T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_U64, T_I64)

# dtype id -> (elements per block, bytes per block); ids are the GGUF type ids
F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20),
         Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
DTYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q8_0: "Q8_0",
               Q4_K: "Q4_K", Q6_K: "Q6_K", BF16: "BF16"}


class GgufError(ValueError):
    pass


def row_bytes(dtype, ncols):
    """Bytes of one row of ncols elements (include/ft/types.h:47-51)."""
    if dtype not in BLOCK:
        raise GgufError("unsupported tensor dtype %d" % dtype)
    eb, bb = BLOCK[dtype]
    return (ncols + eb - 1) // eb * bb


class TensorInfo:
    __slots__ = ("name", "n_dims", "ne", "dtype", "offset", "nbytes")

    def __init__(self, name, n_dims, ne, dtype, offset, nbytes):
        self.name, self.n_dims, self.ne, self.dtype = name, n_dims, ne, dtype
        self.offset, self.nbytes = offset, nbytes

    @property
    def rows(self):
        """Rows of the tensor seen as a matrix of ne[0] columns: every
        plane's rows in order (ne[1] * ne[2] * ne[3])."""
        return self.ne[1] * self.ne[2] * self.ne[3]


class _Reader:
    def __init__(self, buf):
        self.b, self.off = buf, 0

    def need(self, n):
        if self.off + n > len(self.b):
            raise GgufError("gguf: truncated file")

    def scalar(self, fmt):
        n = struct.calcsize(fmt)
        self.need(n)
        v = struct.unpack_from(fmt, self.b, self.off)[0]
        self.off += n
        return v

    def string(self):
        n = self.scalar("<Q")
        self.need(n)
        s = bytes(self.b[self.off:self.off + n]).decode("utf-8", "surrogateescape")
        self.off += n
        return s

    def value(self, kind):
        if kind == T_STR:
            return self.string()
        if kind == T_ARR:
            ek = self.scalar("<I")
            n = self.scalar("<Q")
            if ek == T_STR:
                return (ek, [self.string() for _ in range(n)])
            if ek not in _NP:
                raise GgufError("gguf: unsupported array element type")
            nb = n * np.dtype(_NP[ek]).itemsize
            self.need(nb)
            a = np.frombuffer(self.b, _NP[ek], n, self.off).copy()
            self.off += nb
            return (ek, a)
        if kind not in _SCALAR:
            raise GgufError("gguf: unsupported kv type")
        v = self.scalar(_SCALAR[kind])
        return bool(v) if kind == T_BOOL else v


class GgufFile:
    """A memory-mapped GGUF file: metadata `kv` (key -> (kind, value)) and
    tensor infos `tensors` (name -> TensorInfo, offset from the file start)."""

    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            if size < 24:
                raise GgufError("gguf: empty or tiny file")
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self.size = size
        r = _Reader(memoryview(self._mm))
        if r.scalar("<I") != GGUF_MAGIC:
            raise GgufError("not a GGUF file")
        self.version = r.scalar("<I")
        if self.version not in (2, 3):
            raise GgufError("unsupported GGUF version %d" % self.version)
        n_tensors = r.scalar("<Q")
        n_kv = r.scalar("<Q")
        self.kv = {}
        for _ in range(n_kv):
            key = r.string()
            kind = r.scalar("<I")
            val = (kind, r.value(kind))
            self.kv.setdefault(key, val)  # a repeated key keeps its first value
        align = 32
        if "general.alignment" in self.kv:
            align = self.get_i64("general.alignment")
        if align <= 0 or align & (align - 1):
            align = 32
        self.alignment = align
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            n_dims = r.scalar("<i")
            if n_dims < 1 or n_dims > 4:
                raise GgufError("gguf: bad dims for " + name)
            ne = [1, 1, 1, 1]
            for d in range(n_dims):
                ne[d] = r.scalar("<Q")
            dtype = r.scalar("<I")
            if dtype not in BLOCK:
                raise GgufError("gguf: unsupported tensor dtype %d" % dtype)
            infos.append((name, n_dims, tuple(ne), dtype, r.scalar("<Q")))
        pos = (r.off + align - 1) // align * align
        if pos > size:
            raise GgufError("gguf: data out of bounds")
        self.data_start = pos
        self.tensors = {}
        for name, n_dims, ne, dtype, off in infos:
            if name in self.tensors:
                continue  # a repeated name keeps its first info
            nbytes = row_bytes(dtype, ne[0]) * ne[1] * ne[2] * ne[3]
            if off > size - pos or nbytes > size - pos - off:
                raise GgufError("gguf: tensor out of bounds: " + name)
            self.tensors[name] = TensorInfo(name, n_dims, ne, dtype, pos + off, nbytes)

    def close(self):
        """Unmap the file (left to the garbage collector while a view of
        its bytes is alive)."""
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:
                pass
            self._mm = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- typed accessors (src/gguf.cpp:247-345)
    def has(self, key):
        return key in self.kv

    def get_str(self, key, default=""):
        k = self.kv.get(key)
        return k[1] if k is not None and k[0] == T_STR else default

    def get_i64(self, key, default=0):
        k = self.kv.get(key)
        if k is None:
            return default
        kind, v = k
        if kind in _INT_KINDS:
            return int(v)
        if kind == T_STR:
            return default
        return 0  # float, bool and array values hold no integer

    def get_f64(self, key, default=0.0):
        k = self.kv.get(key)
        if k is None:
            return default
        kind, v = k
        if kind in (T_F32, T_F64):
            return float(v)
        if kind == T_STR:
            return default
        return float(int(v)) if kind in _INT_KINDS else 0.0

    def get_bool(self, key, default=False):
        k = self.kv.get(key)
        return bool(k[1]) if k is not None and k[0] == T_BOOL else default

    def get_str_arr(self, key):
        k = self.kv.get(key)
        if k is None or k[0] != T_ARR or k[1][0] != T_STR:
            return []
        return list(k[1][1])

    def get_f32_arr(self, key):
        """Numeric arrays as float32; string and bool arrays read as zeros
        of their length (src/gguf.cpp:288-330)."""
        k = self.kv.get(key)
        if k is None or k[0] != T_ARR:
            return np.zeros(0, np.float32)
        ek, items = k[1]
        if ek in (T_STR, T_BOOL):
            return np.zeros(len(items), np.float32)
        return np.asarray(items).astype(np.float32)

    def get_i32_arr(self, key):
        return self.get_f32_arr(key).astype(np.int32)

    def tensor(self, name):
        return self.tensors.get(name)

    def data(self, name):
        """The tensor's bytes as a read-only uint8 view of the mapping."""
        t = self.tensors[name]
        return np.frombuffer(self._mm, np.uint8, t.nbytes, t.offset)


# ---------------------------------------------------------------- config

_NEOX_ARCHS = ("qwen", "deepseek", "phi", "glm", "minicpm")


def _kv_i(g, arch, suffixes, default):
    """src/graph.cpp:9-21: the arch's key, then the llama.* key."""
    for prefix in (arch, "llama"):
        for s in suffixes:
            v = g.get_i64(prefix + "." + s, None)
            if v is not None:
                return v
    return default


def config_from_gguf(g):
    """Model config (pyoracle.model_cfg keys plus arch, ctx_train, moe).
    src/graph.cpp:24-80 with the n_ff / vocab fallbacks of Engine::load."""
    arch = g.get_str("general.architecture", "unknown")
    n_layer = _kv_i(g, arch, ["block_count"], 0)
    n_embd = _kv_i(g, arch, ["embedding_length"], 0)
    n_head = _kv_i(g, arch, ["attention.head_count"], 0)
    n_head_kv = _kv_i(g, arch, ["attention.head_count_kv"], n_head)
    head_dim = _kv_i(g, arch, ["attention.key_length", "attention.head_dim"],
                     n_embd // n_head if n_head else 0)
    vocab = _kv_i(g, arch, ["vocab_size"], 0)
    if not vocab:
        vocab = len(g.get_str_arr("tokenizer.ggml.tokens"))
    ctx_train = _kv_i(g, arch, ["context_length"], 4096)
    # the epsilon goes through the integer accessor (src/graph.cpp:42-43): a
    # float-typed key reads as 0 and the default applies
    eps = float(_kv_i(g, arch, ["attention.layer_norm_rms_epsilon"], 0))
    if not eps:
        eps = 1e-5
    theta = g.get_f64(arch + ".rope.freq_base", 0.0)
    if not theta:
        theta = g.get_f64("llama.rope.freq_base", 10000.0)
    n_experts = _kv_i(g, arch, ["expert_count"], 0)
    n_expert_used = _kv_i(g, arch, ["expert_used_count"], 0)
    neox = any(s in arch.lower() for s in _NEOX_ARCHS)
    n_ff = _kv_i(g, arch, ["expert_feed_forward_length", "feed_forward_length"], 0)
    if not (n_layer and n_embd and n_head and head_dim and vocab):
        raise GgufError("gguf: incomplete model config for arch " + arch)
    moe = n_experts > 1 and n_expert_used > 0
    return dict(arch=arch, n_layer=n_layer, n_embd=n_embd, n_head=n_head, n_head_kv=n_head_kv,
                head_dim=head_dim, n_ff=n_ff, vocab=vocab, ctx_train=ctx_train,
                rms_eps=np.float32(eps).item(), rope_theta=float(theta), rope_neox=int(neox),
                moe=int(moe), n_expert=n_experts if moe else 0,
                n_expert_used=n_expert_used if moe else 0)


# tensor names tried per role, first found wins (src/engine.cpp:320-395)
LAYER_NAMES = {
    "attn_norm": ["blk.%d.attn_norm.weight", "blk.%d.input_layernorm.weight"],
    "q": ["blk.%d.attn_q.weight", "blk.%d.self_attn.q_proj.weight"],
    "k": ["blk.%d.attn_k.weight", "blk.%d.self_attn.k_proj.weight"],
    "v": ["blk.%d.attn_v.weight", "blk.%d.self_attn.v_proj.weight"],
    "o": ["blk.%d.attn_output.weight", "blk.%d.self_attn.o_proj.weight"],
    "ffn_norm": ["blk.%d.post_attention_norm.weight", "blk.%d.post_attention_layernorm.weight",
                 "blk.%d.ffn_norm.weight"],
    "gate": ["blk.%d.ffn_gate.weight", "blk.%d.mlp.gate_proj.weight"],
    "up": ["blk.%d.ffn_up.weight", "blk.%d.mlp.up_proj.weight"],
    "down": ["blk.%d.ffn_down.weight", "blk.%d.mlp.down_proj.weight"],
}
# optional layer tensors, by the roles of ftx.LAYER_EXT (src/engine.cpp:325-369)
EXT_NAMES = {
    "q_bias": ["blk.%d.attn_q.bias"], "k_bias": ["blk.%d.attn_k.bias"],
    "v_bias": ["blk.%d.attn_v.bias"],
    "q_norm": ["blk.%d.attn_q_norm.weight", "blk.%d.self_attn.q_norm.weight"],
    "k_norm": ["blk.%d.attn_k_norm.weight", "blk.%d.self_attn.k_norm.weight"],
    "gate_inp": ["blk.%d.ffn_gate_inp.weight"], "gate_exps": ["blk.%d.ffn_gate_exps.weight"],
    "up_exps": ["blk.%d.ffn_up_exps.weight"], "down_exps": ["blk.%d.ffn_down_exps.weight"],
    "router_bias": ["blk.%d.exp_probs_b.bias"], "gate_sh": ["blk.%d.ffn_gate_shexp.weight"],
    "up_sh": ["blk.%d.ffn_up_shexp.weight"], "down_sh": ["blk.%d.ffn_down_shexp.weight"],
}
MOE_ROLES = ("gate_inp", "gate_exps", "up_exps", "down_exps", "router_bias", "gate_sh", "up_sh",
             "down_sh")
EXPERT_PLANES = ("gate_exps", "up_exps", "down_exps")


def model_tensors(g, cfg):
    """The model's tensors by role: name -> (TensorInfo, ne), ne the upload
    shape: ne0 columns of all the tensor's rows (the reference's 3-D
    embedding layout [d, 1, V] is V rows of d), except expert planes, which
    keep (ne0, rows, n_expert).  MoE as Engine::load decides it
    (src/engine.cpp:318-387): from the metadata, or from the first layer
    with a router and expert planes (every later layer is then MoE); a MoE
    layer has no dense FFN tensors.  Fills cfg n_ff, n_expert and
    n_expert_used the way Engine::load does when the metadata has none."""
    out = {}

    def take(role, t, planes=False):
        out[role] = (t, (t.ne[0], t.ne[1], t.ne[2]) if planes else (t.ne[0], t.rows))

    def first(names, l):
        return next((g.tensor(n % l) for n in names if g.tensor(n % l)), None)

    moe = bool(cfg.get("moe"))
    for l in range(cfg["n_layer"]):
        ext = {role: first(names, l) for role, names in EXT_NAMES.items()}
        if not moe and ext["gate_inp"] is not None and ext["gate_exps"] is not None:
            moe = True
        for role, names in LAYER_NAMES.items():
            if moe and role in ("gate", "up", "down"):
                continue
            t = first(names, l)
            if t is None:
                raise GgufError("gguf: missing %s tensor at layer %d" % (role, l))
            take("blk.%d.%s" % (l, role), t)
        if moe:
            if any(ext[r] is None for r in ("gate_inp", "gate_exps", "up_exps", "down_exps")):
                raise GgufError("gguf: incomplete MoE tensors at layer %d" % l)
            if not cfg.get("n_expert"):
                E = ext["gate_exps"].ne[2]
                cfg["n_expert"], cfg["n_expert_used"] = E, (8 if E >= 8 else 2)
            if not cfg["n_ff"]:
                cfg["n_ff"] = ext["gate_exps"].ne[1]
        for role, t in ext.items():
            if t is None or (role in MOE_ROLES and not moe):
                continue
            take("blk.%d.%s" % (l, role), t, planes=role in EXPERT_PLANES)
    if not moe:
        cfg["n_expert"] = cfg["n_expert_used"] = 0
    cfg["moe"] = int(moe)
    emb = g.tensor("token_embd.weight")
    if emb is None:
        raise GgufError("gguf: missing token_embd.weight")
    take("tok_embd", emb)
    on = g.tensor("output_norm.weight")
    if on is None:
        raise GgufError("gguf: missing output_norm.weight")
    take("out_norm", on)
    outw = g.tensor("output.weight")
    take("output", outw if outw is not None else emb)  # tied embeddings
    if not cfg["n_ff"] and "blk.0.gate" in out:
        cfg["n_ff"] = out["blk.0.gate"][1][1]
    return out


def load_model(ctx, path, max_tokens=8):
    """Open `path`, upload its weights to the device of `ctx` and build the
    resident model.  Returns (model, cfg); the model owns the uploaded
    tensors (model.free() releases them) and the mapping is closed on
    return (the device holds its own copies)."""
    with GgufFile(path) as g:
        cfg = config_from_gguf(g)
        roles = model_tensors(g, cfg)
        tensors = {}
        try:
            for role, (t, ne) in roles.items():
                if role == "output" and t.name == "token_embd.weight":
                    continue  # tied: the model reads tok_embd
                tensors[role] = ctx.upload(g.data(t.name), t.dtype, ne)
            model = ctx.model(cfg, tensors, max_tokens=max_tokens)
        except BaseException:
            for t in tensors.values():
                t.free()
            raise
    model.owned = list(tensors.values())
    return model, cfg


# ---------------------------------------------------------------- writer

def _pack_value(kind, v):
    if kind == T_STR:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if kind == T_ARR:
        ek, items = v
        if ek == T_STR:
            return struct.pack("<IQ", ek, len(items)) + b"".join(_pack_value(T_STR, s) for s in items)
        a = np.ascontiguousarray(items, _NP[ek])
        return struct.pack("<IQ", ek, a.size) + a.tobytes()
    return struct.pack(_SCALAR[kind], int(v) if kind == T_BOOL else v)


def write_gguf(path, kv, tensors, alignment=32, version=3):
    """Write a GGUF file.  kv: list of (key, kind, value), array values as
    (element kind, list or array); tensors: list of (name, dtype, ne,
    bytes) with ne = (ne0, ne1[, ne2[, ne3]]) and the bytes in ggml row
    order.  Tensor data are placed at `alignment`-aligned offsets; an
    alignment other than the default 32 is recorded as general.alignment."""
    kv = list(kv)
    for key, kind, v in kv:
        if key == "general.alignment" and v != alignment:
            raise GgufError("general.alignment %r differs from the data alignment %d" % (v, alignment))
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in kv):
        kv.append(("general.alignment", T_U32, alignment))
    head = [struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(kv))]
    for key, kind, v in kv:
        head.append(_pack_value(T_STR, key) + struct.pack("<I", kind) + _pack_value(kind, v))
    off = 0
    placed = []
    for name, dtype, ne, data in tensors:
        data = bytes(data)
        ne = tuple(int(x) for x in ne)
        full = ne + (1,) * (4 - len(ne))
        want = row_bytes(dtype, full[0]) * full[1] * full[2] * full[3]
        if len(data) != want:
            raise GgufError("%s: %d bytes, shape needs %d" % (name, len(data), want))
        off = (off + alignment - 1) // alignment * alignment
        head.append(_pack_value(T_STR, name) + struct.pack("<i", len(ne)) +
                    b"".join(struct.pack("<Q", x) for x in ne) + struct.pack("<IQ", dtype, off))
        placed.append((off, data))
        off += len(data)
    blob = b"".join(head)
    start = (len(blob) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(blob + b"\0" * (start - len(blob)))
        pos = 0
        for o, data in placed:
            f.write(b"\0" * (o - pos))
            f.write(data)
            pos = o + len(data)


def model_kv(cfg, arch="llama", tokens=None, float_eps=True, eos=None):
    """Metadata for a model of `cfg` (pyoracle.model_cfg keys).  The
    epsilon is written as a float, as GGUF converters write it (the
    reference then keeps its default), or as an integer key when
    float_eps is False; eos: the tokenizer's end-of-sequence id
    (tokenizer.ggml.eos_token_id), none when None."""
    a = arch
    kv = [("general.architecture", T_STR, a),
          (a + ".block_count", T_U32, cfg["n_layer"]),
          (a + ".embedding_length", T_U32, cfg["n_embd"]),
          (a + ".attention.head_count", T_U32, cfg["n_head"]),
          (a + ".attention.head_count_kv", T_U32, cfg["n_head_kv"]),
          (a + ".attention.key_length", T_U32, cfg["head_dim"]),
          (a + ".feed_forward_length", T_U32, cfg["n_ff"]),
          (a + ".context_length", T_U32, 4096),
          (a + ".vocab_size", T_U32, cfg["vocab"]),
          (a + ".rope.freq_base", T_F32, float(cfg["rope_theta"]))]
    if float_eps:
        kv.append((a + ".attention.layer_norm_rms_epsilon", T_F32, float(cfg["rms_eps"])))
    if cfg.get("n_expert"):
        kv.append((a + ".expert_count", T_U32, cfg["n_expert"]))
        kv.append((a + ".expert_used_count", T_U32, cfg["n_expert_used"]))
    if tokens is None:
        tokens = ["<t%d>" % i for i in range(cfg["vocab"])]
    kv.append(("tokenizer.ggml.model", T_STR, "llama"))
    kv.append(("tokenizer.ggml.tokens", T_ARR, (T_STR, tokens)))
    if eos is not None:
        kv.append(("tokenizer.ggml.eos_token_id", T_U32, int(eos)))
    return kv


# model-dict role -> GGUF tensor name (the llama.cpp names)
GGUF_NAMES = {"attn_norm": "attn_norm.weight", "q": "attn_q.weight", "k": "attn_k.weight",
              "v": "attn_v.weight", "o": "attn_output.weight", "ffn_norm": "ffn_norm.weight",
              "gate": "ffn_gate.weight", "up": "ffn_up.weight", "down": "ffn_down.weight",
              "q_bias": "attn_q.bias", "k_bias": "attn_k.bias", "v_bias": "attn_v.bias",
              "q_norm": "attn_q_norm.weight", "k_norm": "attn_k_norm.weight",
              "gate_inp": "ffn_gate_inp.weight", "gate_exps": "ffn_gate_exps.weight",
              "up_exps": "ffn_up_exps.weight", "down_exps": "ffn_down_exps.weight",
              "router_bias": "exp_probs_b.bias", "gate_sh": "ffn_gate_shexp.weight",
              "up_sh": "ffn_up_shexp.weight", "down_sh": "ffn_down_shexp.weight"}


def model_tensor_list(model, embd_3d=True, bias_2d=True):
    """GGUF tensor list of a pyoracle-style model dict (name -> {raw,
    dtype, ne0, ne1}).  embd_3d writes the token embedding as [d, 1, V]
    (the layout the reference's plane lookup reads as rows).  Expert planes
    are written as [d, rows, n_expert].  bias_2d writes a bias of n values as
    [1, n]: the reference takes a bias's length from ne[1]
    (src/engine.cpp:334-339), which reads a one-dimensional [n] bias as a
    single value."""
    E = model["cfg"].get("n_expert", 0)
    out = []
    for name, t in model.items():
        if name == "cfg":
            continue
        ne = (t["ne0"], t["ne1"])
        if name == "tok_embd":
            gname = "token_embd.weight"
            if embd_3d:
                ne = (t["ne0"], 1, t["ne1"])
        elif name == "out_norm":
            gname, ne = "output_norm.weight", (t["ne0"],)
        elif name == "output":
            gname = "output.weight"
        else:
            blk, l, role = name.split(".")
            gname = "blk.%s.%s" % (l, GGUF_NAMES[role])
            if role.endswith("norm"):
                ne = (t["ne0"],)
            elif role.endswith("bias"):
                ne = (1, t["ne0"]) if bias_2d else (t["ne0"],)
            elif role.endswith("_exps"):
                ne = (t["ne0"], t["ne1"] // E, E)
        out.append((gname, t["dtype"], ne, np.ascontiguousarray(t["raw"]).tobytes()))
    return out


def tensor_hash(b):
    """sum_i b[i] * ((i + 1) * 0x9E3779B97F4A7C15) mod 2^64 over the bytes b."""
    b = np.asarray(b, np.uint8).astype(np.uint64)
    w = (np.arange(1, b.size + 1, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15))
    with np.errstate(over="ignore"):
        return int((b * w).sum(dtype=np.uint64))


def summary(g, offsets=True, keys=None):
    """Canonical text summary: the config, the typed accessors of `keys`
    (default: every key, sorted) and every tensor (sorted), with its file
    offset (offsets=True) or a hash of its bytes (offsets=False).  The C++
    parser and the reference's parser print the same form."""
    lines = []
    try:
        c = config_from_gguf(g)
        lines.append("config arch=%s n_layer=%d n_embd=%d n_head=%d n_head_kv=%d head_dim=%d "
                     "vocab=%d n_ff=%d ctx_train=%d rms_eps=%.9g rope_theta=%.17g rope_neox=%d"
                     % (c["arch"], c["n_layer"], c["n_embd"], c["n_head"], c["n_head_kv"],
                        c["head_dim"], c["vocab"], c["n_ff"], c["ctx_train"], c["rms_eps"],
                        c["rope_theta"], c["rope_neox"]))
    except GgufError:
        lines.append("config error")
    for key in (sorted(g.kv) if keys is None else keys):
        f32 = g.get_f32_arr(key)
        lines.append("kv %s has=%d i64=%d f64=%.17g str=%s bool=%d nstr=%d nf32=%d hf32=%d" % (
            key, int(g.has(key)), g.get_i64(key, -7), g.get_f64(key, -7.0), g.get_str(key, "-"),
            int(g.get_bool(key, False)), len(g.get_str_arr(key)), f32.size,
            tensor_hash(np.ascontiguousarray(f32, np.float32).view(np.uint8))))
    for name in sorted(g.tensors):
        t = g.tensors[name]
        where = ("offset=%d" % t.offset) if offsets else ("hash=%d" % tensor_hash(g.data(name)))
        lines.append("tensor %s n_dims=%d ne=%d,%d,%d,%d dtype=%d nbytes=%d %s" % (
            name, t.n_dims, t.ne[0], t.ne[1], t.ne[2], t.ne[3], t.dtype, t.nbytes, where))
    return "\n".join(lines) + "\n"
