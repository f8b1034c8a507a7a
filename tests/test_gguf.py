"""The GGUF boundary (xwfes_amd/gguf.py, xwfes_amd/host/gguf.cpp) on the CPU.

Pinned three ways on files written by the package's own writer:
- the C++ parser and the Python reader print the same canonical summary
  (config, every typed accessor of every key, every tensor's offset and
  bytes);
- the reference's own parser (src/gguf.cpp, src/graph.cpp, compiled into
  oracle/_ref) prints the same summary for every file whose dtypes it
  accepts, including its quirks (the RMSNorm epsilon read through the
  integer accessor, numeric accessors of float and bool keys, string-array
  floats, repeated keys);
- the reference Engine loaded from the file (src/engine.cpp:282-396) steps
  through tokens to the oracle's forward logits exactly.
Malformed files are rejected by all three.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

import pyoracle as P
from xwfes_amd import gguf as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SUMMARY_BIN = os.path.join(ROOT, "tests", "cpp", "gguf_summary")

TINY = P.model_cfg(2, 64, 4, 2, 16, 96, 50, rope_theta=10000.0)
TINY_DT = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q4_0, k=P.Q8_0, v=P.Q4_0, o=P.Q8_0,
               gate=P.Q4_0, up=P.Q4_1, down=P.Q8_0)
KQ = P.model_cfg(1, 256, 4, 2, 64, 512, 300, rope_theta=500000.0)
KQ_DT = dict(tok_embd=P.Q4_K, output=P.Q6_K, q=P.Q4_K, k=P.Q4_K, v=P.Q6_K, o=P.Q4_K,
             gate=P.Q4_K, up=P.Q4_K, down=P.Q6_K)


def cpp_summary(path, hashes=False):
    assert os.path.exists(SUMMARY_BIN), "build the package first (tests/cpp/gguf_summary missing)"
    args = [SUMMARY_BIN, path] + (["--hash"] if hashes else [])
    r = subprocess.run(args, capture_output=True, text=True)
    return r.returncode, r.stdout


def write_model(path, orc, cfg, dts, seed, **kv_opts):
    model = P.make_model(orc, cfg, dts, seed=seed)
    G.write_gguf(path, G.model_kv(cfg, **kv_opts), G.model_tensor_list(model))
    return model


def odd_kv():
    """Metadata of every kind, arrays of every element kind, a repeated key,
    an integer-typed epsilon and a missing rope base."""
    kv = [("general.architecture", G.T_STR, "foo"),
          ("llama.block_count", G.T_U16, 2), ("llama.embedding_length", G.T_I64, 64),
          ("llama.attention.head_count", G.T_I8, 4), ("foo.attention.head_count_kv", G.T_U64, 2),
          ("llama.feed_forward_length", G.T_I16, 96),
          ("foo.attention.layer_norm_rms_epsilon", G.T_U32, 2),
          ("k.u8", G.T_U8, 250), ("k.i8", G.T_I8, -5), ("k.u16", G.T_U16, 65535),
          ("k.i16", G.T_I16, -300), ("k.u32", G.T_U32, 4000000000), ("k.i32", G.T_I32, -7),
          ("k.f32", G.T_F32, 1.25), ("k.bool", G.T_BOOL, True), ("k.str", G.T_STR, "hello"),
          ("k.u64", G.T_U64, 2**40 + 3), ("k.i64", G.T_I64, -2**40), ("k.f64", G.T_F64, -2.5e-7),
          ("k.str", G.T_STR, "second value of a repeated key"),
          ("tokenizer.ggml.tokens", G.T_ARR, (G.T_STR, ["<t%d>" % i for i in range(50)]))]
    for ek, vals in ((G.T_U8, [1, 255]), (G.T_I8, [-1, 3]), (G.T_U16, [9, 60000]),
                     (G.T_I16, [-9, 7]), (G.T_U32, [5, 3000000000]), (G.T_I32, [-5, 5]),
                     (G.T_F32, [0.5, -1.5e3]), (G.T_BOOL, [1, 0, 1]), (G.T_U64, [2**35, 1]),
                     (G.T_I64, [-2**35, 2]), (G.T_F64, [1e-3, 7.0])):
        kv.append(("arr.%d" % ek, G.T_ARR, (ek, vals)))
    return kv


def make_files(tmp_path, orc):
    """name -> (path, whether the reference accepts its dtypes)."""
    files = {}
    p = str(tmp_path / "tiny.gguf")
    write_model(p, orc, TINY, TINY_DT, 3)
    files["tiny"] = (p, True)
    p = str(tmp_path / "kq.gguf")
    write_model(p, orc, KQ, KQ_DT, 4)
    files["kquant"] = (p, False)
    p = str(tmp_path / "qwen.gguf")
    m = P.make_model(orc, TINY, TINY_DT, seed=5)
    G.write_gguf(p, G.model_kv(TINY, arch="qwen2", float_eps=False), G.model_tensor_list(m),
                 alignment=64)
    files["qwen_align64"] = (p, True)
    p = str(tmp_path / "odd.gguf")
    G.write_gguf(p, odd_kv(), G.model_tensor_list(m, embd_3d=False), version=2)
    files["odd_v2"] = (p, True)
    return files


def test_writer_reader_roundtrip(tmp_path, orc):
    p = str(tmp_path / "m.gguf")
    model = write_model(p, orc, TINY, TINY_DT, 7)
    with G.GgufFile(p) as g:
        cfg = G.config_from_gguf(g)
        for key in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "vocab"):
            assert cfg[key] == TINY[key], key
        assert cfg["rope_theta"] == TINY["rope_theta"] and cfg["rope_neox"] == 0
        roles = G.model_tensors(g, cfg)
        for name, t in model.items():
            if name == "cfg":
                continue
            info, ne = roles[name]
            assert (ne, info.dtype) == ((t["ne0"], t["ne1"]), t["dtype"]), name
            assert np.array_equal(g.data(info.name), np.ascontiguousarray(t["raw"]).view(np.uint8).ravel())
        assert all(t.offset % 32 == 0 for t in g.tensors.values())


def test_cpp_parser_matches_python(tmp_path, orc):
    for name, (p, _) in make_files(tmp_path, orc).items():
        with G.GgufFile(p) as g:
            rc, text = cpp_summary(p)
            assert rc == 0 and text == G.summary(g), name
            rc, text = cpp_summary(p, hashes=True)
            assert rc == 0 and text == G.summary(g, offsets=False), name


def test_reference_parser_matches(tmp_path, orc, ref):
    for name, (p, ref_ok) in make_files(tmp_path, orc).items():
        with G.GgufFile(p) as g:
            got = ref.gguf_summary(p, sorted(g.kv))
            if ref_ok:
                assert got == G.summary(g, offsets=False), name
            else:  # K-quant dtypes: the reference rejects the file at load
                assert got[0] == "error" and "unsupported tensor dtype" in got[1], name


def test_config_rules(tmp_path, orc):
    files = make_files(tmp_path, orc)
    with G.GgufFile(files["qwen_align64"][0]) as g:
        c = G.config_from_gguf(g)
        assert g.alignment == 64 and c["rope_neox"] == 1 and c["rms_eps"] == np.float32(1e-5)
    with G.GgufFile(files["odd_v2"][0]) as g:
        c = G.config_from_gguf(g)
        # llama.* fallbacks, integer epsilon, head_dim = n_embd / n_head,
        # vocab from the token list, default rope base
        assert (c["arch"], c["n_layer"], c["n_embd"], c["n_head"], c["n_head_kv"]) == ("foo", 2, 64, 4, 2)
        assert (c["head_dim"], c["vocab"], c["n_ff"], c["rms_eps"], c["rope_theta"]) == (16, 50, 96, 2.0, 10000.0)
        assert g.get_str("k.str") == "hello"  # a repeated key keeps its first value
        assert g.get_i64("k.f32", 9) == 0 and g.get_f64("k.u64") == float(2**40 + 3)
        assert g.get_i64("k.bool", 9) == 0 and g.get_bool("k.bool") is True
        assert np.array_equal(g.get_f32_arr("arr.%d" % G.T_BOOL), np.zeros(3, np.float32))
        assert g.get_f32_arr("tokenizer.ggml.tokens").size == 50
        assert g.tensor("token_embd.weight").n_dims == 2


def _corrupt(path, out, edit):
    b = bytearray(open(path, "rb").read())
    edit(b)
    open(out, "wb").write(bytes(b))


def test_malformed_files_rejected(tmp_path, orc, request):
    good = str(tmp_path / "good.gguf")
    write_model(good, orc, TINY, TINY_DT, 9)
    size = os.path.getsize(good)
    with G.GgufFile(good) as g:
        first = min(g.tensors.values(), key=lambda t: t.offset)
        # the first tensor info: name length, name, n_dims, ne..., dtype, offset
        hdr = open(good, "rb").read()
    name_at = hdr.index(b"blk.0.attn_norm.weight") - 8
    n_dims_at = name_at + 8 + len("blk.0.attn_norm.weight")
    dtype_at = n_dims_at + 4 + 8  # 1-D tensor
    off_at = dtype_at + 4
    cases = {
        "truncated": lambda b: b.__delitem__(slice(size - 100, size)),
        "magic": lambda b: b.__setitem__(slice(0, 4), b"GGUX"),
        "version": lambda b: b.__setitem__(slice(4, 8), struct.pack("<I", 4)),
        "n_dims": lambda b: b.__setitem__(slice(n_dims_at, n_dims_at + 4), struct.pack("<i", 5)),
        "dtype": lambda b: b.__setitem__(slice(dtype_at, dtype_at + 4), struct.pack("<I", 7)),
        "offset": lambda b: b.__setitem__(slice(off_at, off_at + 8), struct.pack("<Q", size)),
        "kv_kind": lambda b: b.__setitem__(slice(24 + 8 + len("general.architecture"),
                                                 24 + 12 + len("general.architecture")),
                                           struct.pack("<I", 13)),
        "tiny": lambda b: b.__delitem__(slice(20, size)),
    }
    have_ref = P.Ref.available()
    refl = P.Ref() if have_ref else None
    for name, edit in cases.items():
        p = str(tmp_path / ("bad_%s.gguf" % name))
        _corrupt(good, p, edit)
        with pytest.raises((G.GgufError, ValueError)):
            G.GgufFile(p)
        rc, text = cpp_summary(p)
        assert rc == 1 and text.startswith("error"), (name, text)
        # the reference's unsigned size check (src/gguf.cpp:236-238) wraps for
        # an offset past the end of the file, so it accepts that file and
        # would read past its mapping: that case is not handed to it
        if refl is not None and name != "offset":
            got = refl.gguf_summary(p, [])
            assert isinstance(got, tuple) and got[0] == "error", name
    assert first.offset > 0


def test_model_tensors_refuses_what_it_cannot_run(tmp_path, orc):
    m = P.make_model(orc, TINY, TINY_DT, seed=2)
    tl = G.model_tensor_list(m)
    p = str(tmp_path / "missing.gguf")
    G.write_gguf(p, G.model_kv(TINY), [t for t in tl if t[0] != "blk.1.ffn_up.weight"])
    with G.GgufFile(p) as g:
        with pytest.raises(G.GgufError, match="missing up tensor at layer 1"):
            G.model_tensors(g, G.config_from_gguf(g))
    # MoE by its metadata, without expert tensors (src/engine.cpp:353-356)
    p = str(tmp_path / "moe.gguf")
    G.write_gguf(p, G.model_kv(TINY) + [("llama.expert_count", G.T_U32, 8),
                                         ("llama.expert_used_count", G.T_U32, 2)], tl)
    with G.GgufFile(p) as g:
        with pytest.raises(G.GgufError, match="incomplete MoE tensors at layer 0"):
            G.model_tensors(g, G.config_from_gguf(g))


MOE_DT = dict(TINY_DT, gate_inp=P.F32, gate_exps=P.Q4_0, up_exps=P.Q4_0, down_exps=P.Q4_0,
              gate_sh=P.Q8_0, up_sh=P.Q8_0, down_sh=P.Q8_0)


def test_model_tensors_moe_and_extras(tmp_path, orc):
    """Router, expert planes (three dims), router bias, shared expert and
    the attention extras come back by role with their shapes; without the
    expert keys the expert count comes from the planes and the routed count
    defaults as Engine::load does (8 of >= 8 experts, else 2)."""
    cfg = P.model_cfg(2, 64, 4, 2, 16, 32, 50, n_expert=4, n_expert_used=3)
    ex = ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm", "router_bias", "gate_sh", "up_sh",
          "down_sh")
    m = P.make_model(orc, cfg, MOE_DT, seed=3, extras=ex)
    for keys, want_u in ((True, 3), (False, 2)):
        kv = G.model_kv(cfg)
        if not keys:
            kv = [k for k in kv if "expert" not in k[0]]
        p = str(tmp_path / ("m%d.gguf" % keys))
        G.write_gguf(p, kv, G.model_tensor_list(m))
        with G.GgufFile(p) as g:
            c = G.config_from_gguf(g)
            roles = G.model_tensors(g, c)
        assert (c["n_expert"], c["n_expert_used"], c["moe"]) == (4, want_u, 1)
        assert "blk.0.gate" not in roles
        assert roles["blk.1.gate_exps"][1] == (64, 32, 4)
        assert roles["blk.1.down_exps"][1] == (64, 32, 4)
        assert roles["blk.0.gate_inp"][1] == (64, 4)
        assert roles["blk.0.q_bias"][1] == (1, 64)  # the reference's [1, n] layout
        assert roles["blk.0.k_norm"][1] == (16, 1)
        assert roles["blk.1.down_sh"][1] == (64, 32)
    # a dense model keeps the attention extras
    d = P.make_model(orc, TINY, TINY_DT, seed=4, extras=("q_norm", "k_norm"))
    p = str(tmp_path / "dense.gguf")
    G.write_gguf(p, G.model_kv(TINY), G.model_tensor_list(d))
    with G.GgufFile(p) as g:
        c = G.config_from_gguf(g)
        roles = G.model_tensors(g, c)
    assert c["n_expert"] == 0 and "blk.1.q_norm" in roles and "blk.1.gate" in roles


def test_reference_engine_steps_equal_oracle_forward(tmp_path, orc, ref):
    """The reference Engine loaded from the file, stepped token by token
    (fp32 KV cache), against the oracle's block forward of the same tokens:
    identical logits (both run the reference's loop order in fp32)."""
    for cfg, dts, seed in ((TINY, TINY_DT, 3),
                           (P.model_cfg(3, 128, 8, 2, 16, 160, 70, rope_theta=500000.0),
                            dict(TINY_DT, q=P.Q8_0, tok_embd=P.F32, up=P.F16, gate=P.BF16), 11)):
        p = str(tmp_path / ("eng%d.gguf" % seed))
        model = write_model(p, orc, cfg, dts, seed)
        toks = [3, 17, 42, 0, 9, cfg["vocab"] - 1, 5]
        h = ref.engine_load(p, 1, 64)
        try:
            rows = [ref.engine_step(h, t) for t in toks]
        finally:
            ref.engine_free(h)
        shape = (cfg["n_layer"], 64, cfg["n_head_kv"] * cfg["head_dim"])
        want = orc.forward(model, np.zeros(shape, np.float32), np.zeros(shape, np.float32), 0, toks)
        for i, r in enumerate(rows):
            err = np.abs(r - want[i]).max() / np.abs(want[i]).max()
            assert err <= 1e-6, (seed, i, err)


def test_writer_regenerates_reference_test_model(tmp_path):
    """The package's writer reproduces the reference's own test model byte
    for byte (src/tests/test_core.cpp:79-213: qwen3moe, L 2, D 16, 4 / 2
    heads of 4, 4 experts of FFN 32, vocabulary 27, F32 tensors, norms 1,
    every other weight rnd() * 0.3 from the test's LCG, 32-byte alignment).
    The reference's build writes that file as build/ft_test_model.gguf:
    62240 bytes, sha256 4a024de1...7753."""
    import hashlib
    L, D, H, KVH, HD, E, FF, V = 2, 16, 4, 2, 4, 4, 32, 27
    kv = [("general.architecture", G.T_STR, "qwen3moe"),
          ("qwen3moe.block_count", G.T_U32, L),
          ("qwen3moe.embedding_length", G.T_U32, D),
          ("qwen3moe.attention.head_count", G.T_U32, H),
          ("qwen3moe.attention.head_count_kv", G.T_U32, KVH),
          ("qwen3moe.attention.key_length", G.T_U32, HD),
          ("qwen3moe.context_length", G.T_U32, 128),
          ("qwen3moe.attention.layer_norm_rms_epsilon", G.T_F32, 1e-5),
          ("qwen3moe.rope.freq_base", G.T_F32, 10000.0),
          ("tokenizer.ggml.model", G.T_STR, "llama"),
          ("tokenizer.ggml.tokens", G.T_ARR, (G.T_STR, ["<pad>"] + [chr(c) for c in range(97, 123)])),
          ("tokenizer.ggml.bos_token_id", G.T_I32, -1),
          ("tokenizer.ggml.eos_token_id", G.T_I32, -1)]
    shapes = [("token_embd.weight", (D, V)), ("output_norm.weight", (D,)), ("output.weight", (D, V))]
    for l in range(L):
        p = "blk.%d." % l
        shapes += [(p + "attn_norm.weight", (D,)), (p + "attn_q.weight", (D, H * HD)),
                   (p + "attn_k.weight", (D, KVH * HD)), (p + "attn_v.weight", (D, KVH * HD)),
                   (p + "attn_output.weight", (H * HD, D)), (p + "attn_q_norm.weight", (HD,)),
                   (p + "attn_k_norm.weight", (HD,)), (p + "post_attention_norm.weight", (D,)),
                   (p + "ffn_gate_inp.weight", (D, E)), (p + "ffn_gate_exps.weight", (D, FF, E)),
                   (p + "ffn_up_exps.weight", (D, FF, E)), (p + "ffn_down_exps.weight", (D, FF, E))]
    state = [123456789]

    def rnd():  # g = g * 1664525 + 1013904223 (mod 2^32); uniform in [-1, 1) in float
        state[0] = (state[0] * 1664525 + 1013904223) & 0xFFFFFFFF
        return np.float32((state[0] >> 9) & 0x7FFF) / np.float32(32768) * np.float32(2) - np.float32(1)

    tensors = []
    for name, ne in shapes:
        n = int(np.prod(ne))
        if "norm" in name:
            vals = np.ones(n, np.float32)
        else:
            vals = np.array([rnd() * np.float32(0.3) for _ in range(n)], np.float32)
        tensors.append((name, G.F32, ne, vals.tobytes()))
    path = str(tmp_path / "ft_test_model.gguf")
    G.write_gguf(path, kv, tensors)
    blob = open(path, "rb").read()
    assert len(blob) == 62240
    assert hashlib.sha256(blob).hexdigest() == \
        "4a024de1c8b1e9bc554cefaf211710c9384f3155833fb95518695fb0c8747753"
