"""A GGUF file through the loaders to the device, on the GPU: the Python
loader (xwfes_amd.gguf.load_model) and the C++ one (Gguf ->
weights_from_gguf -> HipVerifier, run by tests/cpp/test_hip_backend
--gguf), each verify step against the oracle's forward of the same weights
(logits within 1e-3 relative per row, as for the verify step itself)."""
import os
import subprocess

import numpy as np
import pytest

import pyoracle as P
from xwfes_amd import ftx
from xwfes_amd import gguf as G

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_hip_backend")
LOGIT_TOL = 1e-3

MOE_DT = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q8_0, k=P.Q8_0, v=P.Q8_0, o=P.Q8_0,
              gate_inp=P.F32, gate_exps=P.Q4_0, up_exps=P.Q4_0, down_exps=P.Q4_0,
              gate_sh=P.Q8_0, up_sh=P.Q8_0, down_sh=P.Q8_0)
MODELS = {
    # reference dtypes, the reference's [d, 1, V] embedding layout
    "tiny": (P.model_cfg(2, 64, 4, 2, 16, 96, 50, rope_theta=10000.0),
             dict(tok_embd=P.F32, output=P.Q4_1, q=P.Q4_0, k=P.Q8_0, v=P.Q4_0, o=P.Q8_0,
                  gate=P.Q4_0, up=P.Q4_0, down=P.Q8_0), {}, ()),
    # K-quants on the MFMA paths (head_dim 128), neox rotation by arch name
    "kquant": (P.model_cfg(2, 1024, 8, 2, 128, 1024, 1000, rope_theta=500000.0, rope_neox=1),
               dict(tok_embd=P.Q4_K, output=P.Q6_K, q=P.Q4_K, k=P.Q4_K, v=P.Q6_K, o=P.Q4_K,
                    gate=P.Q4_K, up=P.Q4_K, down=P.Q6_K), dict(arch="qwen2"), ()),
    # MoE (8 experts, top-2) with a router bias and a shared expert
    "moe": (P.model_cfg(2, 256, 4, 2, 64, 256, 300, n_expert=8, n_expert_used=2), MOE_DT, {},
            ("router_bias", "gate_sh", "up_sh", "down_sh")),
    # q / k / v bias and per-head q / k norms, neox by arch name
    "qwen": (P.model_cfg(2, 256, 4, 2, 64, 512, 300, rope_neox=1),
             dict(MOE_DT, gate=P.Q8_0, up=P.Q8_0, down=P.Q4_0), dict(arch="qwen3"),
             ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm")),
}


def write(tmp_path, orc, name, seed=4):
    cfg, dts, kvo, extras = MODELS[name]
    model = P.make_model(orc, cfg, dts, seed=seed, extras=extras)
    path = str(tmp_path / (name + ".gguf"))
    G.write_gguf(path, G.model_kv(cfg, **kvo), G.model_tensor_list(model))
    return path, model


def rel_err_rows(a, b):
    a = np.atleast_2d(a).astype(np.float64)
    b = np.atleast_2d(b).astype(np.float64)
    return (np.abs(a - b).max(axis=1) / np.maximum(np.abs(b).max(axis=1), 1e-30)).max()


@pytest.mark.parametrize("name", sorted(MODELS))
def test_python_loader_verify(gctx, orc, tmp_path, name):
    path, model = write(tmp_path, orc, name)
    gm, cfg = G.load_model(gctx, path, max_tokens=8)
    assert cfg["rope_neox"] == model["cfg"]["rope_neox"]
    cap, npast = 160, 70
    kv = gm.kv(cap)
    rng = np.random.default_rng(3)
    shape = kv.shape
    k0 = np.zeros(shape, np.float16)
    v0 = np.zeros(shape, np.float16)
    k0[:, :npast] = rng.standard_normal((shape[0], npast, shape[2]))
    v0[:, :npast] = rng.standard_normal((shape[0], npast, shape[2]))
    V = cfg["vocab"]
    buf = gctx.buffer(8 * V * 4)
    toks = [1, V - 1, 7, 0, 3, 11]
    for parents in (None, [-1, 0, 0, 1, 2, 2]):
        kv.write(k0, v0)
        kv.truncate(npast)
        gm.verify(kv, toks, buf.ptr, parents=parents)
        gctx.sync()
        got = buf.read(np.float32, len(toks) * V).reshape(len(toks), V)
        want = orc.forward(model, k0.copy(), v0.copy(), npast, toks, parents=parents)
        assert rel_err_rows(got, want) < LOGIT_TOL, parents
    buf.free()
    kv.free()
    gm.free()


def test_cpp_loader_verify(tmp_path, orc):
    assert os.path.exists(BIN), "build the package first (tests/cpp/test_hip_backend missing)"
    paths = [write(tmp_path, orc, name, seed=6)[0] for name in sorted(MODELS)]
    r = subprocess.run([BIN, "--gguf"] + paths, capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert r.stdout.count("verified") == len(paths) and "checks passed" in r.stdout
