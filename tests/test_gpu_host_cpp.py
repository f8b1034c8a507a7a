"""The C++ host mirror (HipBackend / HipVerifier, xwfes_amd/host/) on the GPU:
runs tests/cpp/test_hip_backend, which checks IBackend::matmul,
run_expert_chunk, the reference's greedy-acceptance known answer, and a
2-layer chain / tree verify plus greedy / ratio acceptance, and a
two-sequence HipVerifier::verify_batch (HipSequence), against the oracle
(tests/cpp/test_hip_backend.cpp)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_hip_backend")


@pytest.mark.gpu
def test_cpp_host_mirror():
    assert os.path.exists(BIN), "build the package first (tests/cpp/test_hip_backend missing)"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert "all" in r.stdout and "checks passed" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("eos_at", [None, 6])
@pytest.mark.parametrize("temp", [0.0, 0.7])
@pytest.mark.parametrize("same_draft", [True, False])
def test_cpp_generate_equals_oracle(tmp_path, orc, temp, same_draft, eos_at):
    """Speculative generate through the C++ host path (GGUF files -> C++
    loader -> HipVerifier target and draft -> DraftModelDrafter + generate,
    xwfes_amd/host/hip_backend.cpp) emits the oracle's tokens and statistics
    (pyoracle.Oracle.generate, pinned against the reference's generate in
    tests/test_spec.py), greedy and sampled, draft equal to and different
    from the target; with eos_at, the target file's
    tokenizer.ggml.eos_token_id is the token the run without one emits at
    that position, and both loops stop there as the reference's does."""
    import numpy as np
    import pyoracle as P
    from xwfes_amd import gguf as G
    cfg = P.model_cfg(2, 64, 4, 2, 16, 96, 48, rope_theta=10000.0)
    dts = dict(tok_embd=P.F32, output=P.Q8_0, q=P.Q8_0, k=P.Q8_0, v=P.Q8_0, o=P.Q8_0,
               gate=P.Q8_0, up=P.Q8_0, down=P.Q8_0)

    def peaked(seed, gain):  # a sharp output distribution, so drafts get accepted
        m = P.make_model(orc, cfg, dts, seed=seed)
        m["out_norm"]["raw"] = np.full(cfg["n_embd"], gain, np.float32).view(np.uint8).copy()
        return m

    target = peaked(31, 30.0)
    draft = target if same_draft else peaked(32, 25.0)
    prompt = [3, 17, 5, 40, 11, 9, 30, 2, 21]
    cap, max_new, k = 128, 30, 4
    eos = -1
    if eos_at is not None:
        full, _ = orc.generate(target, draft, prompt, max_new, spec_k=k, temp=temp, cap=cap)
        eos = full[eos_at]
    paths = []
    for name, m in (("target", target), ("draft", draft)):
        p = str(tmp_path / (name + ".gguf"))
        G.write_gguf(p, G.model_kv(cfg, eos=eos if eos >= 0 else None), G.model_tensor_list(m))
        paths.append(p)
    r = subprocess.run([BIN, "--generate", paths[0], paths[1], str(temp), str(k), str(max_new),
                        str(cap)] + [str(t) for t in prompt], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0, r.stderr
    lines = {ln.split(":")[0]: ln.split(":")[1].split() for ln in r.stdout.splitlines() if ":" in ln}
    got = [int(t) for t in lines["generate tokens"]]
    rounds, drafted, accepted, hit = (int(v) for v in lines["generate stats"])
    want, st = orc.generate(target, draft, prompt, max_new, spec_k=k, temp=temp, cap=cap, eos=eos)
    assert got == want
    assert (rounds, drafted, accepted, bool(hit)) == (st["rounds"], st["drafted"],
                                                       st["accepted"], st["hit_eos"])
    assert drafted > 0 and (accepted > 0 or not same_draft)
    if eos_at is not None:
        assert hit and eos in got and len(got) <= eos_at + k + 1
