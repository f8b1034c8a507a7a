"""bench.py's command line on the CPU: a request for several GPUs ends with
a message and exit status 2 before any device work, and the workload table
names every workload the measurement notes list."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_several_gpus_refused_with_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout == ""


def test_workload_table():
    sys.path.insert(0, ROOT)
    try:
        import bench
    finally:
        sys.path.pop(0)
    names = set(bench.WORKLOADS)
    assert "llama3-8b-q4km-k8-ctx2048" in names
    for n in ("llama3-8b-q8attn-tree52-ctx4096", "llama3-8b-q8attn-tree32-ctx4096",
              "mixtral-8x7b-q4_0-k8x4-ctx1024", "llama3-70b-q4k-tree64x4-ctx8192",
              "llama3-8b-q4km-decode-ctx2048", "llama3-8b-q4km-prefill-512",
              "llama3-8b-q4km+1b-draft-spec4", "tinyllama-q4_0+1l-draft-spec4"):
        assert n in names, n
    for n, w in bench.WORKLOADS.items():
        assert w["kind"] in ("verify", "tree", "batch", "decode", "prefill", "generate"), n
        assert w["ctx"] >= 0 and w["M"] >= 1, n
