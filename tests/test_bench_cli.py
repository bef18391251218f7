"""bench.py's command line on the CPU: the one-GPU build refuses a multi-GPU run with a
message and exit status 2 before it touches a device, and its help names every section."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT, timeout=120,
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def test_bench_refuses_more_than_one_gpu():
    r = _run("--gpus", "2")
    assert r.returncode == 2, r.stdout
    assert "one GPU only" in r.stdout


def test_bench_help_lists_sections():
    r = _run("--help")
    assert r.returncode == 0, r.stdout
    for section in ("gemm_q6k", "gemm_q80", "q4_k_m", "q8_0_model", "decode_eager"):
        assert section in r.stdout, section
