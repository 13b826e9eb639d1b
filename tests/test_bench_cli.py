"""CPU: bench.py's command-line contract that needs no GPU -- more than one
GPU is refused with a message and a non-zero status (this build measures one
GPU), and --help lists the workloads."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_help_lists_workloads():
    r = _run("--help")
    assert r.returncode == 0
    for w in ("decode", "prefill", "splitk", "harness", "norms", "model", "chunked", "ceilings"):
        assert w in r.stdout
