"""bench.py's command line on the CPU: the run on more than one GPU is refused with a message
before anything touches torch or a GPU (this build measures one GPU)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1"],
                       capture_output=True, text=True, timeout=60, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line


def test_bench_rejects_unknown_section():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--only", "ffn"],
                       capture_output=True, text=True, timeout=60, cwd=ROOT)
    assert r.returncode != 0
    assert "invalid choice" in r.stderr
