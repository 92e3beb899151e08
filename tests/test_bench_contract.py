"""bench.py's command-line contract on the CPU: one GPU only, so --gpus N > 1
exits with a message and a non-zero status before touching a device."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120, cwd=REPO)
    assert proc.returncode != 0
    assert "one GPU only" in proc.stdout + proc.stderr
    assert proc.stdout.strip() == "" or not proc.stdout.lstrip().startswith("{"), "no JSON line for --gpus 2"
