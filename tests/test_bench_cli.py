"""bench.py's command-line contract on CPU: one GPU only (--gpus N > 1 exits
with a message), and the workloads it accepts."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=REPO)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_workload_choices():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--help"], capture_output=True, text=True,
                       timeout=300, cwd=REPO)
    assert r.returncode == 0
    for w in ("c1", "c2", "c3", "c4", "c5", "boundary", "server"):
        assert w in r.stdout
