"""bench.py's command-line contract on the CPU: one GPU only (--gpus N > 1 exits with a message before anything
touches a GPU), and the --tp / --config choices it documents."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True, timeout=120,
                       cwd=ROOT, env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_tp_choices():
    r = run_bench("--tp", "3")
    assert r.returncode != 0 and "invalid choice" in r.stderr
    h = run_bench("--help")
    assert h.returncode == 0 and "--tp" in h.stdout and "xover" in h.stdout
