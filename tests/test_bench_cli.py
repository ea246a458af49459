"""bench.py's command line on the host: the one-GPU contract and the diagnostic modes' options,
checked without a device (the refusal happens before anything touches a GPU)."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
BENCH = os.path.join(HERE, "..", "bench.py")


def run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    for n in ("2", "8"):
        r = run("--gpus", n)
        assert r.returncode == 2, (n, r.stdout, r.stderr)
        assert "one GPU" in r.stderr and "--gpus 1" in r.stderr
        assert r.stdout == ""  # no JSON line: nothing was measured


def test_world_size_above_one_is_refused_too():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, BENCH], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_diagnostic_modes_are_listed():
    r = run("--help")
    assert r.returncode == 0
    for opt in ("--q4", "--q4-m", "--dense-gemm", "--model", "--model-matrix", "--timeline", "--copy-calibration"):
        assert opt in r.stdout, opt
