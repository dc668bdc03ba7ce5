"""bench.py's command-line contract, on the CPU: more than one GPU is refused with a message before
any GPU work, and every kernel choice the docs name is accepted."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=300, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    out = run("--gpus", "2")
    assert out.returncode == 2
    assert "one GPU" in out.stderr
    assert out.stdout == ""


def test_world_size_above_one_exits_too():
    env = dict(os.environ, WORLD_SIZE="2")
    out = subprocess.run([sys.executable, BENCH], capture_output=True, text=True, timeout=300, cwd=ROOT, env=env)
    assert out.returncode == 2
    assert "one GPU" in out.stderr


def test_help_lists_every_kernel_choice():
    out = run("--help")
    assert out.returncode == 0
    for choice in ("plan", "scalar", "valu", "wide_b"):
        assert choice in out.stdout
