"""bench.py's command-line contract on the CPU: one GPU only (a multi-GPU request exits with a message
and status 2, before any GPU work), and the documented modes are known to its argument parser."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args, env=None):
    e = dict(os.environ)
    if env:
        e.update(env)
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          env=e, timeout=120)


def test_multi_gpu_request_exits_with_a_message():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_world_size_above_one_exits_with_a_message():
    r = run_bench("--gpus", "1", env={"WORLD_SIZE": "2"})
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_help_lists_the_modes():
    r = run_bench("--help")
    assert r.returncode == 0
    for flag in ("--steps", "--warmup", "--only", "--read-sweep", "--dispatch-floor", "--timeline", "--no-cpu", "--no-extras"):
        assert flag in r.stdout
