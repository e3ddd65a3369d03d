"""bench.py's command-line contract on the CPU: the single-GPU refusal (no
GPU is touched before it) and the argument set the driver and the profile
commands use."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120)


def test_multi_gpu_refused_with_a_message():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "single MI355X" in r.stderr and "--gpus 1" in r.stderr


def test_world_size_above_one_refused():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True,
                       text=True, timeout=120, env=env)
    assert r.returncode == 2


def test_help_lists_the_profile_switches():
    r = run("--help")
    assert r.returncode == 0
    for flag in ("--steps", "--warmup", "--gpus", "--no-decode", "--no-cpu-baseline",
                 "--no-grouped", "--no-quantize", "--decode-only", "--calibrate-copy"):
        assert flag in r.stdout, flag
