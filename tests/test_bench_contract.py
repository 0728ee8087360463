"""The benchmark's command-line contract that needs no GPU: more than one GPU is refused with a
message (the path is measured on one MI355X), before anything touches a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args, capture_output=True,
                          text=True, timeout=120, env=env)


def test_more_than_one_gpu_is_refused():
    r = _run(["--gpus", "2"])
    assert r.returncode == 2
    assert "single GPU" in r.stderr and r.stdout == ""


def test_distributed_launch_is_refused():
    r = _run(["--gpus", "1"], {"WORLD_SIZE": "4"})
    assert r.returncode == 2 and r.stdout == ""
