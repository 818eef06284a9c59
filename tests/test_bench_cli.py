"""bench.py's command line on the CPU: it refuses more than one GPU before
touching any, and every secondary config is reachable through --config."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT, capture_output=True,
                          text=True, timeout=120)


def test_more_than_one_gpu_is_refused_with_exit_code_2():
    out = _run("--gpus", "2")
    assert out.returncode == 2
    assert "one GPU" in out.stderr and out.stdout == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="2")
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], cwd=ROOT, capture_output=True, text=True,
                         timeout=120, env=env)
    assert out.returncode == 2


def test_every_secondary_config_is_a_config_choice():
    sys.path.insert(0, ROOT)
    import bench
    out = _run("--help")
    assert out.returncode == 0
    for name in bench.SECONDARY_CONFIGS:
        assert name in out.stdout.replace("\n", "").replace(" ", "")
