"""bench.py's command-line contract on the CPU: it measures one GPU and says
so (exit status 2, before any device work) when asked for more, and its
options parse."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args, env=None):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, env=env)


def test_more_than_one_gpu_is_refused_with_the_reason():
    r = _bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and r.stdout == ""


def test_a_multi_rank_launch_is_refused_too():
    env = dict(os.environ, WORLD_SIZE="8", RANK="0", LOCAL_RANK="0")
    r = _bench("--gpus", "1", env=env)
    assert r.returncode == 2 and "measures one GPU" in r.stderr


def test_options_parse():
    r = _bench("--help")
    assert r.returncode == 0
    for opt in ("--gpus", "--steps", "--warmup", "--no-cpu", "--no-other", "--no-views", "--only-other"):
        assert opt in r.stdout, opt
