"""bench.py's command-line contract on the host: more than one GPU is refused up front.

The library measures the SpartonHead path on one GPU; `--gpus N` with N > 1, or a launcher's
WORLD_SIZE > 1, must exit with status 2 and a message on stderr before anything touches a
device (the refusal happens before torch is imported, so these run on any host).
"""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.pop("WORLD_SIZE", None)
    if env_extra:
        env.update(env_extra)
    return subprocess.run([sys.executable, BENCH] + args, capture_output=True, text=True,
                          env=env, timeout=120)


def test_more_than_one_gpu_is_refused():
    r = _run(["--gpus", "2"])
    assert r.returncode == 2
    assert r.stdout == ""  # no JSON line
    assert "--gpus 2" in r.stderr and "one GPU" in r.stderr


def test_launcher_world_size_is_refused():
    r = _run(["--gpus", "1"], {"WORLD_SIZE": "4"})
    assert r.returncode == 2
    assert r.stdout == ""
    assert "WORLD_SIZE=4" in r.stderr


def test_help_lists_the_contract_flags():
    r = _run(["--help"])
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--config"):
        assert flag in r.stdout
