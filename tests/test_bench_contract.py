"""bench.py's command-line contract on the CPU: more than one GPU is refused
with a message before anything touches a device."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=REPO)


def test_more_than_one_gpu_is_refused():
    for n in ("2", "8"):
        r = _bench("--gpus", n, "--steps", "1", "--warmup", "0")
        assert r.returncode == 2, r.stderr
        assert r.stdout == ""                      # no JSON line
        assert "one GPU only" in r.stderr


def test_help_lists_the_driver_flags():
    r = _bench("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in r.stdout
