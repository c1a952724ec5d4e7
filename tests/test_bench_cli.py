"""bench.py's command line on the CPU: a run on more than one GPU is refused
with a message (this build measures one GPU), and every measured leg is a
selectable config.  Nothing here touches a GPU."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_every_leg_is_a_config():
    r = _run("--help")
    assert r.returncode == 0
    for cfg in ("decode", "indexer", "prefill", "fwdbwd", "paged", "dash", "page", "kl", "blockmax", "copycal"):
        assert cfg in r.stdout
