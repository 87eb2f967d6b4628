"""bench.py's command-line contract on the CPU: one GPU only (N > 1 exits
with a message), and every configuration name parses."""
from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=120)


def test_multi_gpu_request_exits_with_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_help_lists_configs():
    r = _run("--help")
    assert r.returncode == 0
    for name in ("c1", "c2", "c3", "c4step", "c4mod_w4a8", "c5down_w4a8"):
        assert name in r.stdout
