"""bench.py's command-line contract that needs no GPU: it measures one GPU
and refuses a multi-GPU request before touching a device."""

from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1"],
                         capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert res.returncode == 2
    assert res.stdout == ""
    assert "measures one GPU" in res.stderr and "--gpus 1" in res.stderr
