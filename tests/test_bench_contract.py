"""bench.py's command-line contract that holds without a GPU."""

from __future__ import annotations

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    """``--gpus N`` with N > 1 exits non-zero before touching a device and
    says why in one JSON line (the build runs on one GPU)."""
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    line = r.stdout.strip().splitlines()[-1]
    msg = json.loads(line)
    assert msg["n_gpus"] == 2 and "one GPU" in msg["error"]
