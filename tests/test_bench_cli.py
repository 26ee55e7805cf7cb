"""bench.py's command line on the CPU: more than one GPU is refused with a message (one GPU per
box; the line's value is one GPU's throughput), before any device work."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr) and r.stdout.strip() == ""
