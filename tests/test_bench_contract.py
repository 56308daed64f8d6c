"""bench.py's command-line contract on the CPU: more than one GPU is refused with a
message and exit status 2 before anything touches a GPU or imports torch."""

import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120, cwd=REPO)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout == ""
