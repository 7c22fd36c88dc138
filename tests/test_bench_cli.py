"""bench.py's command-line contract that needs no GPU: it measures one GPU
and refuses a multi-GPU request with exit status 2 and a message."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_bench_refuses_more_than_one_gpu():
    result = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True, timeout=120
    )
    assert result.returncode == 2
    assert "one GPU only" in result.stderr
    assert result.stdout == ""
