"""CPU: bench.py's command-line contract that needs no GPU.

One process per GPU is not part of this build: `--gpus N` above 1 must stop
with a message saying so (and a nonzero status) before any device work.
"""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
    assert '"metric"' not in r.stdout  # no bench line
