"""Row 137 with the fused finish (SILVANN_GFX950_DECODE_FUSED=1: the last split of each row and head block merges
the others, no merge launch). The switch is read once a process, so the whole decode suite (tests/test_gpu_decode.py:
the oracle, the torch fp32 reference, zero-length rows, the closed forms, page-table bit-exactness, determinism)
runs again in a child process with it on.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

HERE = Path(__file__).resolve().parent


def test_decode_suite_with_fused_finish(dev):
    print("case: tests/test_gpu_decode.py with SILVANN_GFX950_DECODE_FUSED=1 (child process)", flush=True)
    cmd = [sys.executable, "-u", "-m", "pytest", str(HERE / "test_gpu_decode.py"), "-m", "gpu", "-x", "-q",
           "-p", "no:cacheprovider"]
    r = subprocess.run(cmd, cwd=str(HERE.parent), env={**os.environ, "SILVANN_GFX950_DECODE_FUSED": "1"},
                       capture_output=True, text=True, timeout=600)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
