"""causal_pipe (SILVANN_GFX950_PREFILL=pipe), the head_dim-256 prefill kernel with a deeper K/V ring: the whole
prefill suite (tests/test_gpu_prefill.py) in a child process with the switch on. Not collected until it has passed on
a GPU once: run it by naming this file."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

HERE = Path(__file__).resolve().parent


@pytest.mark.timeout(400)
def test_prefill_suite_with_pipe(dev):
    print("case: test_gpu_prefill.py with SILVANN_GFX950_PREFILL=pipe (child process)", flush=True)
    cmd = [sys.executable, "-u", "-m", "pytest", str(HERE / "test_gpu_prefill.py"), "-m", "gpu", "-x", "-v",
           "-p", "no:cacheprovider", "--timeout", "120", "--timeout-method", "thread"]
    r = subprocess.run(cmd, cwd=str(HERE.parent), env={**os.environ, "SILVANN_GFX950_PREFILL": "pipe"},
                       capture_output=True, text=True, timeout=360)
    print(r.stdout[-6000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
