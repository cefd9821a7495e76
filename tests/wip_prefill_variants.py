"""Row 138 with each of its opt-in head_dim-256 kernels (SILVANN_GFX950_PREFILL), the candidates for its default:

- pipe: causal_pipe, one wave a SIMD, software-pipelined two tiles deep with K and V rings of their own;
- duo: causal_duo, two waves a SIMD over alternate key tiles, merged through LDS (head_dim 128 and 256), for row 138
  and, in its residual form, row 140 (the tiered prefill window's suite, tests/test_gpu_window.py).

The switch is read once a process, so each suite runs in a child process with it on. Not collected until it has
passed on a GPU: run it by naming this file."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

HERE = Path(__file__).resolve().parent


@pytest.mark.timeout(400)
@pytest.mark.parametrize("kernel,suite", [("duo", "test_gpu_prefill.py"), ("pipe", "test_gpu_prefill.py"),
                                          ("duo", "test_gpu_window.py")])
def test_prefill_suite_with(dev, kernel, suite):
    print(f"case: {suite} with SILVANN_GFX950_PREFILL={kernel} (child process)", flush=True)
    cmd = [sys.executable, "-u", "-m", "pytest", str(HERE / suite), "-m", "gpu", "-x", "-v",
           "-p", "no:cacheprovider", "--timeout", "120", "--timeout-method", "thread"]
    r = subprocess.run(cmd, cwd=str(HERE.parent),
                       env={**os.environ, "SILVANN_GFX950_PREFILL": kernel, "SILVANN_GPU_UNVERIFIED": "1"},
                       capture_output=True, text=True, timeout=360)
    print(r.stdout[-6000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
