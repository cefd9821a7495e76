"""Row 137 with each of its opt-in forms, the candidates for its default:

- SILVANN_GFX950_DECODE_FUSED=1: the last split of each row and head block merges the others (no merge launch);
- SILVANN_GFX950_DECODE_INLINE=1: each workgroup makes the plan itself at batches of at most 64 rows (no plan launch);
- both of those: one launch a step, the finished-split counts tagged with the call's tag instead of cleared;
- SILVANN_GFX950_DECODE_VTR=1: the V^T operand through the transposing LDS read at head_dim <= 256;
- SILVANN_GFX950_DECODE_LATENT=wide: latent attention (head_dim 512, keys the values) with a workgroup's four waves
  over four head blocks of one split, sharing its tiles (decode_latent).

A switch is read once a process, so the whole decode suite (tests/test_gpu_decode.py: the oracle, the torch fp32
reference, zero-length rows, the closed forms, page-table bit-exactness, determinism) runs again in a child process
with it on — and with the inline plan, which the deferred chains' fused routes take too, the chain and latent suites.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

HERE = Path(__file__).resolve().parent


SUITES = {   # name: (switches, suites)
    "fused": ({"SILVANN_GFX950_DECODE_FUSED": "1"}, ["test_gpu_decode.py"]),
    "inline": ({"SILVANN_GFX950_DECODE_INLINE": "1"}, ["test_gpu_decode.py", "test_gpu_chains.py", "test_gpu_latent.py"]),
    "one-launch": ({"SILVANN_GFX950_DECODE_FUSED": "1", "SILVANN_GFX950_DECODE_INLINE": "1"},
                   ["test_gpu_decode.py", "test_gpu_chains.py"]),
    "vtr": ({"SILVANN_GFX950_DECODE_VTR": "1"}, ["test_gpu_decode.py"]),
    "latent-wide": ({"SILVANN_GFX950_DECODE_LATENT": "wide"}, ["test_gpu_latent.py"]),
}


@pytest.mark.timeout(400)
@pytest.mark.parametrize("name", list(SUITES))
def test_decode_suite_with(dev, name):
    switches, files = SUITES[name]
    print(f"case: {' '.join(files)} with {switches} (child process)", flush=True)
    cmd = [sys.executable, "-u", "-m", "pytest", *[str(HERE / f) for f in files], "-m", "gpu", "-x", "-q",
           "-p", "no:cacheprovider", "--timeout", "120", "--timeout-method", "thread"]
    r = subprocess.run(cmd, cwd=str(HERE.parent), env={**os.environ, **switches},
                       capture_output=True, text=True, timeout=360)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
