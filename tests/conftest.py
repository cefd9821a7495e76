import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import ORACLE_SO, Oracle
    if not ORACLE_SO.exists():
        import subprocess
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "oracle"], check=True)
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.oracle import RefFamily, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref/libsilvann_x86_avx2.so not built (needs /root/reference): make -C oracle ref")
    return RefFamily()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import silvann_amd
    silvann_amd.lib()   # fails loudly if the library is not built
    return torch.device("cuda:0")


def parity(got, want, atol=2e-3, cos_min=0.9999):
    """The north star's bar on fp16 outputs: max-abs <= 2e-3 and cosine >= 0.9999."""
    g = np.asarray(got, dtype=np.float64).ravel()
    w = np.asarray(want, dtype=np.float64).ravel()
    assert g.shape == w.shape
    assert np.all(np.isfinite(g)), "non-finite output"
    err = float(np.max(np.abs(g - w))) if g.size else 0.0
    denom = np.linalg.norm(g) * np.linalg.norm(w)
    cos = float(np.dot(g, w) / denom) if denom > 0 else (1.0 if err == 0 else 0.0)
    assert err <= atol, f"max-abs {err:.3e} > {atol}"
    assert cos >= cos_min, f"cosine {cos:.6f} < {cos_min}"
    return err, cos
