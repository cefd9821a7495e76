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


# GPU suites whose kernels have passed on an MI355X run first, so that under `pytest -x` a failure in a newer suite
# cannot hide their results; the rest keep their collection order after them.
GPU_FIRST = ("test_gpu_decode.py", "test_gpu_doors.py", "test_gpu_prefill.py")
# The opt-in variants of the decode (candidates for its default, not paths a caller gets) run after every suite of
# a path a caller gets, so that a failure among them cannot hide those suites' results either.
GPU_LAST = ("test_gpu_decode_variants.py",)


# GPU suites whose kernels have never run on an MI355X (checked only in the CPU emulation of tests/emu). A first run
# of a new kernel can fault the GPU and end the process, and with it every result of the session, so these are
# skipped unless SILVANN_GPU_UNVERIFIED=1: a builder's session runs each of them once, on its own, and a suite
# leaves this list when it has passed there.
GPU_UNVERIFIED = ("test_gpu_tq.py", "test_gpu_window.py", "test_gpu_cache.py", "test_gpu_latent.py",
                  "test_gpu_chains.py", "test_gpu_family.py", "test_gpu_softmax_sink.py", "test_gpu_rows_pairs.py",
                  "test_gpu_decode_variants.py")

_current = {"test": "(collecting)"}


def pytest_sessionstart(session):
    """Under `-m gpu`: a heartbeat file, gpurun_out/pytest_heartbeat.txt, rewritten every 20 s with the running test
    and its time so far, so a long test (a child-process suite, whose output pytest holds until it ends) shows
    progress to a run that watches for silence."""
    if (session.config.option.markexpr or "").strip() != "gpu":
        return
    import threading
    import time
    out = ROOT / "gpurun_out"

    def beat():
        t0, last = time.time(), None
        while True:
            test = _current["test"]
            if test != last:
                t_test, last = time.time(), test
            try:
                out.mkdir(exist_ok=True)
                (out / "pytest_heartbeat.txt").write_text(
                    f"{time.time() - t0:.0f} s into the session; {test} for {time.time() - t_test:.0f} s\n")
            except OSError:
                return
            time.sleep(20)

    threading.Thread(target=beat, daemon=True, name="pytest-heartbeat").start()


def pytest_runtest_logstart(nodeid, location):
    _current["test"] = nodeid


def pytest_collection_modifyitems(config, items):
    def rank(item):
        name = Path(str(item.fspath)).name
        if name in GPU_FIRST:
            return GPU_FIRST.index(name)
        return len(GPU_FIRST) + (1 + GPU_LAST.index(name) if name in GPU_LAST else 0)
    items[:] = sorted(items, key=rank)
    if os.environ.get("SILVANN_GPU_UNVERIFIED") != "1":
        skip = pytest.mark.skip(reason="kernels not yet run on an MI355X (CPU emulation only): run this suite once "
                                       "with SILVANN_GPU_UNVERIFIED=1")
        for item in items:
            if Path(str(item.fspath)).name in GPU_UNVERIFIED:
                item.add_marker(skip)


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


def residual_parity(got, want, hd):
    """Residuals {m, l, acc} a (row, head) against the oracle's: m (the largest scaled score) to fp32 rounding of
    the scores, which go through the matrix cores from fp16 operands; l and acc, at the oracle's m (a residual is
    defined up to a common factor e^m, which attention_merge takes as it comes), to the weights' fp16 rounding;
    and the answers acc / l to the fp16 bar."""
    w = hd + 2
    g, o = got.reshape(-1, w).astype(np.float64), want.reshape(-1, w).astype(np.float64)
    assert np.all(np.isfinite(g)), "non-finite residual"
    np.testing.assert_allclose(g[:, 0], o[:, 0], rtol=0, atol=1e-4 * max(1.0, float(np.abs(o[:, 0]).max())))
    at = np.exp(g[:, 0] - o[:, 0])[:, None]
    np.testing.assert_allclose(g[:, 1:2] * at, o[:, 1:2], rtol=2e-3)
    np.testing.assert_allclose(g[:, 2:] * at, o[:, 2:], rtol=0, atol=4e-3 * float(np.abs(o[:, 2:]).max()))
    fin = lambda r: (r[:, 2:] / r[:, 1:2]).astype(np.float16)  # noqa: E731
    parity(fin(g), fin(o))

