"""TurboQuant rows on gfx950 (gpu.cuh:163-164, 197-198) against the C oracle, through the C ABI.

The same shapes and bars as the emulated kernel tests in tests/test_tq.py: weights within 1e-4 relative,
the residual's {m, l} within 1e-5 relative and its acc within 1e-4 relative, and the finished fp16 answer at
max-abs <= 2e-3, cos >= 0.9999.
"""
import numpy as np
import pytest
import torch

from silvann_amd import doors
from tests.conftest import parity
from tests.gpu_util import t
from tests.test_tq import header_levels, make

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def each_door_on_its_own(dev):
    """test_tq_doors reads the weights between the doors, so no pair is deferred here (tests/test_gpu_chains.py
    covers the deferred pairs)."""
    doors.set_defer(False)
    yield
    doors.set_defer(True)


@pytest.mark.parametrize("d,hd,qh,kvh,length,rows", [
    (8, 128, 8, 2, 300, 0),
    (4, 256, 16, 2, 2500, 0),
    (3, 100, 6, 3, 50, 0),
    (8, 320, 2, 1, 64, 0),
    (4, 64, 4, 2, 2100, 3),
    (8, 128, 16, 2, 70000, 0),   # a long cold tier: many splits
])
def test_tq_doors(dev, oracle, d, hd, qh, kvh, length, rows):
    rng = np.random.default_rng(d + hd + length)
    lev = header_levels(d)
    n = max(rows, 1)
    q, codes, scales = make(rng, qh, kvh, hd, length, d, rows=n)
    print(f"case: tq d{d} hd{hd} qh{qh} kvh{kvh} length{length} rows{rows}", flush=True)
    p = torch.zeros(n * qh * length, dtype=torch.float32, device=dev)
    res = torch.full((n * qh * (hd + 2),), float("nan"), dtype=torch.float32, device=dev)
    qd, cd, sd = t(q, dev), t(codes, dev), t(scales, dev)
    if rows:
        doors.attention_weights_tq_rows(p, res, qd, cd, sd, qh, kvh, hd, length, d, rows)
        po, ro = oracle.weights_tq_rows(q, codes, scales, qh, kvh, hd, length, d, n, lev)
    else:
        doors.attention_weights_tq(p, res, qd, cd, sd, qh, kvh, hd, length, d)
        po, ro = oracle.weights_tq(q, codes, scales, qh, kvh, hd, length, d, lev)
    w = hd + 2
    np.testing.assert_allclose(p.cpu().numpy(), po, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(res.cpu().numpy().reshape(-1, w)[:, :2], ro.reshape(-1, w)[:, :2], rtol=1e-5)
    if rows:
        doors.attention_residual_mix_tq_rows(res, p, cd, sd, qh, kvh, hd, length, d, rows)
        ro2 = oracle.residual_mix_tq_rows(ro, po, codes, scales, qh, kvh, hd, length, d, n, lev)
    else:
        doors.attention_residual_mix_tq(res, p, cd, sd, qh, kvh, hd, length, d)
        ro2 = oracle.residual_mix_tq(ro, po, codes, scales, qh, kvh, hd, length, d, lev)
    got = res.cpu().numpy()
    np.testing.assert_allclose(got.reshape(-1, w)[:, 2:], ro2.reshape(-1, w)[:, 2:], rtol=1e-4,
                               atol=1e-5 * float(np.abs(ro2).max()))
    fin = lambda r: (r.reshape(-1, w)[:, 2:] / r.reshape(-1, w)[:, 1:2]).astype(np.float16)  # noqa: E731
    parity(fin(got), fin(ro2))
    assert not doors.launch_failed()


def test_tq_refuses_unknown_width(dev):
    p = torch.zeros(64, dtype=torch.float32, device=dev)
    res = torch.zeros(2 * 66, dtype=torch.float32, device=dev)
    q = torch.zeros(2 * 64, dtype=torch.float16, device=dev)
    codes = torch.zeros(64, dtype=torch.uint8, device=dev)
    scales = torch.zeros(4, dtype=torch.float16, device=dev)
    doors.launch_failed()
    doors.attention_weights_tq(p, res, q, codes, scales, 2, 1, 64, 1, 6)
    assert doors.launch_failed()


@pytest.mark.parametrize("d,hd,qh,kvh,length,rows", [
    (4, 128, 8, 2, 300, 1),
    (8, 256, 16, 2, 700, 1),
    (4, 64, 4, 4, 130, 3),
    (8, 128, 32, 2, 64, 1),
    (4, 128, 16, 2, 100000, 1),   # a long cold tier
])
def test_fused_residual(dev, oracle, d, hd, qh, kvh, length, rows):
    """attention_residual_tq (row 139) against weights_tq_rows + residual_mix_tq_rows in the oracle, the
    residual compared at the oracle's m (a residual is {m, l, acc} up to a common e^m), the answer at the bar."""
    from silvann_amd import verbs
    rng = np.random.default_rng(d * 5 + hd + length)
    lev = header_levels(d)
    q, kc, ks = make(rng, qh, kvh, hd, length, d, rows=rows)
    _, vc, vs = make(rng, qh, kvh, hd, length, d)
    print(f"case: tq fused d{d} hd{hd} qh{qh} kvh{kvh} length{length} rows{rows}", flush=True)
    res = torch.full((rows * qh * (hd + 2),), float("nan"), dtype=torch.float32, device=dev)
    scratch = torch.empty(verbs.residual_tq_scratch_bytes(qh, kvh, hd, length, d, rows), dtype=torch.uint8, device=dev)
    verbs.residual_tq_fused(t(q, dev), t(kc, dev), t(ks, dev), t(vc, dev), t(vs, dev), res, scratch, qh, kvh, hd, d,
                            length, rows)
    po, ro = oracle.weights_tq_rows(q, kc, ks, qh, kvh, hd, length, d, rows, lev)
    ro = oracle.residual_mix_tq_rows(ro, po, vc, vs, qh, kvh, hd, length, d, rows, lev)
    w = hd + 2
    got, want = res.cpu().numpy().reshape(-1, w).astype(np.float64), ro.reshape(-1, w).astype(np.float64)
    np.testing.assert_allclose(got[:, 0], want[:, 0], rtol=0, atol=2e-3 * max(1.0, float(np.abs(want[:, 0]).max())))
    at = np.exp(got[:, 0] - want[:, 0])[:, None]
    np.testing.assert_allclose(got[:, 1:2] * at, want[:, 1:2], rtol=2e-3)
    fin = lambda r: (r[:, 2:] / r[:, 1:2]).astype(np.float16)  # noqa: E731
    parity(fin(got), fin(want))
    assert not doors.launch_failed()
