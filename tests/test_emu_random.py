"""Seeded random shapes through the emulated kernels (tests/emu) against the oracle: row 137 in each of its forms
(row order and the fused finish in one or two levels, the inline plan, latent attention's wide form), row 138 and its
residual form 140, and the TurboQuant row 139 — head counts that are not multiples of the head blocks, empty and
one-position rows, rows of many splits, page sizes from 16 to 256. The shapes come from fixed seeds, so a failure
names a case that reruns as it failed."""
import random

import numpy as np
import pytest

from silvann_amd import workloads as W
from tests.conftest import parity, residual_parity
from tests.emu import emu

pytestmark = pytest.mark.skipif(emu.compiler() is None, reason="no clang++ for the CPU emulation")

FORMS = [None, {"SILVANN_GFX950_DECODE_FUSED": "1"}, {"SILVANN_GFX950_DECODE_INLINE": "1"},
         {"SILVANN_GFX950_DECODE_FUSED": "1", "SILVANN_GFX950_DECODE_INLINE": "1"}]


def _decode_case(seed):
    rng = random.Random(seed)
    hd = rng.choice([64, 128, 256])
    kvh = rng.choice([1, 2, 4])
    qh = kvh * rng.choice([1, 2, 3, 8, 20])
    rows = rng.choice([1, 2, 5, 33])
    most = rng.choice([40, 700, 6000])
    lens = [rng.randrange(0, most) for _ in range(rows)]
    lens[rng.randrange(rows)] = most   # one row as long as the batch's bound
    return qh, kvh, hd, lens, rng.choice([0, 16, 32, 64, 256]), FORMS[seed % len(FORMS)]


@pytest.mark.parametrize("seed", range(12))
def test_decode(oracle, seed):
    qh, kvh, hd, lens, ps, env = _decode_case(seed)
    print(f"case: decode qh{qh} kvh{kvh} hd{hd} lens{lens} ps{ps} {env}", flush=True)
    w = W.decode("rand", qh, kvh, hd, lens, page_size=ps, seed=seed)
    got, over, _ = emu.run_decode(w, env=env)
    want, _ = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, kvh, hd,
                                  w.rows)
    parity(got, want)
    assert over == 0


@pytest.mark.parametrize("seed", range(6))
def test_latent(oracle, seed):
    rng = random.Random(100 + seed)
    kvh = rng.choice([1, 2])
    qh = kvh * rng.choice([8, 17, 48, 64, 80])
    lens = [rng.randrange(0, 3000) for _ in range(rng.choice([1, 2, 4]))]
    lens[0] = max(lens[0], 1)
    ps = rng.choice([0, 16, 64])
    env = {"SILVANN_GFX950_DECODE_LATENT": "wide"} if seed % 2 == 0 else None
    print(f"case: latent qh{qh} kvh{kvh} lens{lens} ps{ps} {env}", flush=True)
    w = W.decode("rand", qh, kvh, 512, lens, page_size=ps, seed=100 + seed)
    got, over, _ = emu.run_decode(w, shared=True, env=env)
    want, _ = oracle.decode_paged(w.q, w.k, w.k, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, kvh, 512,
                                  w.rows)
    parity(got, want)
    assert over == 0


@pytest.mark.parametrize("seed", range(8))
def test_causal(oracle, seed):
    rng = random.Random(200 + seed)
    hd = rng.choice([64, 128, 256])
    kvh = rng.choice([1, 2])
    qh = kvh * rng.choice([1, 2, 3, 4, 6, 8])
    first, rows, ps = rng.choice([0, 1, 33, 300]), rng.choice([1, 31, 33, 97, 130]), rng.choice([0, 32, 64, 96])
    residual = seed % 2 == 1
    print(f"case: causal{' residual' if residual else ''} qh{qh} kvh{kvh} hd{hd} first{first} rows{rows} ps{ps}",
          flush=True)
    w = W.causal("rand", qh, kvh, hd, first, rows, page_size=ps, seed=200 + seed)
    if residual:
        got, over, _ = emu.run_causal_res(w)
        k, v = w.gathered()
        p, res = oracle.weights_rows(w.q, k, qh, kvh, hd, first, rows)
        residual_parity(got, oracle.residual_mix_rows(res, p, v, qh, kvh, hd, first, rows), hd)
    else:
        got, over, _ = emu.run_causal(w)
        want, _ = oracle.causal_rows(w.q, w.k, w.v, w.pages, w.page_size, qh, kvh, hd, first, list(range(rows)))
        parity(got, want)
    assert over == 0


@pytest.mark.parametrize("seed", range(6))
def test_tq(oracle, seed):
    from tests.test_tq import header_levels, make
    rng = random.Random(300 + seed)
    d, hd, kvh = rng.choice([4, 8]), rng.choice([64, 128, 256]), rng.choice([1, 2])
    qh = kvh * rng.choice([1, 3, 8, 20])
    length, rows = rng.choice([1, 31, 300, 1100]), rng.choice([1, 3])
    print(f"case: tq d{d} hd{hd} qh{qh} kvh{kvh} len{length} rows{rows}", flush=True)
    nrng = np.random.default_rng(300 + seed)
    lev = header_levels(d)
    q, kc, ks = make(nrng, qh, kvh, hd, length, d, rows=rows)
    _, vc, vs = make(nrng, qh, kvh, hd, length, d)
    res, over, _ = emu.run_tq_fused(q, kc, ks, vc, vs, qh, kvh, hd, length, d, rows=rows)
    po, ro = oracle.weights_tq_rows(q, kc, ks, qh, kvh, hd, length, d, rows, lev)
    ro = oracle.residual_mix_tq_rows(ro, po, vc, vs, qh, kvh, hd, length, d, rows, lev)
    w_ = hd + 2
    got, want = res.reshape(-1, w_).astype(np.float64), ro.reshape(-1, w_).astype(np.float64)
    np.testing.assert_allclose(got[:, 0], want[:, 0], rtol=0, atol=2e-3 * max(1.0, float(np.abs(want[:, 0]).max())))
    at = np.exp(got[:, 0] - want[:, 0])[:, None]
    np.testing.assert_allclose(got[:, 1:2] * at, want[:, 1:2], rtol=2e-3)
    fin = lambda r: (r[:, 2:] / r[:, 1:2]).astype(np.float16)  # noqa: E731
    parity(fin(got), fin(want))


@pytest.mark.parametrize("seed", range(10))
def test_causal_duo(oracle, seed):
    """SILVANN_GFX950_PREFILL=duo over random shapes: groups of 4 and 8 take causal_duo at head_dim 128 and 256;
    other groups and widths fall back to causal_mfma under the same switch."""
    rng = random.Random(400 + seed)
    hd = rng.choice([128, 256, 256, 64])
    kvh = rng.choice([1, 2])
    qh = kvh * rng.choice([4, 8, 8, 2])
    first, rows, ps = rng.choice([0, 1, 33, 300]), rng.choice([1, 31, 33, 97, 130]), rng.choice([0, 32, 64, 96])
    print(f"case: causal duo qh{qh} kvh{kvh} hd{hd} first{first} rows{rows} ps{ps}", flush=True)
    w = W.causal("rand", qh, kvh, hd, first, rows, page_size=ps, seed=400 + seed)
    got, over, _ = emu.run_causal(w, {"SILVANN_GFX950_PREFILL": "duo"})
    want, _ = oracle.causal_rows(w.q, w.k, w.v, w.pages, w.page_size, qh, kvh, hd, first, list(range(rows)))
    parity(got, want)
    assert over == 0
