"""TurboQuant rows (gpu.cuh:163-164, 197-198; kernels.cuh:2957-3026): the level tables, the oracle, and the
library's kernels in the CPU emulation.

How each part is pinned:
  - the level tables (silvann_amd/csrc/tq_levels.hpp, from silvann_amd/tq_levels.py) are read back through
    the reference family's own residual_mix_tq door (oracle/_ref) and must match bit for bit, every width;
  - the oracle's weights_tq / residual_mix_tq (and their _rows forms) against the reference family's doors,
    within fp32 rounding (that family's build contracts the sums into FMAs);
  - without the reference: with power-of-two scales every value level·scale is an exact fp16, so the TurboQuant
    doors must equal the fp16 doors (attention_weights / attention_residual_mix) over the decoded cache bit for
    bit — a dropped scale, a wrong container, shift or row index fails it;
  - the library's kernels run in the CPU emulation (tests/emu) against the oracle: the weights and residuals
    within fp32 rounding, and the finished fp16 answer at the GPU tests' bar (max-abs <= 2e-3, cos >= 0.9999).
"""
import re

import numpy as np
import pytest

from silvann_amd import tq_levels
from tests.conftest import parity

HEADER = tq_levels.OUT


def header_levels(d):
    m = re.search(r"kTqLevels%d\[\d+\] = \{(.*?)\};" % d, HEADER.read_text(), re.S)
    return np.array([int(x, 16) for x in re.findall(r"0x[0-9A-F]{4}", m.group(1))], np.uint16)


def make(rng, qh, kvh, hd, length, d, rows=1, pow2=False):
    per = 16 // d
    rb = (hd + per - 1) // per * 2
    codes = rng.integers(0, 256, length * kvh * rb, dtype=np.uint8)
    if pow2:
        scales = (2.0 ** rng.integers(-3, 2, length * kvh)).astype(np.float16).view(np.uint16)
    else:
        scales = rng.uniform(0.05, 0.6, length * kvh).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(rows * qh * hd).astype(np.float16)
    return q, codes, scales


def decoded(codes, scales, kvh, hd, length, d, levels):
    """The cache as fp16 [position][kv head][dim]: level · scale (exact when the scale is a power of two)."""
    per = 16 // d
    rb = (hd + per - 1) // per * 2
    lv = levels.view(np.float16).astype(np.float32)
    out = np.zeros((length * kvh, hd), np.float32)
    units = codes.reshape(length * kvh, rb).view(np.uint16).astype(np.uint32)
    for c in range(hd):
        code = (units[:, c // per] >> (d * (c % per))) & ((1 << d) - 1)
        out[:, c] = lv[code] * scales.view(np.float16).astype(np.float32)
    return out.astype(np.float16).reshape(-1)


@pytest.mark.parametrize("d", [1, 2, 3, 4, 5, 8])
def test_levels_are_the_reference_tables(ref, d):
    assert np.array_equal(ref.tq_levels(d), header_levels(d))


def test_levels_generator_reproduces_header():
    assert tq_levels.emit() == HEADER.read_text()


SHAPES = [(8, 128, 8, 2, 300), (4, 128, 8, 2, 300), (8, 64, 4, 4, 77), (4, 256, 16, 2, 1000), (3, 100, 6, 3, 50)]


@pytest.mark.parametrize("d,hd,qh,kvh,length", SHAPES)
def test_oracle_matches_reference(ref, oracle, d, hd, qh, kvh, length):
    rng = np.random.default_rng(d * 1000 + hd)
    lev = header_levels(d)
    q, codes, scales = make(rng, qh, kvh, hd, length, d)
    pr, rr = ref.weights_tq(q, codes, scales, qh, kvh, hd, length, d)
    po, ro = oracle.weights_tq(q, codes, scales, qh, kvh, hd, length, d, lev)
    np.testing.assert_allclose(po, pr, rtol=2e-5, atol=1e-7)
    np.testing.assert_allclose(ro, rr, rtol=2e-6)
    rr2 = ref.residual_mix_tq(rr, pr, codes, scales, qh, kvh, hd, length, d)
    ro2 = oracle.residual_mix_tq(ro, po, codes, scales, qh, kvh, hd, length, d, lev)
    np.testing.assert_allclose(ro2, rr2, rtol=2e-5, atol=2e-5 * float(np.abs(rr2).max()))


def test_oracle_rows_match_reference(ref, oracle):
    rng = np.random.default_rng(11)
    d, hd, qh, kvh, length, rows = 4, 64, 4, 2, 90, 3
    lev = header_levels(d)
    q, codes, scales = make(rng, qh, kvh, hd, length, d, rows=rows)
    pr, rr = ref.weights_tq_rows(q, codes, scales, qh, kvh, hd, length, d, rows)
    po, ro = oracle.weights_tq_rows(q, codes, scales, qh, kvh, hd, length, d, rows, lev)
    np.testing.assert_allclose(po, pr, rtol=2e-5, atol=1e-7)
    rr2 = ref.residual_mix_tq_rows(rr, pr, codes, scales, qh, kvh, hd, length, d, rows)
    ro2 = oracle.residual_mix_tq_rows(ro, po, codes, scales, qh, kvh, hd, length, d, rows, lev)
    np.testing.assert_allclose(ro2, rr2, rtol=2e-5, atol=2e-5 * float(np.abs(rr2).max()))


@pytest.mark.parametrize("d,hd,qh,kvh,length", SHAPES)
def test_oracle_is_the_fp16_path_on_exact_values(oracle, d, hd, qh, kvh, length):
    rng = np.random.default_rng(d * 77 + hd)
    lev = header_levels(d)
    q, codes, scales = make(rng, qh, kvh, hd, length, d, pow2=True)
    kv = decoded(codes, scales, kvh, hd, length, d, lev)
    pt, rt = oracle.weights_tq(q, codes, scales, qh, kvh, hd, length, d, lev)
    pf, rf = oracle.weights(q, kv, qh, kvh, hd, length)
    assert np.array_equal(pt, pf) and np.array_equal(rt, rf)
    assert np.array_equal(oracle.residual_mix_tq(rt, pt, codes, scales, qh, kvh, hd, length, d, lev),
                          oracle.residual_mix(rf, pf, kv, qh, kvh, hd, length))


# ── the library's kernels in the CPU emulation ───────────────────────────────────────────────────────────

@pytest.mark.parametrize("d,hd,qh,kvh,length,rows", [
    (8, 128, 8, 2, 300, 0),      # one split: the sums go straight into the residual
    (4, 256, 16, 2, 2500, 0),    # two splits: sums kept in p, then reduced
    (3, 100, 6, 3, 50, 0),       # five codes a container, a part-filled last container
    (8, 320, 2, 1, 64, 0),       # head_dim past 256: one split, two passes of lanes
    (4, 64, 4, 2, 2100, 3),      # the _rows forms, split
])
def test_emulated_kernels(oracle, d, hd, qh, kvh, length, rows):
    from tests.emu import emu
    if emu.compiler() is None:
        pytest.skip("no clang++ for the CPU emulation")
    rng = np.random.default_rng(d + hd + length)
    lev = header_levels(d)
    n = max(rows, 1)
    q, codes, scales = make(rng, qh, kvh, hd, length, d, rows=n)
    p, res_w, res, over, _ = emu.run_tq(q, codes, scales, qh, kvh, hd, length, d, rows=rows)
    if rows:
        po, ro = oracle.weights_tq_rows(q, codes, scales, qh, kvh, hd, length, d, n, lev)
        ro2 = oracle.residual_mix_tq_rows(ro, po, codes, scales, qh, kvh, hd, length, d, n, lev)
    else:
        po, ro = oracle.weights_tq(q, codes, scales, qh, kvh, hd, length, d, lev)
        ro2 = oracle.residual_mix_tq(ro, po, codes, scales, qh, kvh, hd, length, d, lev)
    np.testing.assert_allclose(p, po, rtol=1e-4, atol=1e-6)
    w = hd + 2
    np.testing.assert_allclose(res_w.reshape(-1, w)[:, :2], ro.reshape(-1, w)[:, :2], rtol=1e-5)
    np.testing.assert_allclose(res.reshape(-1, w)[:, 2:], ro2.reshape(-1, w)[:, 2:], rtol=1e-4,
                               atol=1e-5 * float(np.abs(ro2).max()))
    # the finished answer, as attention_finish gives it: acc / l in fp16
    fin = lambda r: (r.reshape(-1, w)[:, 2:] / r.reshape(-1, w)[:, 1:2]).astype(np.float16)  # noqa: E731
    parity(fin(res), fin(ro2))


# ── the fused row (attention_residual_tq, row 139) in the CPU emulation ──────────────────────────────────

@pytest.mark.parametrize("d,hd,qh,kvh,length,rows", [
    (4, 128, 8, 2, 300, 1),      # the cold tier's width, one decode query
    (8, 256, 16, 2, 700, 1),     # the warm tier's width, several splits
    (4, 64, 4, 4, 130, 3),       # group 1, three query rows (the tiered prefill window)
    (8, 128, 32, 2, 64, 1),      # a group of 16: one full head block
])
def test_emulated_fused_residual(oracle, d, hd, qh, kvh, length, rows):
    from tests.emu import emu
    if emu.compiler() is None:
        pytest.skip("no clang++ for the CPU emulation")
    rng = np.random.default_rng(d * 5 + hd + length)
    lev = header_levels(d)
    q, kc, ks = make(rng, qh, kvh, hd, length, d, rows=rows)
    _, vc, vs = make(rng, qh, kvh, hd, length, d)
    res, over, _ = emu.run_tq_fused(q, kc, ks, vc, vs, qh, kvh, hd, length, d, rows=rows)
    po, ro = oracle.weights_tq_rows(q, kc, ks, qh, kvh, hd, length, d, rows, lev)
    ro = oracle.residual_mix_tq_rows(ro, po, vc, vs, qh, kvh, hd, length, d, rows, lev)
    w = hd + 2
    got, want = res.reshape(-1, w).astype(np.float64), ro.reshape(-1, w).astype(np.float64)
    # m is the largest score: the keys go through the matrix cores as fp16 (level · scale rounded), so within
    # that rounding. A residual is {m, l, acc} up to a common factor e^m (attention_merge takes any), so l and acc
    # are compared at the reference's m.
    np.testing.assert_allclose(got[:, 0], want[:, 0], rtol=0, atol=2e-3 * max(1.0, float(np.abs(want[:, 0]).max())))
    at = np.exp(got[:, 0] - want[:, 0])[:, None]
    np.testing.assert_allclose(got[:, 1:2] * at, want[:, 1:2], rtol=2e-3)
    np.testing.assert_allclose(got[:, 2:] * at, want[:, 2:], rtol=0, atol=4e-3 * float(np.abs(want[:, 2:]).max()))
    fin = lambda r: (r[:, 2:] / r[:, 1:2]).astype(np.float16)  # noqa: E731
    parity(fin(got), fin(want))
