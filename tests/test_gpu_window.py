"""The causal residual row (silvann_gfx950_attention_causal_residual_paged, row 140) and the tiered prefill window
verbs on gfx950, through the C ABI.

- Row 140 against the oracle's attention_weights_rows + attention_residual_mix_rows over the gathered cache, the pair
  it replaces (tests/conftest.py::residual_parity: m to fp32 rounding, l and acc at the oracle's m to the weights'
  fp16 rounding, answers to the fp16 bar); bit for bit the same under a permuted page table as over the gathered
  contiguous cache; and finished, the fp16 bar against row 138's answers.
- window_attention (the reference's doors in the reference's order) and window_attention_fused (rows 138-140)
  against tests/test_window.py::oracle_window, and against each other.
"""
import numpy as np
import pytest
import torch

from silvann_amd import doors, verbs
from silvann_amd import workloads as W
from tests.conftest import parity, residual_parity
from tests.gpu_util import t
from tests.test_window import make_window, oracle_window

pytestmark = pytest.mark.gpu


def _res(dev, rows, qh, hd, blocks=1):
    return torch.full((blocks * rows * qh * (hd + 2),), float("nan"), dtype=torch.float32, device=dev)


@pytest.mark.parametrize("hd,qh,kvh,first,rows,ps", [
    (256, 16, 2, 0, 130, 0),       # chunk from position 0, paired row tiles, the steady loop
    (256, 16, 2, 77, 95, 64),      # paged, page table in LDS
    (128, 6, 2, 10, 70, 0),        # group 3: one head a wave
    (128, 32, 4, 300, 64, 32),     # prefix longer than the chunk
    (64, 8, 2, 5, 200, 0),
])
def test_causal_residual_against_oracle(dev, oracle, hd, qh, kvh, first, rows, ps):
    print(f"case: causal_residual hd{hd} qh{qh} kvh{kvh} first{first} rows{rows} ps{ps}", flush=True)
    w = W.causal("res", qh, kvh, hd, first, rows, page_size=ps, seed=hd + rows + 1)
    res = _res(dev, rows, qh, hd)
    pages = None if w.pages is None else t(w.pages.astype(np.int32), dev)
    verbs.causal_residual_paged(t(w.q, dev), t(w.k, dev), t(w.v, dev), pages, res, qh, kvh, hd, first, rows,
                                page_size=ps)
    got = res.cpu().numpy()
    assert not doors.launch_failed()
    k, v = w.gathered()
    p, r = oracle.weights_rows(w.q, k, qh, kvh, hd, first, rows)
    want = oracle.residual_mix_rows(r, p, v, qh, kvh, hd, first, rows)
    residual_parity(got, want, hd)


def test_causal_residual_pages_bit_exact(dev):
    """A permuted page table gives the same bits as the gathered contiguous cache."""
    hd, qh, kvh, first, rows, ps = 256, 16, 2, 500, 100, 64
    print("case: causal_residual pages bit-exact", flush=True)
    w = W.causal("res", qh, kvh, hd, first, rows, page_size=ps, seed=11)
    k, v = w.gathered()
    a, b = _res(dev, rows, qh, hd), _res(dev, rows, qh, hd)
    verbs.causal_residual_paged(t(w.q, dev), t(w.k, dev), t(w.v, dev), t(w.pages.astype(np.int32), dev), a, qh, kvh,
                                hd, first, rows, page_size=ps)
    verbs.causal_residual_paged(t(w.q, dev), t(k, dev), t(v, dev), None, b, qh, kvh, hd, first, rows)
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_causal_residual_finishes_to_causal(dev):
    """finish(row 140) is row 138's answer (to fp16 rounding: one divides, the other multiplies by 1/l)."""
    hd, qh, kvh, first, rows = 128, 16, 2, 1000, 256
    print("case: causal_residual finish", flush=True)
    w = W.causal("res", qh, kvh, hd, first, rows, seed=12)
    qd, kd, vd = t(w.q, dev), t(w.k, dev), t(w.v, dev)
    res = _res(dev, rows, qh, hd)
    verbs.causal_residual_paged(qd, kd, vd, None, res, qh, kvh, hd, first, rows)
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    fin = torch.zeros(rows * qh * hd, dtype=torch.float16, device=dev)
    doors.attention_finish(fin, res, rows * qh, hd, over)
    direct = torch.zeros_like(fin)
    verbs.causal_paged(qd, kd, vd, None, direct, qh, kvh, hd, first, rows)
    parity(fin.cpu().numpy(), direct.cpu().numpy())
    assert int(over.item()) == 0


def _dev_tier(tier, dev):
    if tier is None:
        return None
    kc, ks, vc, vs, count = tier
    return (t(kc, dev), t(ks, dev), t(vc, dev), t(vs, dev), count)


@pytest.mark.parametrize("qh,kvh,hd,first_w,rows,n_warm,n_cold", [
    (16, 2, 256, 200, 64, 300, 500),    # both tiers (Qwen's shape)
    (16, 2, 256, 0, 48, 0, 0),          # the window is the whole cache: the causal route
    (8, 2, 128, 1000, 100, 2048, 0),    # warm only
    (4, 4, 64, 33, 17, 0, 4000),        # cold only, a long one (several splits)
])
def test_window_verbs(dev, oracle, qh, kvh, hd, first_w, rows, n_warm, n_cold):
    print(f"case: window qh{qh} kvh{kvh} hd{hd} first_w{first_w} rows{rows} warm{n_warm} cold{n_cold}", flush=True)
    q, wk, wv, warm, cold = make_window(qh + hd + rows, qh, kvh, hd, first_w, rows, n_warm, n_cold)
    want = oracle_window(oracle, q, wk, wv, first_w, rows, warm, cold, qh, kvh, hd)
    qd, wkd, wvd = t(q, dev), t(wk, dev), t(wv, dev)
    wd, cd = _dev_tier(warm, dev), _dev_tier(cold, dev)
    window = first_w + rows
    longest = max(window, n_warm, n_cold)
    over = torch.zeros(1, dtype=torch.int32, device=dev)

    att = torch.zeros(rows * qh * hd, dtype=torch.float16, device=dev)
    scores = torch.zeros(qh * longest, dtype=torch.float32, device=dev)
    rows_scores = torch.zeros(rows * qh * longest, dtype=torch.float32, device=dev)
    verbs.window_attention(qd, wkd, wvd, first_w, rows, wd, cd, scores, rows_scores, _res(dev, rows, qh, hd, 3), att,
                           qh, kvh, hd, over)
    ref_order = att.cpu().numpy()
    parity(ref_order, want)

    fused = torch.zeros_like(att)
    need = verbs.window_scratch_bytes(qh, kvh, hd, rows, n_warm, n_cold)
    scratch = torch.empty(max(need, 4), dtype=torch.uint8, device=dev)
    verbs.window_attention_fused(qd, wkd, wvd, first_w, rows, wd, cd, _res(dev, rows, qh, hd, 3), scratch, fused, qh,
                                 kvh, hd, over)
    got = fused.cpu().numpy()
    parity(got, want)
    parity(got, ref_order)
    assert int(over.item()) == 0
    assert not doors.launch_failed()
