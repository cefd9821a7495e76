"""The tiered prefill window (ai_qwen_3 prefill__abi.cuh:409-447, step ④) on the CPU: the oracle's composition
of it, pinned against what the mathematics fixes, and the verbs' refusals.

The reference's step ④ gives each chunk row three residuals — over the fp16 window up to its own position
(weights_rows + residual_mix_rows), over the whole 8-bit warm tier and over the whole 4-bit cold tier
(weights_tq_rows + residual_mix_tq_rows) — and merges and finishes them. A merge of residuals is attention over the
union of their keys (kernels.cuh:1180-1185), so with power-of-two scales (the tiers' values then decode to fp16
exactly) the composed answer must be the causal attention of the same rows over one cache that holds the cold
tier, the warm tier and then the window: row r at position n_cold + n_warm + first_w + r. `oracle_window` is the
checker the GPU tests hold the library's verbs to.
"""
import numpy as np
import pytest
import torch

from silvann_amd import verbs
from tests.conftest import parity
from tests.test_tq import decoded, header_levels, make


def oracle_window(oracle, q, wk, wv, first_w, rows, warm, cold, qh, kvh, hd):
    """Step ④ in the oracle: fp16 answers of the chunk's rows. `warm` / `cold` are (kc, ks, vc, vs, count) numpy
    arrays or None."""
    if warm is None and cold is None:
        o, _ = oracle.causal_rows(q, wk, wv, None, 0, qh, kvh, hd, first_w, list(range(rows)))
        return o
    p, r0 = oracle.weights_rows(q, wk, qh, kvh, hd, first_w, rows)
    r0 = oracle.residual_mix_rows(r0, p, wv, qh, kvh, hd, first_w, rows)
    for tier, d in ((warm, verbs.WARM_BITS), (cold, verbs.COLD_BITS)):
        if tier is None:
            continue
        kc, ks, vc, vs, count = tier
        lev = header_levels(d)
        pt, rt = oracle.weights_tq_rows(q, kc, ks, qh, kvh, hd, count, d, rows, lev)
        rt = oracle.residual_mix_tq_rows(rt, pt, vc, vs, qh, kvh, hd, count, d, rows, lev)
        r0 = oracle.merge(r0, rt, rows * qh, hd)
    o, _ = oracle.finish(r0, rows * qh, hd)
    return o


def make_window(seed, qh, kvh, hd, first_w, rows, n_warm, n_cold, pow2=False):
    rng = np.random.default_rng(seed)
    window = first_w + rows
    q = rng.standard_normal(rows * qh * hd).astype(np.float16)
    wk = rng.standard_normal(window * kvh * hd).astype(np.float16)
    wv = rng.standard_normal(window * kvh * hd).astype(np.float16)
    tiers = []
    for count, d in ((n_warm, verbs.WARM_BITS), (n_cold, verbs.COLD_BITS)):
        if count == 0:
            tiers.append(None)
            continue
        _, kc, ks = make(rng, qh, kvh, hd, count, d, pow2=pow2)
        _, vc, vs = make(rng, qh, kvh, hd, count, d, pow2=pow2)
        tiers.append((kc, ks, vc, vs, count))
    return q, wk, wv, tiers[0], tiers[1]


@pytest.mark.parametrize("qh,kvh,hd,first_w,rows,n_warm,n_cold", [
    (4, 2, 64, 20, 9, 30, 0),      # warm tier only
    (6, 3, 32, 5, 7, 0, 25),       # cold tier only
    (8, 2, 64, 40, 12, 33, 50),    # both
])
def test_oracle_window_is_causal_over_the_concatenated_cache(oracle, qh, kvh, hd, first_w, rows, n_warm, n_cold):
    q, wk, wv, warm, cold = make_window(qh + hd + rows, qh, kvh, hd, first_w, rows, n_warm, n_cold, pow2=True)
    got = oracle_window(oracle, q, wk, wv, first_w, rows, warm, cold, qh, kvh, hd)
    parts_k, parts_v = [], []
    for tier, d in ((cold, verbs.COLD_BITS), (warm, verbs.WARM_BITS)):
        if tier is None:
            continue
        kc, ks, vc, vs, count = tier
        lev = header_levels(d)
        parts_k.append(decoded(kc, ks, kvh, hd, count, d, lev))
        parts_v.append(decoded(vc, vs, kvh, hd, count, d, lev))
    k = np.concatenate(parts_k + [wk])
    v = np.concatenate(parts_v + [wv])
    first = n_warm + n_cold + first_w
    want, _ = oracle.causal_rows(q, k, v, None, 0, qh, kvh, hd, first, list(range(rows)))
    parity(got, want)


def test_oracle_window_without_tiers_is_the_window_causal(oracle):
    """No warm or cold rows: the residual route (one tier of zero rows skipped) and the causal route agree."""
    qh, kvh, hd, first_w, rows = 4, 2, 64, 30, 10
    q, wk, wv, _, _ = make_window(3, qh, kvh, hd, first_w, rows, 0, 0)
    direct = oracle_window(oracle, q, wk, wv, first_w, rows, None, None, qh, kvh, hd)
    p, r = oracle.weights_rows(q, wk, qh, kvh, hd, first_w, rows)
    r = oracle.residual_mix_rows(r, p, wv, qh, kvh, hd, first_w, rows)
    o, _ = oracle.finish(r, rows * qh, hd)
    parity(o, direct)


def _cpu(n, dtype=torch.float16):
    return torch.zeros(n, dtype=dtype)


@pytest.mark.parametrize("fused", [False, True])
def test_window_verbs_refuse_before_any_door(fused):
    """The checks raise before a door runs (CPU tensors: any door call would fail differently)."""
    qh, kvh, hd, first_w, rows = 4, 2, 64, 10, 4
    q, att = _cpu(rows * qh * hd), _cpu(rows * qh * hd)
    wk, wv = _cpu((first_w + rows) * kvh * hd), _cpu((first_w + rows) * kvh * hd)
    res = _cpu(3 * rows * qh * (hd + 2), torch.float32)
    # the codes' room, in halves, must hold their bytes (the reference's count, attention__abi.cuh:262-265)
    cb = 2 * 50 * kvh * verbs.tq_row_bytes(verbs.WARM_BITS, hd)
    warm = (torch.zeros(cb, dtype=torch.uint8), _cpu(50 * kvh), torch.zeros(cb, dtype=torch.uint8), _cpu(50 * kvh), 50)

    def call(**kw):
        a = dict(q=q, window_k=wk, window_v=wv, first_w=first_w, rows=rows, warm=warm, cold=None, res=res, att=att,
                 q_heads=qh, kv_heads=kvh, head_dim=hd, over=None)
        a.update(kw)
        if fused:
            return verbs.window_attention_fused(scratch=None, **a)
        return verbs.window_attention(scores=_cpu(1, torch.float32), rows_scores=_cpu(1, torch.float32), **a)

    with pytest.raises(verbs.Fault) as e:
        call(window_k=_cpu(10))                         # the window's keys short
    assert e.value.word == verbs.FAULT_BOUNDS
    with pytest.raises(verbs.Fault) as e:
        call(res=_cpu(10, torch.float32))               # no room for the three residual blocks
    assert e.value.word == verbs.FAULT_BOUNDS
    short = (warm[0][:10], warm[1], warm[2], warm[3], 50)
    with pytest.raises(verbs.Fault) as e:
        call(warm=short)                                # the warm codes short of 50 rows
    assert e.value.word == verbs.FAULT_BOUNDS
    with pytest.raises(verbs.Fault) as e:
        call(q_heads=5)                                 # heads not a multiple of the kv heads
    assert e.value.word == verbs.FAULT_TYPE
    with pytest.raises(verbs.Fault) as e:
        call()                                          # fused: no scratch; reference order: no room for weights
    assert e.value.word == (verbs.FAULT_BOUNDS if fused else verbs.FAULT_ROOM)
