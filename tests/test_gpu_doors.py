"""The reference's nn attention door rows on gfx950 against the C oracle, row by row, through the C ABI.

Tolerances: fp32 weights and scores within 1e-5 absolute (weights ≤ 1) / 2e-5 relative (scores); residual
{m, l, acc} within 2e-5 relative; fp16 outputs within the north star's 2e-3 / 0.9999. The overflow flag is
bit-exact ("NPOV").
"""
import numpy as np
import pytest
import torch

from oracle.oracle import FAULT_OVERFLOW, inputs
from silvann_amd import doors, verbs
from tests.conftest import parity
from tests.gpu_util import t

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def each_door_on_its_own(dev):
    """These tests read every door's buffers between doors, so no chain is deferred here (tests/test_gpu_chains.py
    covers the deferred chains)."""
    doors.set_defer(False)
    yield
    doors.set_defer(True)

SHAPES = [(16, 2, 256, 333), (8, 8, 64, 65), (32, 4, 128, 1000), (64, 1, 128, 100), (6, 2, 72, 50),
          (6, 3, 9, 41)]   # an odd head_dim takes the dots' per-element arm (kernels.cuh:986-990)


def close(got, want, atol, rtol=0.0):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want)
    tol = atol + rtol * np.abs(want)
    assert np.all(err <= tol), f"max err {err.max():.3e} at {int(np.argmax(err - tol))}"


def dev_zeros(n, dtype, dev):
    return torch.zeros(n, dtype=dtype, device=dev)


@pytest.mark.parametrize("qh,kvh,hd,L", SHAPES)
def test_scores_mix(dev, oracle, qh, kvh, hd, L):
    q, k, v = inputs(100 + L, (qh * hd,), (L * kvh * hd,), (L * kvh * hd,))
    p = dev_zeros(qh * L, torch.float32, dev)
    o = dev_zeros(qh * hd, torch.float16, dev)
    over = dev_zeros(1, torch.int32, dev)
    doors.attention_scores(p, t(q, dev), t(k, dev), qh, kvh, hd, L)
    want_p = oracle.scores(q, k, qh, kvh, hd, L)
    close(p.cpu().numpy(), want_p, 1e-5)
    doors.attention_mix(o, p, t(v, dev), qh, kvh, hd, L, over)
    want_o, _ = oracle.mix(want_p, v, qh, kvh, hd, L)
    parity(o.cpu().numpy(), want_o)
    assert int(over.item()) == 0


@pytest.mark.parametrize("qh,kvh,hd,L", SHAPES)
def test_weights_residual_merge_finish(dev, oracle, qh, kvh, hd, L):
    q, k, v = inputs(200 + L, (qh * hd,), (L * kvh * hd,), (L * kvh * hd,))
    p = dev_zeros(qh * L, torch.float32, dev)
    res = dev_zeros(qh * (hd + 2), torch.float32, dev)
    doors.attention_weights(p, res, t(q, dev), t(k, dev), qh, kvh, hd, L)
    wp, wres = oracle.weights(q, k, qh, kvh, hd, L)
    close(p.cpu().numpy(), wp, 1e-5)
    close(res.cpu().numpy(), wres, 1e-5, 2e-5)
    doors.attention_residual_mix(res, p, t(v, dev), qh, kvh, hd, L)
    wres = oracle.residual_mix(wres, wp, v, qh, kvh, hd, L)
    close(res.cpu().numpy(), wres, 1e-4, 2e-5)
    # split the range in two, merge the residuals: the one-call softmax (kernels.cuh:1180-1185)
    cut = L // 2 or 1
    row = kvh * hd
    ra = dev_zeros(qh * (hd + 2), torch.float32, dev)
    rb = dev_zeros(qh * (hd + 2), torch.float32, dev)
    kd, vd = t(k, dev), t(v, dev)
    pa = dev_zeros(qh * L, torch.float32, dev)
    doors.attention_weights(pa, ra, t(q, dev), kd, qh, kvh, hd, cut)
    doors.attention_residual_mix(ra, pa, vd, qh, kvh, hd, cut)
    if L > cut:
        doors.attention_weights(pa, rb, t(q, dev), kd.data_ptr() + 2 * cut * row, qh, kvh, hd, L - cut)
        doors.attention_residual_mix(rb, pa, vd.data_ptr() + 2 * cut * row, qh, kvh, hd, L - cut)
        doors.attention_merge(ra, ra, rb, qh, hd)   # `into` may be `a`
    o = dev_zeros(qh * hd, torch.float16, dev)
    over = dev_zeros(1, torch.int32, dev)
    doors.attention_finish(o, ra, qh, hd, over)
    want_o, _ = oracle.finish(wres, qh, hd)
    parity(o.cpu().numpy(), want_o)


@pytest.mark.parametrize("qh,kvh,hd,first,rows", [(16, 2, 256, 40, 24), (8, 2, 64, 0, 70), (6, 3, 72, 5, 9)])
def test_causal_rows(dev, oracle, qh, kvh, hd, first, rows):
    n = first + rows
    q, k, v = inputs(300 + rows, (rows * qh * hd,), (n * kvh * hd,), (n * kvh * hd,))
    qd, kd, vd = t(q, dev), t(k, dev), t(v, dev)
    span = first + rows
    # causal_scores (with its softmax) and causal_mix
    p = dev_zeros(rows * qh * span, torch.float32, dev)
    doors.attention_causal_scores(p, qd, kd, qh, kvh, hd, first, rows)
    wp = oracle.causal_scores(q, k, qh, kvh, hd, first, rows)
    close(p.cpu().numpy(), wp, 1e-5)
    o = dev_zeros(rows * qh * hd, torch.float16, dev)
    over = dev_zeros(1, torch.int32, dev)
    doors.attention_causal_mix(o, p, vd, qh, kvh, hd, first, rows, over)
    wo, _ = oracle.causal_mix(wp, v, qh, kvh, hd, first, rows)
    parity(o.cpu().numpy(), wo)
    # the grouped scores then the causal softmax (what nn__attention__rows calls)
    p2 = dev_zeros(rows * qh * span, torch.float32, dev)
    doors.attention_causal_scores_grouped(p2, qd, kd, qh, kvh, hd, first, rows)
    wp2 = oracle.causal_scores_grouped(q, k, qh, kvh, hd, first, rows)
    close(p2.cpu().numpy(), wp2, 1e-4, 2e-5)
    doors.attention_causal_softmax(p2, qh, first, rows)
    close(p2.cpu().numpy(), oracle.causal_softmax(wp2, qh, first, rows), 1e-5)
    # the many-row residuals (doors.cuh:417-432)
    p3 = dev_zeros(rows * qh * span, torch.float32, dev)
    res = dev_zeros(rows * qh * (hd + 2), torch.float32, dev)
    doors.attention_weights_rows(p3, res, qd, kd, qh, kvh, hd, first, rows)
    wp3, wres = oracle.weights_rows(q, k, qh, kvh, hd, first, rows)
    close(p3.cpu().numpy(), wp3, 1e-5)
    close(res.cpu().numpy(), wres, 1e-5, 2e-5)
    doors.attention_residual_mix_rows(res, p3, vd, qh, kvh, hd, first, rows)
    wres = oracle.residual_mix_rows(wres, wp3, v, qh, kvh, hd, first, rows)
    close(res.cpu().numpy(), wres, 1e-4, 2e-5)


@pytest.mark.parametrize("qh,kvh,hd,L", SHAPES[:3])
def test_grouped_and_softmax_rows(dev, oracle, qh, kvh, hd, L):
    q, k = inputs(400 + L, (qh * hd,), (L * kvh * hd,))
    p = dev_zeros(qh * L, torch.float32, dev)
    doors.attention_scores_grouped(p, t(q, dev), t(k, dev), qh, kvh, hd, L)
    wp = oracle.scores_grouped(q, k, qh, kvh, hd, L)
    close(p.cpu().numpy(), wp, 1e-4, 2e-5)
    doors.attention_softmax_rows(p, qh, L)
    close(p.cpu().numpy(), oracle.softmax_rows(wp, qh, L), 1e-5)


def test_unaligned_query_and_odd_head_dim_grouped(dev, oracle):
    """A query 2 bytes past a 4-byte boundary, and an odd head_dim: the element-wise arm of the dots."""
    for qh, kvh, hd, L in ((8, 2, 64, 50), (6, 3, 9, 41)):
        buf, k = inputs(600 + hd, (qh * hd + 1,), (L * kvh * hd,))
        qd = t(buf, dev)
        p = dev_zeros(qh * L, torch.float32, dev)
        print(f"case: grouped unaligned q qh{qh} kvh{kvh} hd{hd} L{L}", flush=True)
        doors.attention_scores_grouped(p, qd.data_ptr() + 2, t(k, dev), qh, kvh, hd, L)
        close(p.cpu().numpy(), oracle.scores_grouped(buf[1:], k, qh, kvh, hd, L), 1e-4, 2e-5)


def test_refused_shape_launches_nothing(dev):
    """A door given a shape it does not take launches nothing, leaves its output alone and reports the
    refusal through silvann_gfx950_launch_failed (then clears it)."""
    doors.launch_failed()   # clears what an earlier test may have left
    o = torch.full((16 * 96,), 7.0, dtype=torch.float16, device=dev)
    q = torch.zeros(16 * 96, dtype=torch.float16, device=dev)
    kv = torch.zeros(64 * 2 * 96, dtype=torch.float16, device=dev)
    lens = torch.tensor([64], dtype=torch.int32, device=dev)
    scratch = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    over = dev_zeros(1, torch.int32, dev)
    doors.attention_decode_paged(o, q, kv, kv, None, 0, 0, 0, lens, 16, 2, 96, 64, 1, scratch, over)   # head_dim 96
    torch.cuda.synchronize()
    assert doors.launch_failed() == 1
    assert doors.launch_failed() == 0
    assert torch.all(o == 7.0)
    # refused on another thread, read on this one: the flag is the device's (amd_rocm_base/sys.cuh:39-62)
    import threading
    th = threading.Thread(target=lambda: doors.attention_causal_paged(o, q, kv, kv, None, 0, 16, 2, 96, 0, 64, over))
    th.start()
    th.join()
    torch.cuda.synchronize()
    assert doors.launch_failed() == 1
    assert torch.all(o == 7.0) and int(over.item()) == 0


def test_refused_operands_of_the_appended_rows(dev):
    """Rows 137 and 138 refuse, launching nothing, q_heads 0 (0 % kv_heads is 0, which a divisibility check alone lets
    through to a zero-size grid), an unaligned q or k (their kernels load 16 bytes at a time) and, for 137, a scratch
    at 4 mod 8 (its counters are 64-bit)."""
    doors.launch_failed()
    o = torch.full((16 * 128,), 7.0, dtype=torch.float16, device=dev)
    q = torch.zeros(16 * 128 + 8, dtype=torch.float16, device=dev)
    kv = torch.zeros(64 * 2 * 128 + 8, dtype=torch.float16, device=dev)
    lens = torch.tensor([64], dtype=torch.int32, device=dev)
    scratch = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    over = dev_zeros(1, torch.int32, dev)
    cases = [
        ("decode q_heads 0", lambda: doors.attention_decode_paged(o, q, kv, kv, None, 0, 0, 0, lens, 0, 2, 128, 64, 1,
                                                                  scratch, over)),
        ("decode q at 2 mod 16", lambda: doors.attention_decode_paged(o, q.data_ptr() + 2, kv, kv, None, 0, 0, 0, lens,
                                                                      16, 2, 128, 64, 1, scratch, over)),
        ("decode scratch at 4 mod 8", lambda: doors.attention_decode_paged(o, q, kv, kv, None, 0, 0, 0, lens, 16, 2,
                                                                           128, 64, 1, scratch.data_ptr() + 4, over)),
        ("causal q_heads 0", lambda: doors.attention_causal_paged(o, q, kv, kv, None, 0, 0, 2, 128, 0, 8, over)),
        ("causal k at 2 mod 16", lambda: doors.attention_causal_paged(o, q, kv.data_ptr() + 2, kv, None, 0, 16, 2, 128,
                                                                      0, 8, over)),
    ]
    for name, call in cases:
        print(f"case: refusal, {name}", flush=True)
        call()
        torch.cuda.synchronize()
        assert doors.launch_failed() == 1, name
        assert torch.all(o == 7.0) and int(over.item()) == 0, name


def test_lens_rows(dev, oracle):
    qh, kvh, hd, rows = 16, 4, 128, 5
    lens = np.array([7, 100, 1, 64, 250], np.uint32)
    most = int(lens.max())
    q_row, k_row = qh * hd + 64, most * kvh * hd + 128
    p_row = qh * most
    o_row = qh * hd + 32
    q, k, v = inputs(500, (rows * q_row,), (rows * k_row,), (rows * k_row,))
    p = dev_zeros(rows * p_row, torch.float32, dev)
    ld = t(lens, dev)
    doors.attention_scores_grouped_rows(p, p_row, t(q, dev), q_row, t(k, dev), k_row, ld, qh, kvh, hd, most, rows)
    wp = oracle.scores_grouped_rows(p_row, q, q_row, k, k_row, lens, qh, kvh, hd, most, rows)
    close(p.cpu().numpy(), wp, 1e-4, 2e-5)
    doors.attention_softmax_lens(p, p_row, ld, qh, rows)
    wp = oracle.softmax_lens(wp, p_row, lens, qh, rows)
    close(p.cpu().numpy(), wp, 1e-5)
    o = dev_zeros(rows * o_row, torch.float16, dev)
    over = dev_zeros(1, torch.int32, dev)
    doors.attention_mix_rows(o, o_row, p, p_row, t(v, dev), k_row, ld, qh, kvh, hd, rows, over)
    wo, _ = oracle.mix_rows(o_row, wp, p_row, v, k_row, lens, qh, kvh, hd, rows)
    parity(o.cpu().numpy(), wo)


def test_overflow_flag(dev, oracle):
    """A finite fp16 answer past 65504 stores NPOV (kernels.cuh:29-40, 2763-2808); an answer that fits does not."""
    qh, kvh, hd, L = 2, 1, 64, 2
    v = np.full(L * hd, 40000.0, np.float16)
    p = np.full(qh * L, 1.0, np.float32)   # unnormalised weights: 2 × 40000 = 80000 overflows
    o = dev_zeros(qh * hd, torch.float16, dev)
    over = dev_zeros(1, torch.int32, dev)
    doors.attention_mix(o, t(p, dev), t(v, dev), qh, kvh, hd, L, over)
    assert (int(over.item()) & 0xFFFFFFFF) == FAULT_OVERFLOW
    _, wover = oracle.mix(p, v, qh, kvh, hd, L)
    assert wover == FAULT_OVERFLOW
    assert np.all(np.isinf(o.cpu().float().numpy()))
    # finish: acc / l over the largest half's rounding edge
    res = np.zeros(qh * (hd + 2), np.float32)
    res[1::hd + 2] = 1.0
    res[2:hd + 2] = 65519.0       # rounds to 65504: no flag
    res[hd + 4:] = 65520.0        # rounds to inf: flag
    o2 = dev_zeros(qh * hd, torch.float16, dev)
    over2 = dev_zeros(1, torch.int32, dev)
    doors.attention_finish(o2, t(res, dev), qh, hd, over2)
    wo, wover = oracle.finish(res, qh, hd)
    assert np.array_equal(o2.cpu().numpy().view(np.uint16), wo.view(np.uint16))
    assert (int(over2.item()) & 0xFFFFFFFF) == wover == FAULT_OVERFLOW


def test_decode_verb_matches_oracle_range(dev, oracle):
    """The host verb (attention__abi.cuh:129-160): a range [from, to) of the cache through scores + mix."""
    qh, kvh, hd, to, frm = 16, 2, 256, 900, 123
    q, k, v = inputs(600, (qh * hd,), (to * kvh * hd,), (to * kvh * hd,))
    scores = dev_zeros(qh * to, torch.float32, dev)
    out = dev_zeros(qh * hd, torch.float16, dev)
    over = dev_zeros(1, torch.int32, dev)
    verbs.decode(t(q, dev), t(k, dev), t(v, dev), scores, out, qh, kvh, hd, frm, to, over)
    row = kvh * hd
    wp = oracle.scores(q, k[frm * row:], qh, kvh, hd, to - frm)
    wo, _ = oracle.mix(wp, v[frm * row:], qh, kvh, hd, to - frm)
    parity(out.cpu().numpy(), wo)
    verbs.check_fault(over)


def test_rows_attention_passes(dev, oracle):
    """nn__attention__rows' attention part with a scores room that forces several passes."""
    qh, kvh, hd, first, rows = 16, 2, 128, 30, 50
    n = first + rows
    q, k, v = inputs(700, (rows * qh * hd,), (n * kvh * hd,), (n * kvh * hd,))
    scores = dev_zeros(qh * n * 7, torch.float32, dev)   # 7 rows a pass
    att = dev_zeros(rows * qh * hd, torch.float16, dev)
    over = dev_zeros(1, torch.int32, dev)
    verbs.rows_attention(t(q, dev), t(k, dev), t(v, dev), scores, att, qh, kvh, hd, first, rows, over)
    wo, _ = oracle.causal_rows(q, k, v, None, 0, qh, kvh, hd, first, list(range(rows)))
    parity(att.cpu().numpy(), wo)

