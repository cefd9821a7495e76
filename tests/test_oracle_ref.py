"""The C oracle against the reference's own x86_avx2 family, live (oracle/_ref; skipped where it is not built).

Rows the family runs through the generic body (its override table, x86_avx2/overrides/nn.cuh:2299-2337,
leaves them alone) agree bit for bit: scores, merge, finish, causal_scores, scores_grouped, softmax_rows,
causal_softmax, scores_grouped_rows, softmax_lens — except mix_rows, where the family's build
(g++ -O3 -mfma, engine/scripts/build_silicon_families.sh:198, whose default contracts a multiply-add into
an FMA) rounds `sum += p·v` once instead of twice: within one fp16 ulp there; the oracle stays the serial
IEEE sum (built -ffp-contract=off). Rows the family overrides with its own loop order agree within fp32
rounding: mix, weights, residual_mix, causal_scores_grouped, causal_mix.
Shapes include an odd head_dim (the dots' per-element arm, kernels.cuh:986-990) and a query at an address
that is 2 mod 4 (the same arm by alignment).
"""
import numpy as np
import pytest

from oracle.oracle import inputs

SHAPES = [(16, 2, 256, 300), (8, 8, 64, 33), (32, 4, 128, 700), (6, 3, 9, 41), (64, 1, 128, 17)]


def same(a, b):
    assert np.array_equal(np.asarray(a).view(np.uint32 if np.asarray(a).dtype == np.float32 else np.uint16),
                          np.asarray(b).view(np.uint32 if np.asarray(b).dtype == np.float32 else np.uint16))


@pytest.mark.parametrize("qh,kvh,hd,L", SHAPES)
def test_decode_rows(oracle, ref, qh, kvh, hd, L):
    q, k, v = inputs(L + hd, (qh * hd,), (L * kvh * hd,), (L * kvh * hd,))
    p = oracle.scores(q, k, qh, kvh, hd, L)
    same(p, ref.scores(q, k, qh, kvh, hd, L))
    o, _ = oracle.mix(p, v, qh, kvh, hd, L)
    ro, _ = ref.mix(p, v, qh, kvh, hd, L)
    np.testing.assert_allclose(o.astype(np.float32), ro.astype(np.float32), atol=2e-3, rtol=1e-3)
    wp, wres = oracle.weights(q, k, qh, kvh, hd, L)
    rp, rres = ref.weights(q, k, qh, kvh, hd, L)
    np.testing.assert_allclose(wp, rp, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(wres, rres, rtol=1e-5, atol=1e-6)
    wres = oracle.residual_mix(wres, wp, v, qh, kvh, hd, L)
    rres2 = ref.residual_mix(wres, wp, v, qh, kvh, hd, L)
    np.testing.assert_allclose(wres, rres2, rtol=1e-5, atol=1e-5)
    same(oracle.finish(wres, qh, hd)[0], ref.finish(wres, qh, hd)[0])
    half = wres.copy()
    half[2::hd + 2] *= 0.5
    same(oracle.merge(wres, half, qh, hd), ref.merge(wres, half, qh, hd))
    g = oracle.scores_grouped(q, k, qh, kvh, hd, L)
    same(g, ref.scores_grouped(q, k, qh, kvh, hd, L))
    same(oracle.softmax_rows(g, qh, L), ref.softmax_rows(g, qh, L))


def test_unaligned_query_takes_the_element_arm(oracle, ref):
    qh, kvh, hd, L = 8, 2, 64, 50
    buf, k = inputs(5, (qh * hd + 1,), (L * kvh * hd,))
    q = buf[1:]   # 2 bytes past a 4-byte boundary
    assert q.ctypes.data % 4 == 2
    same(oracle.scores_grouped(q, k, qh, kvh, hd, L), ref.scores_grouped(q, k, qh, kvh, hd, L))


@pytest.mark.parametrize("qh,kvh,hd,first,rows", [(16, 2, 256, 40, 24), (8, 2, 64, 0, 37), (6, 3, 9, 5, 11)])
def test_causal_rows(oracle, ref, qh, kvh, hd, first, rows):
    n = first + rows
    q, k, v = inputs(first + rows + hd, (rows * qh * hd,), (n * kvh * hd,), (n * kvh * hd,))
    p = oracle.causal_scores(q, k, qh, kvh, hd, first, rows)
    same(p, ref.causal_scores(q, k, qh, kvh, hd, first, rows))
    o, _ = oracle.causal_mix(p, v, qh, kvh, hd, first, rows)
    ro, _ = ref.causal_mix(p, v, qh, kvh, hd, first, rows)
    np.testing.assert_allclose(o.astype(np.float32), ro.astype(np.float32), atol=2e-3, rtol=1e-3)
    g = oracle.causal_scores_grouped(q, k, qh, kvh, hd, first, rows)
    rg = ref.causal_scores_grouped(q, k, qh, kvh, hd, first, rows)
    np.testing.assert_allclose(g, rg, rtol=2e-5, atol=2e-5)
    same(oracle.causal_softmax(g, qh, first, rows), ref.causal_softmax(g, qh, first, rows))
    wp, wres = oracle.weights_rows(q, k, qh, kvh, hd, first, rows)
    rp, rres = ref.weights_rows(q, k, qh, kvh, hd, first, rows)
    np.testing.assert_allclose(wp, rp, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(wres, rres, rtol=1e-5, atol=1e-6)
    a = oracle.residual_mix_rows(wres, wp, v, qh, kvh, hd, first, rows)
    b = ref.residual_mix_rows(wres, wp, v, qh, kvh, hd, first, rows)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5)


def test_lens_rows(oracle, ref):
    qh, kvh, hd, rows = 16, 4, 128, 4
    lens = np.array([7, 100, 1, 64], np.uint32)
    most = int(lens.max())
    q_row, k_row, p_row, o_row = qh * hd + 64, most * kvh * hd + 128, qh * most, qh * hd + 32
    q, k, v = inputs(9, (rows * q_row,), (rows * k_row,), (rows * k_row,))
    p = oracle.scores_grouped_rows(p_row, q, q_row, k, k_row, lens, qh, kvh, hd, most, rows)
    same(p, ref.scores_grouped_rows(p_row, q, q_row, k, k_row, lens, qh, kvh, hd, most, rows))
    same(oracle.softmax_lens(p, p_row, lens, qh, rows), ref.softmax_lens(p, p_row, lens, qh, rows))
    p = oracle.softmax_lens(p, p_row, lens, qh, rows)
    a = oracle.mix_rows(o_row, p, p_row, v, k_row, lens, qh, kvh, hd, rows)[0].view(np.uint16).astype(np.int32)
    b = ref.mix_rows(o_row, p, p_row, v, k_row, lens, qh, kvh, hd, rows)[0].view(np.uint16).astype(np.int32)
    assert np.max(np.abs(a - b)) <= 1          # same sign everywhere here, so bits 1 apart = 1 ulp


@pytest.mark.parametrize("rows,length,sink_at", [(16, 700, 0.0), (5, 33, 9.0), (3, 1, -40.0)])
def test_softmax_sink(oracle, ref, rows, length, sink_at):
    """attention_softmax_sink (gpu.cuh:201): the oracle is the family's door to the bit, with sinks below, inside and
    above the scores' range (a large sink takes the top, kernels.cuh:1112-1114)."""
    rng = np.random.default_rng(rows + length)
    p = (rng.standard_normal(rows * length) * 3).astype(np.float32)
    sink = (sink_at + rng.standard_normal(rows)).astype(np.float16).view(np.uint16)
    same(oracle.softmax_sink(p, sink, rows, length), ref.softmax_sink(p, sink, rows, length))


def test_softmax_sink_without_a_sink_is_the_softmax(oracle):
    """A sink of -inf weighs nothing: the row softmax (kernels.cuh:1085-1094) to fp32 rounding."""
    rng = np.random.default_rng(3)
    rows, length = 4, 300
    p = rng.standard_normal(rows * length).astype(np.float32)
    sink = np.full(rows, np.float16(-np.inf)).view(np.uint16)
    np.testing.assert_allclose(oracle.softmax_sink(p, sink, rows, length), oracle.softmax_rows(p, rows, length),
                               rtol=1e-6, atol=1e-9)
    # and the sink's own weight is what the row gives up: 1 - Σ p = e^(s - top) / (Σ e^(x - top) + e^(s - top))
    sink = np.full(rows, np.float16(1.5)).view(np.uint16)
    got = oracle.softmax_sink(p, sink, rows, length).reshape(rows, length).astype(np.float64)
    x = p.reshape(rows, length).astype(np.float64)
    want = 1.0 - np.exp(1.5) / (np.exp(x).sum(axis=1) + np.exp(1.5))
    np.testing.assert_allclose(got.sum(axis=1), want, rtol=1e-5)
