"""The C oracle against what the mathematics fixes, independently of the reference's code.

* half <-> float: exhaustive over every half (widening), and over a large sample of floats plus the
  boundary cases (narrowing), against numpy's IEEE conversions (kernels.cuh:2733-2808 are RNE with
  subnormals kept); the overflow flag is "finite in, infinite out".
* softmax attention in float64 by brute force on small shapes, with the GQA map kv = h / (qh / kvh)
  written out as a loop over heads: a transposed operand, a wrong head map, a missing scale or a
  wrong mask fails it (decode, causal, grouped and the split-K residual route).
* closed forms: one position gives v exactly; identical keys give the mean of v; causal row r is
  decode at position first + r; merging the residuals of two halves gives the whole.
* pages: a permuted page table gives the bits of the contiguous cache.
"""
import numpy as np
import pytest

from oracle.oracle import inputs

# within two fp16 ulps of the float64 answer (the oracle's fp32 sums add a few fp32 roundings to the one
# fp16 rounding) plus a floor for answers near zero
def near(got, want, ulps=2):
    g = np.asarray(got, np.float16).astype(np.float64).ravel()
    w = np.asarray(want, np.float64).ravel()
    spacing = np.spacing(np.abs(w).astype(np.float16)).astype(np.float64)
    bad = np.abs(g - w) > ulps * spacing + 1e-6
    assert not bad.any(), (np.flatnonzero(bad)[:5], g[bad][:5], w[bad][:5])


def brute_decode(q, k, v, qh, kvh, hd, n):
    """softmax(q·kᵀ / sqrt(hd)) · v in float64, head h reading kv head h // (qh // kvh)."""
    q = q.astype(np.float64).reshape(qh, hd)
    k = k.astype(np.float64)[: n * kvh * hd].reshape(n, kvh, hd)
    v = v.astype(np.float64)[: n * kvh * hd].reshape(n, kvh, hd)
    group = qh // kvh
    out = np.zeros((qh, hd))
    for h in range(qh):
        g = h // group
        s = k[:, g, :] @ q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, g, :]
    return out


# ── conversions ──────────────────────────────────────────────────────────────────────────────────────

def test_half_to_float_every_half(oracle):
    allh = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = allh.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([oracle.half_to_float(int(h)) for h in allh], np.float32).view(np.uint32)
    # a signalling NaN comes back quiet: ctypes returns the float through a Python double. Payload and sign
    # must still be the half's (mantissa << 13)
    nan = np.isnan(allh.view(np.float16))
    assert np.array_equal(got[~nan], want[~nan])
    assert np.array_equal(got[nan] | 0x00400000, want[nan] | 0x00400000)


def test_float_to_half_sample_and_boundaries(oracle):
    rng = np.random.default_rng(11)
    sample = rng.integers(0, 1 << 32, 150_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # every half's neighbourhood: the half itself, the midpoints to its neighbours (ties) and one float past
    h = np.arange(0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    edges = np.concatenate([h, mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0)),
                            np.array([65504, 65519.99, 65520, 65536, 1e30, np.inf, -np.inf, np.nan, 5.96e-8,
                                      2.98e-8, 2.99e-8, 1e-10, 0.0, -0.0], np.float32)])
    f = np.concatenate([sample, edges, -edges])
    with np.errstate(over="ignore"):
        want = f.astype(np.float16)
    for x, w in zip(f, want):
        hb, over = oracle.float_to_half(float(x))
        wb = int(w.view(np.uint16))
        if np.isnan(x):
            assert (hb & 0x7C00) == 0x7C00 and (hb & 0x3FF) != 0
        else:
            assert hb == wb, (float(x), hex(hb), hex(wb))
        assert over == (bool(np.isfinite(x)) and bool(np.isinf(w))), float(x)


# ── brute force ──────────────────────────────────────────────────────────────────────────────────────

SHAPES = [(6, 3, 16, 13), (8, 2, 32, 40), (4, 4, 8, 7), (16, 2, 64, 100), (3, 1, 10, 5)]


@pytest.mark.parametrize("qh,kvh,hd,n", SHAPES)
def test_decode_routes_against_float64(oracle, qh, kvh, hd, n):
    q, k, v = inputs(100 + n, (qh * hd,), (n * kvh * hd,), (n * kvh * hd,))
    want = brute_decode(q, k, v, qh, kvh, hd, n)
    # scores + mix (nn__attention__decode)
    p = oracle.scores(q, k, qh, kvh, hd, n)
    o, over = oracle.mix(p, v, qh, kvh, hd, n)
    assert over == 0
    near(o, want)
    # weights + residual_mix + finish (the split-K residual route)
    wp, res = oracle.weights(q, k, qh, kvh, hd, n)
    res = oracle.residual_mix(res, wp, v, qh, kvh, hd, n)
    o2, over = oracle.finish(res, qh, hd)
    assert over == 0
    near(o2, want)
    # scores_grouped (raw scores) + softmax_rows, then mix
    g = oracle.softmax_rows(oracle.scores_grouped(q, k, qh, kvh, hd, n), qh, n)
    o3, _ = oracle.mix(g, v, qh, kvh, hd, n)
    near(o3, want)


@pytest.mark.parametrize("qh,kvh,hd,first,rows", [(6, 3, 16, 0, 9), (8, 2, 32, 5, 12), (4, 1, 8, 20, 3)])
def test_causal_routes_against_float64(oracle, qh, kvh, hd, first, rows):
    n = first + rows
    q, k, v = inputs(200 + n, (rows * qh * hd,), (n * kvh * hd,), (n * kvh * hd,))
    want = np.stack([brute_decode(q[r * qh * hd:(r + 1) * qh * hd], k, v, qh, kvh, hd, first + r + 1)
                     for r in range(rows)])
    p = oracle.causal_scores(q, k, qh, kvh, hd, first, rows)
    o, over = oracle.causal_mix(p, v, qh, kvh, hd, first, rows)
    assert over == 0
    near(o, want)
    g = oracle.causal_softmax(oracle.causal_scores_grouped(q, k, qh, kvh, hd, first, rows), qh, first, rows)
    o2, _ = oracle.causal_mix(g, v, qh, kvh, hd, first, rows)
    near(o2, want)
    o3, _ = oracle.causal_rows(q, k, v, None, 0, qh, kvh, hd, first, np.arange(rows))
    near(o3, want)


# ── closed forms ─────────────────────────────────────────────────────────────────────────────────────

def test_one_position_gives_v_exactly(oracle):
    qh, kvh, hd = 8, 2, 64
    q, k, v = inputs(7, (qh * hd,), (kvh * hd,), (kvh * hd,))
    p = oracle.scores(q, k, qh, kvh, hd, 1)
    assert np.all(p == 1.0)
    o, _ = oracle.mix(p, v, qh, kvh, hd, 1)
    want = np.repeat(v.reshape(kvh, 1, hd), qh // kvh, axis=1).reshape(-1)
    assert np.array_equal(o.view(np.uint16), want.view(np.uint16))
    wp, res = oracle.weights(q, k, qh, kvh, hd, 1)
    o2, _ = oracle.finish(oracle.residual_mix(res, wp, v, qh, kvh, hd, 1), qh, hd)
    assert np.array_equal(o2.view(np.uint16), want.view(np.uint16))


def test_identical_keys_give_the_mean_of_v(oracle):
    qh, kvh, hd, n = 4, 2, 32, 50
    q, k1, v = inputs(8, (qh * hd,), (kvh * hd,), (n * kvh * hd,))
    k = np.tile(k1, n)
    p = oracle.scores(q, k, qh, kvh, hd, n).reshape(qh, n)
    assert np.allclose(p, 1.0 / n, rtol=1e-6)
    o, _ = oracle.mix(p.ravel(), v, qh, kvh, hd, n)
    mean = v.astype(np.float64).reshape(n, kvh, hd).mean(axis=0)
    want = np.repeat(mean[:, None, :], qh // kvh, axis=1).reshape(-1)
    near(o, want)


def test_causal_row_is_decode_at_its_position(oracle):
    qh, kvh, hd, first, rows = 8, 2, 32, 17, 10
    n = first + rows
    q, k, v = inputs(9, (rows * qh * hd,), (n * kvh * hd,), (n * kvh * hd,))
    o, _ = oracle.causal_rows(q, k, v, None, 0, qh, kvh, hd, first, np.arange(rows))
    o = o.reshape(rows, -1)
    for r in range(rows):
        qr = q[r * qh * hd:(r + 1) * qh * hd]
        p = oracle.scores(qr, k, qh, kvh, hd, first + r + 1)
        d, _ = oracle.mix(p, v, qh, kvh, hd, first + r + 1)
        assert np.array_equal(o[r].view(np.uint16), d.view(np.uint16)), r


def test_merge_of_halves_is_the_whole(oracle):
    qh, kvh, hd, n, cut = 8, 2, 64, 90, 37
    q, k, v = inputs(10, (qh * hd,), (n * kvh * hd,), (n * kvh * hd,))
    row = kvh * hd

    def residual(lo, hi):
        wp, res = oracle.weights(q, k[lo * row:hi * row], qh, kvh, hd, hi - lo)
        return oracle.residual_mix(res, wp, v[lo * row:hi * row], qh, kvh, hd, hi - lo)
    a, b = residual(0, cut), residual(cut, n)
    whole = residual(0, n)
    m = oracle.merge(a, b, qh, hd)
    np.testing.assert_allclose(m, whole, rtol=2e-6, atol=1e-6)
    # merge is symmetric
    np.testing.assert_allclose(oracle.merge(b, a, qh, hd), m, rtol=1e-6, atol=1e-7)
    o, _ = oracle.finish(m, qh, hd)
    near(o, brute_decode(q, k, v, qh, kvh, hd, n))


# ── pages ────────────────────────────────────────────────────────────────────────────────────────────

def test_permuted_pages_give_the_contiguous_bits(oracle):
    qh, kvh, hd, ps, rows = 8, 2, 32, 16, 3
    lens = np.array([50, 16, 33], np.uint32)
    npages = [(int(x) + ps - 1) // ps for x in lens]
    pages_row = max(npages)
    pool = sum(npages)
    row = kvh * hd
    q, k, v = inputs(12, (rows * qh * hd,), (pool * ps * row,), (pool * ps * row,))
    rng = np.random.default_rng(13)
    perm = rng.permutation(pool).astype(np.uint32)
    table = np.zeros(rows * pages_row, np.uint32)
    at = 0
    for u in range(rows):
        table[u * pages_row:u * pages_row + npages[u]] = perm[at:at + npages[u]]
        at += npages[u]
    o, over = oracle.decode_paged(q, k, v, table, pages_row, ps, 0, lens, qh, kvh, hd, rows)
    assert over == 0
    o = o.reshape(rows, -1)
    kk, vv = k.reshape(pool, ps * row), v.reshape(pool, ps * row)
    for u in range(rows):
        pg = table[u * pages_row:u * pages_row + npages[u]]
        kc, vc = kk[pg].reshape(-1), vv[pg].reshape(-1)
        p = oracle.scores(q[u * qh * hd:(u + 1) * qh * hd], kc, qh, kvh, hd, int(lens[u]))
        d, _ = oracle.mix(p, vc, qh, kvh, hd, int(lens[u]))
        assert np.array_equal(o[u].view(np.uint16), d.view(np.uint16)), u
