"""Deferred door chains in the CPU emulation (tests/emu): the reference verbs' chains — attention_scores then
attention_mix, attention_weights then attention_residual_mix, attention_causal_scores_grouped then
attention_causal_softmax then attention_causal_mix — called through the library's doors as the verbs call them.

- Deferred (the default) the chain runs fused, and the weights buffer shows it: untouched by the causal chain, the
  split-K scratch (no weights) after the decode pairs; the answers meet the oracle at the fp16 bar, the residual
  at tests/conftest.py::residual_parity's.
- A pair too short for its splits to fit the weights buffer, another door inside the chain, and deferral switched
  off all run each door on its own: the buffer then holds the oracle's weights.
"""
import numpy as np
import pytest

from tests.conftest import parity, residual_parity
from tests.emu import emu

pytestmark = pytest.mark.skipif(emu.compiler() is None, reason="no clang++ for the CPU emulation")


def _inputs(seed, qh, kvh, hd, n, rows=1):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(rows * qh * hd).astype(np.float16)
    k = rng.standard_normal(n * kvh * hd).astype(np.float16)
    v = rng.standard_normal(n * kvh * hd).astype(np.float16)
    return q, k, v


@pytest.mark.parametrize("qh,kvh,hd,length,interleave,defer,fused", [
    (16, 2, 256, 2048, False, True, True),    # fused: the splits fit the weights buffer
    (16, 2, 256, 2048, True, True, False),    # another door between: each door on its own
    (16, 2, 256, 2048, False, False, False),  # deferral off
    (8, 2, 128, 40, False, True, False),      # too short for the splits to fit: each door on its own
    (32, 1, 512, 600, False, True, True),     # one kv head, head_dim 512, two head blocks
])
def test_decode_pair(oracle, qh, kvh, hd, length, interleave, defer, fused):
    q, k, v = _inputs(qh + hd + length, qh, kvh, hd, length)
    o, p, _, over, _ = emu.run_chain("decode", q, k, v, qh, kvh, hd, length, interleave=interleave, defer=defer)
    want_p = oracle.scores(q, k, qh, kvh, hd, length)
    want_o, _ = oracle.mix(want_p, v, qh, kvh, hd, length)
    parity(o, want_o)
    assert over == 0
    if fused:
        assert not np.allclose(p, want_p, rtol=1e-4, atol=1e-6, equal_nan=False)
    else:
        np.testing.assert_allclose(p, want_p, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("qh,kvh,hd,length,interleave,fused", [
    (16, 2, 128, 3000, False, True),
    (16, 2, 128, 3000, True, False),
])
def test_weights_pair(oracle, qh, kvh, hd, length, interleave, fused):
    q, k, v = _inputs(7 + length, qh, kvh, hd, length)
    _, p, res, _, _ = emu.run_chain("weights", q, k, v, qh, kvh, hd, length, interleave=interleave)
    wp, wres = oracle.weights(q, k, qh, kvh, hd, length)
    wres = oracle.residual_mix(wres, wp, v, qh, kvh, hd, length)
    residual_parity(res, wres, hd)
    if fused:
        assert not np.allclose(p, wp, rtol=1e-4, atol=1e-6)
    else:
        np.testing.assert_allclose(p, wp, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("qh,kvh,hd,first,rows,interleave,route,shared", [
    (16, 2, 256, 77, 95, False, "mfma", False),    # causal_mfma: the weights never written
    (6, 3, 128, 10, 30, True, "doors", False),     # another door inside: each door on its own
    (8, 1, 512, 530, 3, False, "decode", False),   # head_dim 512: each row a decode over the same cache
    (20, 1, 512, 530, 2, False, "decode", True),   # latent attention's block prefill: the latents are k and v
    (8, 1, 512, 5, 20, False, "doors", False),     # a prefix too short for the splits to fit: door by door
])
def test_causal_chain(oracle, qh, kvh, hd, first, rows, interleave, route, shared):
    q, k, v = _inputs(first + rows, qh, kvh, hd, first + rows, rows)
    if shared:
        v = k
    o, p, over, _ = emu.run_chain("causal", q, k, None if shared else v, qh, kvh, hd, first, rows,
                                  interleave=interleave)
    want, _ = oracle.causal_rows(q, k, v, None, 0, qh, kvh, hd, first, list(range(rows)))
    parity(o, want)
    assert over == 0
    wp = oracle.causal_softmax(oracle.causal_scores_grouped(q, k, qh, kvh, hd, first, rows), qh, first, rows)
    # row r's weights are its first + r + 1 positions; past them the buffer keeps what it held
    span = first + rows
    valid = (np.arange(span)[None, :] <= first + np.repeat(np.arange(rows), qh)[:, None]).ravel()
    if route == "mfma":
        assert np.all(p.view(np.uint32) == 0xFFFFFFFF)   # the weights were never written
    elif route == "decode":
        assert not np.allclose(p[valid], wp[valid], rtol=1e-4, atol=1e-6)   # the buffer held the splits' scratch
    else:
        np.testing.assert_allclose(p[valid], wp[valid], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("first,rows,interleave,fused", [(100, 20, False, True), (100, 20, True, False)])
def test_weights_rows_pair(oracle, first, rows, interleave, fused):
    """weights_rows + residual_mix_rows (the tiered prefill window's part 0) as the causal residual (row 140)."""
    qh, kvh, hd = 8, 2, 256
    q, k, v = _inputs(first + rows + 5, qh, kvh, hd, first + rows, rows)
    p, res, _, _ = emu.run_chain_residual("rows", q, k, None, v, None, qh, kvh, hd, first, rows=rows,
                                          interleave=interleave)
    wp, wres = oracle.weights_rows(q, k, qh, kvh, hd, first, rows)
    wres = oracle.residual_mix_rows(wres, wp, v, qh, kvh, hd, first, rows)
    residual_parity(res, wres, hd)
    if fused:
        assert np.all(p.view(np.uint32) == 0xFFFFFFFF)
    else:
        assert not np.all(p.view(np.uint32) == 0xFFFFFFFF)


@pytest.mark.parametrize("kind,d,hd,length,rows,interleave,fused", [
    ("tq", 8, 128, 3000, 1, False, True),       # a tier's residual (the tiers' verbs)
    ("tq", 4, 128, 3000, 1, True, False),
    ("tq_rows", 4, 64, 2000, 3, False, True),   # the tiered prefill window's tier part
])
def test_tq_pair(oracle, kind, d, hd, length, rows, interleave, fused):
    from tests.test_tq import header_levels, make
    qh, kvh = 8, 2
    rng = np.random.default_rng(d + hd + length + rows)
    lev = header_levels(d)
    q, kc, ks = make(rng, qh, kvh, hd, length, d, rows=rows)
    _, vc, vs = make(rng, qh, kvh, hd, length, d)
    p, res, _, _ = emu.run_chain_residual(kind, q, kc, ks, vc, vs, qh, kvh, hd, length, rows=rows, d=d,
                                          interleave=interleave)
    wp, wres = oracle.weights_tq_rows(q, kc, ks, qh, kvh, hd, length, d, rows, lev)
    wres = oracle.residual_mix_tq_rows(wres, wp, vc, vs, qh, kvh, hd, length, d, rows, lev)
    # the fused form's keys go through the matrix cores as fp16 (level · scale rounded): m to that rounding
    w = hd + 2
    g, o = res.reshape(-1, w).astype(np.float64), wres.reshape(-1, w).astype(np.float64)
    np.testing.assert_allclose(g[:, 0], o[:, 0], rtol=0, atol=2e-3 * max(1.0, float(np.abs(o[:, 0]).max())))
    at = np.exp(g[:, 0] - o[:, 0])[:, None]
    np.testing.assert_allclose(g[:, 1:2] * at, o[:, 1:2], rtol=2e-3)
    np.testing.assert_allclose(g[:, 2:] * at, o[:, 2:], rtol=0, atol=4e-3 * float(np.abs(o[:, 2:]).max()))
    if not fused:   # each door on its own: the oracle's residual to the doors' own bar
        np.testing.assert_allclose(res, wres, rtol=1e-4, atol=1e-5 * float(np.abs(wres).max()))


@pytest.mark.parametrize("qh,hd,length,sink,interleave,fused", [
    (16, 512, 1100, False, False, True),   # GLM 5.3: scores_grouped, softmax_rows, mix over the latents
    (16, 512, 1100, True, False, True),    # DeepSeek V4: the softmax with a sink
    (16, 512, 1100, True, True, False),    # another door inside: each door on its own
])
def test_grouped_chain(oracle, qh, hd, length, sink, interleave, fused):
    """Latent attention's chain (one kv head, the latents as keys and values) through the library's doors."""
    rng = np.random.default_rng(qh + length + sink)
    q = rng.standard_normal(qh * hd).astype(np.float16)
    lat = rng.standard_normal(length * hd).astype(np.float16)
    s = (rng.standard_normal(qh) * 2 + 1).astype(np.float16).view(np.uint16) if sink else None
    o, p, over, _ = emu.run_chain_grouped(q, lat, None, qh, 1, hd, length, sink=s, interleave=interleave)
    raw = oracle.scores_grouped(q, lat, qh, 1, hd, length)
    wp = oracle.softmax_sink(raw, s, qh, length) if sink else oracle.softmax_rows(raw, qh, length)
    want, _ = oracle.mix(wp, lat, qh, 1, hd, length)
    parity(o, want)
    assert over == 0
    if fused:
        assert not np.allclose(p, wp, rtol=1e-4, atol=1e-6)
    else:
        np.testing.assert_allclose(p, wp, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("interleave,fused", [(False, True), (True, False)])
def test_grouped_rows_chain(oracle, interleave, fused):
    """GLM 5.3's block of rows over their gathered latents (layer__abi.cuh:1037-1043): scores_grouped_rows,
    softmax_lens, mix_rows as one split-K decode of every row, the weights buffer its scratch."""
    qh, hd, lens = 16, 512, [1100, 1, 700]
    most, rows = max(lens), len(lens)
    rng = np.random.default_rng(11 + interleave)
    q = rng.standard_normal(rows * qh * hd).astype(np.float16)
    lat = rng.standard_normal(rows * most * hd).astype(np.float16)
    lens_np = np.asarray(lens, np.uint32)
    o, p, over, _ = emu.run_chain_grouped_rows(q, lat, lens_np, qh, hd, most, interleave=interleave)
    p_row = qh * most
    raw = oracle.scores_grouped_rows(p_row, q, qh * hd, lat, most * hd, lens_np, qh, 1, hd, most, rows)
    wp = oracle.softmax_lens(raw, p_row, lens_np, qh, rows)
    want, _ = oracle.mix_rows(qh * hd, wp, p_row, lat, most * hd, lens_np, qh, 1, hd, rows)
    parity(o, want)
    assert over == 0
    valid = np.concatenate([np.r_[np.ones(qh * n, bool), np.zeros(p_row - qh * n, bool)] for n in lens])
    if fused:
        assert not np.allclose(p[valid], wp[valid], rtol=1e-4, atol=1e-6)
    else:
        np.testing.assert_allclose(p[valid], wp[valid], rtol=1e-4, atol=1e-6)


INLINE = {"SILVANN_GFX950_DECODE_INLINE": "1", "EMU_LAUNCHES": "1"}
PLANS = ("decode_plan", "causal_lens")   # decode_plan_one too


def _launched(log):
    return [ln[len("emu launch "):] for ln in log.splitlines() if ln.startswith("emu launch ")]


@pytest.mark.parametrize("kind,qh,kvh,hd,a0,a1,shared", [
    ("decode", 16, 2, 256, 2048, 0, False),   # the decode verb's pair, one query of a host length
    ("decode", 32, 1, 512, 600, 0, False),    # head_dim 512, two head blocks
    ("weights", 16, 2, 128, 3000, 0, False),  # the residual pair: the merge writes the residual
    ("causal", 8, 1, 512, 530, 3, False),     # head_dim 512 rows: lengths first + u + 1 made in the kernel
    ("causal", 20, 1, 512, 530, 2, True),     # latent block prefill, keys = values
])
def test_chains_with_inline_plan(oracle, kind, qh, kvh, hd, a0, a1, shared):
    """The fused decode routes with the plan made inside decode_split (SILVANN_GFX950_DECODE_INLINE=1): the same
    answers, and no plan or length kernel launched (the emulation's launch log)."""
    rows = a1 or 1
    n = a0 + a1 if kind == "causal" else a0
    q, k, v = _inputs(qh + hd + n + 1, qh, kvh, hd, n, rows)
    if shared:
        v = k
    if kind == "causal":
        o, p, over, log = emu.run_chain("causal", q, k, None if shared else v, qh, kvh, hd, a0, a1,
                                        extra_env=INLINE)
        want, _ = oracle.causal_rows(q, k, v, None, 0, qh, kvh, hd, a0, list(range(a1)))
        parity(o, want)
    else:
        o, p, res, over, log = emu.run_chain(kind, q, k, v, qh, kvh, hd, a0, extra_env=INLINE)
        if kind == "decode":
            want_o, _ = oracle.mix(oracle.scores(q, k, qh, kvh, hd, a0), v, qh, kvh, hd, a0)
            parity(o, want_o)
        else:
            wp, wres = oracle.weights(q, k, qh, kvh, hd, a0)
            residual_parity(res, oracle.residual_mix(wres, wp, v, qh, kvh, hd, a0), hd)
    assert over == 0
    launched = _launched(log)
    assert any("decode_split" in x for x in launched), launched
    assert not [x for x in launched if x.startswith(PLANS)], launched


def test_latent_chains_with_inline_plan(oracle):
    """Latent attention's decode chain (scores_grouped, softmax_sink, mix) and block chain (scores_grouped_rows,
    softmax_lens, mix_rows) with the plan made inside decode_split."""
    qh, hd, length = 16, 512, 1100
    rng = np.random.default_rng(5)
    q = rng.standard_normal(qh * hd).astype(np.float16)
    lat = rng.standard_normal(length * hd).astype(np.float16)
    s = (rng.standard_normal(qh) * 2 + 1).astype(np.float16).view(np.uint16)
    o, _, over, log = emu.run_chain_grouped(q, lat, None, qh, 1, hd, length, sink=s, extra_env=INLINE)
    wp = oracle.softmax_sink(oracle.scores_grouped(q, lat, qh, 1, hd, length), s, qh, length)
    parity(o, oracle.mix(wp, lat, qh, 1, hd, length)[0])
    assert over == 0 and not [x for x in _launched(log) if x.startswith(PLANS)]

    lens = np.asarray([1100, 1, 700], np.uint32)
    most, rows = int(lens.max()), len(lens)
    q = rng.standard_normal(rows * qh * hd).astype(np.float16)
    lat = rng.standard_normal(rows * most * hd).astype(np.float16)
    o, _, over, log = emu.run_chain_grouped_rows(q, lat, lens, qh, hd, most, extra_env=INLINE)
    p_row = qh * most
    raw = oracle.scores_grouped_rows(p_row, q, qh * hd, lat, most * hd, lens, qh, 1, hd, most, rows)
    wp = oracle.softmax_lens(raw, p_row, lens, qh, rows)
    parity(o, oracle.mix_rows(qh * hd, wp, p_row, lat, most * hd, lens, qh, 1, hd, rows)[0])
    assert over == 0 and not [x for x in _launched(log) if x.startswith(PLANS)]


@pytest.mark.parametrize("qh,kvh,hd,length", [(16, 2, 256, 2048), (8, 2, 128, 3000), (8, 8, 64, 700)])
def test_decode_pair_in_one_launch(oracle, qh, kvh, hd, length):
    """The decode verb's pair (attention_scores + attention_mix) with the fused finish and the inline plan on: one
    decode_split launch, its finished-split counts tagged in the weights buffer (whatever it held), the answers the
    oracle's."""
    q, k, v = _inputs(qh + hd + length + 2, qh, kvh, hd, length)
    env = {**INLINE, "SILVANN_GFX950_DECODE_FUSED": "1"}
    o, p, _, over, log = emu.run_chain("decode", q, k, v, qh, kvh, hd, length, extra_env=env)
    want_o, _ = oracle.mix(oracle.scores(q, k, qh, kvh, hd, length), v, qh, kvh, hd, length)
    parity(o, want_o)
    assert over == 0
    launched = _launched(log)
    assert len(launched) == 1 and "decode_split" in launched[0], launched


@pytest.mark.parametrize("kind,misalign", [("decode", "q"), ("decode", "p"), ("causal", "q")])
def test_unaligned_operands_run_door_by_door(oracle, kind, misalign):
    """The fused forms read q, K and V in 16-byte vectors and keep 64-bit counters in the weights buffer: a q at
    2 mod 16, or a weights buffer at 4 mod 8, makes the chain run door by door (the buffer then holds the oracle's
    weights) with the same answers."""
    env = {"EMU_MISALIGN": misalign}
    if kind == "decode":
        qh, kvh, hd, length = 16, 2, 256, 2048
        q, k, v = _inputs(91, qh, kvh, hd, length)
        o, p, _, over, _ = emu.run_chain("decode", q, k, v, qh, kvh, hd, length, extra_env=env)
        want_p = oracle.scores(q, k, qh, kvh, hd, length)
        want_o, _ = oracle.mix(want_p, v, qh, kvh, hd, length)
    else:
        qh, kvh, hd, first, rows = 8, 2, 64, 10, 40
        q, k, v = _inputs(92, qh, kvh, hd, first + rows, rows)
        o, p, over, _ = emu.run_chain("causal", q, k, v, qh, kvh, hd, first, rows, extra_env=env)
        want_o, _ = oracle.causal_rows(q, k, v, None, 0, qh, kvh, hd, first, list(range(rows)))
        want_p = oracle.causal_softmax(oracle.causal_scores_grouped(q, k, qh, kvh, hd, first, rows), qh, first, rows)
        # row r's weights are its first + r + 1 positions; past them the buffer keeps what it held
        valid = (np.arange(first + rows)[None, :] <= first + np.repeat(np.arange(rows), qh)[:, None]).ravel()
        p, want_p = p[valid], want_p[valid]
    parity(o, want_o)
    assert over == 0
    np.testing.assert_allclose(p, want_p, rtol=1e-4, atol=1e-6)
