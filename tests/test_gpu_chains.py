"""Deferred door chains on gfx950 (the same checks as tests/test_chains.py, on the GPU through the C ABI), at the
BASELINE shapes: the reference's decode verb (attention_scores + attention_mix) over C1 and C5's caches, its
residual verb (attention_weights + attention_residual_mix), its rows verb (causal_scores_grouped + causal_softmax +
causal_mix in passes) over C3's chunk and its tiers' verb (attention_weights_tq + attention_residual_mix_tq) — each
fused, against the oracle at the fp16 bar (tests/test_gpu_window.py runs the window's many-row pairs); and the
orders that must run each door on its own (another door inside the chain, a flush, a change of stream, deferral
off), whose weights buffer then holds the oracle's weights.
"""
import numpy as np
import pytest
import torch

from oracle.oracle import inputs
from silvann_amd import doors, verbs
from silvann_amd import workloads as W
from tests.conftest import parity, residual_parity
from tests.gpu_util import t

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def deferral_on(dev):
    doors.set_defer(True)
    yield
    doors.flush()


def _z(dev, n, dtype=torch.float32):
    return torch.zeros(n, dtype=dtype, device=dev)


def _decode_case(seed, qh, kvh, hd, L):
    return inputs(seed, (qh * hd,), (L * kvh * hd,), (L * kvh * hd,))


@pytest.mark.parametrize("name,seed,qh,kvh,hd,L", [
    ("C1", 1, 16, 2, 256, 2048),
    ("C5", 5, 16, 2, 256, 262144),
    ("mqa", 9, 32, 1, 128, 5000),
])
def test_decode_verb_runs_fused(dev, oracle, name, seed, qh, kvh, hd, L):
    print(f"case: decode verb chain {name} qh{qh} kvh{kvh} hd{hd} L{L}", flush=True)
    q, k, v = _decode_case(seed, qh, kvh, hd, L)
    scores, out, over = _z(dev, qh * L), _z(dev, qh * hd, torch.float16), _z(dev, 1, torch.int32)
    verbs.decode(t(q, dev), t(k, dev), t(v, dev), scores, out, qh, kvh, hd, 0, L, over)
    want_p = oracle.scores(q, k, qh, kvh, hd, L)
    want_o, _ = oracle.mix(want_p, v, qh, kvh, hd, L)
    parity(out.cpu().numpy(), want_o)
    assert int(over.item()) == 0
    # fused: the scores buffer held the splits' scratch, never the weights
    assert not np.allclose(scores.cpu().numpy(), want_p, rtol=1e-4, atol=1e-6)
    assert not doors.launch_failed()


def test_residual_verb_runs_fused(dev, oracle):
    qh, kvh, hd, L = 16, 2, 128, 30000
    print("case: residual verb chain", flush=True)
    q, k, v = _decode_case(31, qh, kvh, hd, L)
    scores, res = _z(dev, qh * L), _z(dev, qh * (hd + 2))
    verbs.residual(t(q, dev), t(k, dev), t(v, dev), scores, res, qh, kvh, hd, 0, L)
    wp, wres = oracle.weights(q, k, qh, kvh, hd, L)
    wres = oracle.residual_mix(wres, wp, v, qh, kvh, hd, L)
    residual_parity(res.cpu().numpy(), wres, hd)
    assert not doors.launch_failed()


def test_rows_verb_runs_fused(dev, oracle):
    """C3's chunk through nn__attention__rows' attention part: passes of causal_scores_grouped, causal_softmax,
    causal_mix, each pass one fused causal launch."""
    w = W.config3()
    print("case: rows verb chain C3", flush=True)
    qh, kvh, hd, rows = w.q_heads, w.kv_heads, w.head_dim, w.rows
    scores = _z(dev, 256 * qh * rows)   # room for passes of 256 rows
    att = _z(dev, rows * qh * hd, torch.float16)
    over = _z(dev, 1, torch.int32)
    verbs.rows_attention(t(w.q, dev), t(w.k, dev), t(w.v, dev), scores, att, qh, kvh, hd, 0, rows, over)
    which = [0, 1, 255, 256, 2047, rows - 1]
    want, _ = oracle.causal_rows(w.q, w.k, w.v, None, 0, qh, kvh, hd, 0, which)
    got = att.cpu().numpy().reshape(rows, qh * hd)[which].ravel()
    parity(got, want)
    assert int(over.item()) == 0
    assert torch.count_nonzero(scores) == 0   # the weights were never written
    assert not doors.launch_failed()


@pytest.mark.parametrize("between", ["door", "flush", "stream", "off"])
def test_orders_that_run_each_door_alone(dev, oracle, between):
    qh, kvh, hd, L = 16, 2, 256, 2048
    print(f"case: decode chain with {between} between", flush=True)
    q, k, v = _decode_case(41, qh, kvh, hd, L)
    scores, out, over = _z(dev, qh * L), _z(dev, qh * hd, torch.float16), _z(dev, 1, torch.int32)
    if between == "off":
        doors.set_defer(False)
    doors.attention_scores(scores, t(q, dev), t(k, dev), qh, kvh, hd, L)
    if between == "door":
        r = _z(dev, 2 * (hd + 2))
        doors.attention_merge(r, r, r[hd + 2:], 1, hd)
    elif between == "flush":
        doors.flush()
    elif between == "stream":
        s = torch.cuda.Stream()
        doors.set_stream(s)
        doors.set_stream(None)
        s.synchronize()
    want_p = oracle.scores(q, k, qh, kvh, hd, L)
    torch.cuda.synchronize()
    np.testing.assert_allclose(scores.cpu().numpy(), want_p, rtol=1e-5, atol=1e-7)
    doors.attention_mix(out, scores, t(v, dev), qh, kvh, hd, L, over)
    want_o, _ = oracle.mix(want_p, v, qh, kvh, hd, L)
    parity(out.cpu().numpy(), want_o)
    doors.set_defer(True)
    assert not doors.launch_failed()


@pytest.mark.parametrize("d,length", [(4, 70000), (8, 3000)])
def test_tier_verb_runs_fused(dev, oracle, d, length):
    """The tiers' verb (nn__attention__residual_tq: weights_tq then residual_mix_tq) as row 139, the weights buffer
    its scratch."""
    from tests.test_tq import header_levels, make
    qh, kvh, hd = 16, 2, 256
    print(f"case: tier verb chain d{d} length{length}", flush=True)
    rng = np.random.default_rng(d + length)
    lev = header_levels(d)
    q, kc, ks = make(rng, qh, kvh, hd, length, d)
    _, vc, vs = make(rng, qh, kvh, hd, length, d)
    scores, res = _z(dev, 2 * qh * length), _z(dev, qh * (hd + 2))
    verbs.residual_tq(t(q, dev), t(kc, dev), t(ks, dev), t(vc, dev), t(vs, dev), scores, res, qh, kvh, hd, d, length)
    wp, wres = oracle.weights_tq(q, kc, ks, qh, kvh, hd, length, d, lev)
    wres = oracle.residual_mix_tq(wres, wp, vc, vs, qh, kvh, hd, length, d, lev)
    w = hd + 2
    g, o = res.cpu().numpy().reshape(-1, w).astype(np.float64), wres.reshape(-1, w).astype(np.float64)
    np.testing.assert_allclose(g[:, 0], o[:, 0], rtol=0, atol=2e-3 * max(1.0, float(np.abs(o[:, 0]).max())))
    at = np.exp(g[:, 0] - o[:, 0])[:, None]
    fin = lambda r: (r[:, 2:] / r[:, 1:2]).astype(np.float16)  # noqa: E731
    np.testing.assert_allclose(g[:, 1:2] * at, o[:, 1:2], rtol=2e-3)
    parity(fin(g), fin(o))
    assert not doors.launch_failed()


def test_latent_block_prefill_runs_fused(dev, oracle):
    """GLM 5.3's block prefill chain (ai_z__glm_5_3/cpu/opcodes/layer__abi.cuh:1004-1009): causal_scores_grouped,
    causal_softmax, causal_mix with one kv head, head_dim 512, the latent cache as both keys and values — each row a
    split-K decode over the same cache, the weights buffer its scratch."""
    heads, lat, first, rows = 64, 512, 5000, 64
    print("case: latent block prefill chain", flush=True)
    rng = np.random.default_rng(77)
    q = rng.standard_normal(rows * heads * lat).astype(np.float16)
    cache = rng.standard_normal((first + rows) * lat).astype(np.float16)
    qd, cd = t(q, dev), t(cache, dev)
    p = _z(dev, rows * heads * (first + rows))
    o = _z(dev, rows * heads * lat, torch.float16)
    over = _z(dev, 1, torch.int32)
    doors.attention_causal_scores_grouped(p, qd, cd, heads, 1, lat, first, rows)
    doors.attention_causal_softmax(p, heads, first, rows)
    doors.attention_causal_mix(o, p, cd, heads, 1, lat, first, rows, over)
    which = [0, 1, 31, rows - 1]
    want, _ = oracle.causal_rows(q, cache, cache, None, 0, heads, 1, lat, first, which)
    got = o.cpu().numpy().reshape(rows, heads * lat)[which].ravel()
    parity(got, want)
    assert int(over.item()) == 0
    assert not doors.launch_failed()


@pytest.mark.parametrize("heads,length,sink", [(64, 2048, False), (64, 2048, True), (16, 100000, True)])
def test_latent_decode_chain_runs_fused(dev, oracle, heads, length, sink):
    """Latent attention's decode chain: GLM 5.3's scores_grouped, softmax_rows, mix (layer__abi.cuh:283-289) and
    DeepSeek V4's with softmax_sink (ai_deepseek_4/cpu/opcodes/layer__abi.cuh:299-301), one kv head, 512-wide
    latents as keys and values — as one split-K decode, the sink folded into its merge."""
    hd = 512
    print(f"case: latent decode chain heads{heads} length{length} sink{sink}", flush=True)
    rng = np.random.default_rng(heads + length + sink)
    q = rng.standard_normal(heads * hd).astype(np.float16)
    lat = rng.standard_normal(length * hd).astype(np.float16)
    s = (rng.standard_normal(heads) * 2 + 1).astype(np.float16).view(np.uint16)
    qd, ld = t(q, dev), t(lat, dev)
    p = _z(dev, heads * length)
    o = _z(dev, heads * hd, torch.float16)
    over = _z(dev, 1, torch.int32)
    doors.attention_scores_grouped(p, qd, ld, heads, 1, hd, length)
    if sink:
        doors.attention_softmax_sink(p, t(s, dev), heads, length)
    else:
        doors.attention_softmax_rows(p, heads, length)
    doors.attention_mix(o, p, ld, heads, 1, hd, length, over)
    raw = oracle.scores_grouped(q, lat, heads, 1, hd, length)
    wp = oracle.softmax_sink(raw, s, heads, length) if sink else oracle.softmax_rows(raw, heads, length)
    want, _ = oracle.mix(wp, lat, heads, 1, hd, length)
    parity(o.cpu().numpy(), want)
    assert int(over.item()) == 0
    assert not np.allclose(p.cpu().numpy(), wp, rtol=1e-4, atol=1e-6)   # fused: no weights were written
    assert not doors.launch_failed()


@pytest.mark.parametrize("misalign", ["q", "p"])
def test_unaligned_decode_chain_runs_door_by_door(dev, oracle, misalign):
    """With deferral on, a q at 2 mod 16 (a view one half into its buffer) or a weights buffer at 4 mod 8 keeps the
    decode verb's pair off the fused kernel, whose 16-byte loads and 64-bit counters need alignment: each door runs
    on its own, the weights buffer holds the oracle's weights and the answers meet it."""
    qh, kvh, hd, L = 16, 2, 256, 2048
    print(f"case: decode chain, {misalign} misaligned", flush=True)
    q, k, v = _decode_case(43, qh, kvh, hd, L)
    qd = t(q, dev)
    if misalign == "q":
        qbuf = _z(dev, qh * hd + 8, torch.float16)
        qbuf[1:1 + qh * hd] = qd
        qd = qbuf[1:1 + qh * hd]
    sbuf = _z(dev, qh * L + 2)
    scores = sbuf[1:1 + qh * L] if misalign == "p" else sbuf[:qh * L]
    out, over = _z(dev, qh * hd, torch.float16), _z(dev, 1, torch.int32)
    assert (qd.data_ptr() % 16 != 0) == (misalign == "q") and (scores.data_ptr() % 8 != 0) == (misalign == "p")
    verbs.decode(qd, t(k, dev), t(v, dev), scores, out, qh, kvh, hd, 0, L, over)
    want_p = oracle.scores(q, k, qh, kvh, hd, L)
    want_o, _ = oracle.mix(want_p, v, qh, kvh, hd, L)
    parity(out.cpu().numpy(), want_o)
    assert int(over.item()) == 0
    np.testing.assert_allclose(scores.cpu().numpy(), want_p, rtol=1e-5, atol=1e-7)
    assert not doors.launch_failed()
