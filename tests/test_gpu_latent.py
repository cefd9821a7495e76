"""Latent attention (GLM 5.3's MLA: 64 query heads over 512-wide latents that are both keys and values) through row
137's shared-tile form, against the oracle's route of the reference's doors — scores_grouped_rows, softmax_lens,
mix_rows with one kv head (ai_z__glm_5_3/cpu/opcodes/layer__abi.cuh:1037-1043) — and against the library's own
three generic doors, at the fp16 bar (tests/conftest.py::parity).
"""
import numpy as np
import pytest
import torch

from silvann_amd import doors, verbs
from tests.conftest import parity
from tests.gpu_util import t

pytestmark = pytest.mark.gpu


def _oracle(oracle, q, lat, lens, heads, hd, most):
    rows = len(lens)
    p_row = heads * most
    p = oracle.scores_grouped_rows(p_row, q, heads * hd, lat, most * hd, lens, heads, 1, hd, most, rows)
    p = oracle.softmax_lens(p, p_row, lens, heads, rows)
    o, _ = oracle.mix_rows(heads * hd, p, p_row, lat, most * hd, lens, heads, 1, hd, rows)
    return o


@pytest.mark.parametrize("heads,hd,lens", [
    (64, 512, [2048]),                  # one decode query over the top-2048 gathered latents
    (64, 512, [2048, 1500, 37, 2048]),  # a block of prefill rows, each over its own gathered set
    (16, 512, [5000]),                  # a tensor-parallel share of the heads, a dense cache
    (32, 256, [900, 3]),
])
def test_latent_attention(dev, oracle, heads, hd, lens):
    print(f"case: latent heads{heads} hd{hd} lens{lens}", flush=True)
    rng = np.random.default_rng(heads + hd + len(lens))
    rows, most = len(lens), max(lens)
    q = rng.standard_normal(rows * heads * hd).astype(np.float16)
    lat = rng.standard_normal(rows * most * hd).astype(np.float16)
    lens_np = np.asarray(lens, np.uint32)
    want = _oracle(oracle, q, lat, lens_np, heads, hd, most)
    out = torch.zeros(rows * heads * hd, dtype=torch.float16, device=dev)
    verbs.latent_attention(t(q, dev), t(lat, dev), t(lens_np, dev), out, heads, hd, most, k_row=most * hd)
    got = out.cpu().numpy()
    parity(got, want)
    assert not doors.launch_failed()
    # the library's generic doors in the reference's order, each on its own, agree too
    doors.set_defer(False)
    qd, ld, lnd = t(q, dev), t(lat, dev), t(lens_np, dev)
    p = torch.zeros(rows * heads * most, dtype=torch.float32, device=dev)
    o2 = torch.zeros_like(out)
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    doors.attention_scores_grouped_rows(p, heads * most, qd, heads * hd, ld, most * hd, lnd, heads, 1, hd, most, rows)
    doors.attention_softmax_lens(p, heads * most, lnd, heads, rows)
    doors.attention_mix_rows(o2, heads * hd, p, heads * most, ld, most * hd, lnd, heads, 1, hd, rows, over)
    doors.set_defer(True)
    parity(got, o2.cpu().numpy())
    assert int(over.item()) == 0


def test_block_chain_runs_fused(dev, oracle):
    """The same doors called as GLM's block prefill calls them (layer__abi.cuh:1037-1043), deferral on: the chain
    runs as one split-K decode of every row, the weights buffer its scratch."""
    heads, hd, lens = 64, 512, [2048, 1, 1500, 2048]
    print("case: latent block chain", flush=True)
    rng = np.random.default_rng(5)
    rows, most = len(lens), max(lens)
    q = rng.standard_normal(rows * heads * hd).astype(np.float16)
    lat = rng.standard_normal(rows * most * hd).astype(np.float16)
    lens_np = np.asarray(lens, np.uint32)
    want = _oracle(oracle, q, lat, lens_np, heads, hd, most)
    qd, ld, lnd = t(q, dev), t(lat, dev), t(lens_np, dev)
    p = torch.zeros(rows * heads * most, dtype=torch.float32, device=dev)
    o = torch.zeros(rows * heads * hd, dtype=torch.float16, device=dev)
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    doors.set_defer(True)
    doors.attention_scores_grouped_rows(p, heads * most, qd, heads * hd, ld, most * hd, lnd, heads, 1, hd, most, rows)
    doors.attention_softmax_lens(p, heads * most, lnd, heads, rows)
    doors.attention_mix_rows(o, heads * hd, p, heads * most, ld, most * hd, lnd, heads, 1, hd, rows, over)
    parity(o.cpu().numpy(), want)
    assert int(over.item()) == 0
    p_row = heads * most
    wp = oracle.softmax_lens(oracle.scores_grouped_rows(p_row, q, heads * hd, lat, most * hd, lens_np, heads, 1, hd, most,
                                                        rows), p_row, lens_np, heads, rows)
    # fused: the buffer held the splits' scratch, not the weights
    assert not np.allclose(p.cpu().numpy()[: heads * lens[0]], wp[: heads * lens[0]], rtol=1e-4, atol=1e-6)
    assert not doors.launch_failed()
