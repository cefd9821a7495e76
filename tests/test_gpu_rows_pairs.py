"""One-row and many-row door pairs agree bit for bit on gfx950 (the reference's requirement of a family,
engine/src/silicon_families/add_a_family.md:51-55; kernels.cuh:952 "each the one-row door's to the bit"): the same
pairs and the same comparisons as tests/test_rows_pairs.py, on the GPU through the C ABI, at larger shapes.
"""
import numpy as np
import pytest
import torch

from silvann_amd import doors
from tests.gpu_util import t
from tests.test_tq import make

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def each_door_on_its_own(dev):
    """These tests read every door's buffers between doors, so no chain is deferred here (tests/test_gpu_chains.py
    covers the deferred chains)."""
    doors.set_defer(False)
    yield
    doors.set_defer(True)


def _z(dev, n, dtype=torch.float32):
    return torch.full((n,), float("nan"), dtype=dtype, device=dev)


def test_weights_rows_pair(dev):
    qh, kvh, hd, first, rows = 16, 2, 256, 700, 40
    print("case: weights_rows / residual_mix_rows against the one-row doors", flush=True)
    rng = np.random.default_rng(1)
    q = t(rng.standard_normal(rows * qh * hd).astype(np.float16), dev)
    k = t(rng.standard_normal((first + rows) * kvh * hd).astype(np.float16), dev)
    v = t(rng.standard_normal((first + rows) * kvh * hd).astype(np.float16), dev)
    span, rf = first + rows, hd + 2
    p, res = _z(dev, rows * qh * span), _z(dev, rows * qh * rf)
    doors.attention_weights_rows(p, res, q, k, qh, kvh, hd, first, rows)
    doors.attention_residual_mix_rows(res, p, v, qh, kvh, hd, first, rows)
    for u in (0, 1, 17, rows - 1):
        n = first + u + 1
        p1, r1 = _z(dev, qh * n), _z(dev, qh * rf)
        qu = q[u * qh * hd:(u + 1) * qh * hd]
        doors.attention_weights(p1, r1, qu, k, qh, kvh, hd, n)
        assert torch.equal(p[u * qh * span:u * qh * span + qh * n].view(torch.int32), p1.view(torch.int32)), u
        doors.attention_residual_mix(r1, p1, v, qh, kvh, hd, n)
        assert torch.equal(res[u * qh * rf:(u + 1) * qh * rf].view(torch.int32), r1.view(torch.int32)), u
    assert not doors.launch_failed()


@pytest.mark.parametrize("d,hd,length", [(4, 128, 5000), (8, 256, 900)])
def test_tq_rows_pair(dev, d, hd, length):
    qh, kvh, rows = 16, 2, 6
    print(f"case: tq rows pair d{d} hd{hd} length{length}", flush=True)
    rng = np.random.default_rng(d + hd)
    q, codes, scales = make(rng, qh, kvh, hd, length, d, rows=rows)
    qd, cd, sd = t(q, dev), t(codes, dev), t(scales, dev)
    rf = hd + 2
    p, res = _z(dev, rows * qh * length), _z(dev, rows * qh * rf)
    doors.attention_weights_tq_rows(p, res, qd, cd, sd, qh, kvh, hd, length, d, rows)
    p_keep = p.clone()
    doors.attention_residual_mix_tq_rows(res, p, cd, sd, qh, kvh, hd, length, d, rows)
    for u in range(rows):
        p1, r1 = _z(dev, qh * length), _z(dev, qh * rf)
        doors.attention_weights_tq(p1, r1, qd[u * qh * hd:(u + 1) * qh * hd], cd, sd, qh, kvh, hd, length, d)
        assert torch.equal(p_keep[u * qh * length:(u + 1) * qh * length].view(torch.int32), p1.view(torch.int32)), u
        doors.attention_residual_mix_tq(r1, p1, cd, sd, qh, kvh, hd, length, d)
        assert torch.equal(res[u * qh * rf:(u + 1) * qh * rf].view(torch.int32), r1.view(torch.int32)), u
    assert not doors.launch_failed()


def test_grouped_rows_pair(dev):
    qh, kvh, hd = 64, 1, 512
    lens = [2048, 1, 1500, 257]
    print("case: scores_grouped_rows / softmax_lens / mix_rows against the one-row doors", flush=True)
    most, rows = max(lens), len(lens)
    rng = np.random.default_rng(3)
    q = t(rng.standard_normal(rows * qh * hd).astype(np.float16), dev)
    k = t(rng.standard_normal(rows * most * hd).astype(np.float16), dev)
    v = t(rng.standard_normal(rows * most * hd).astype(np.float16), dev)
    lens_d = t(np.asarray(lens, np.uint32), dev)
    k_row, p_row, o_row = most * hd, qh * most, qh * hd
    p = _z(dev, rows * p_row)
    o = torch.zeros(rows * o_row, dtype=torch.float16, device=dev)
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    doors.attention_scores_grouped_rows(p, p_row, q, o_row, k, k_row, lens_d, qh, kvh, hd, most, rows)
    doors.attention_softmax_lens(p, p_row, lens_d, qh, rows)
    doors.attention_mix_rows(o, o_row, p, p_row, v, k_row, lens_d, qh, kvh, hd, rows, over)
    for u, n in enumerate(lens):
        p1 = _z(dev, qh * n)
        o1 = torch.zeros(o_row, dtype=torch.float16, device=dev)
        ku, vu = k[u * k_row:u * k_row + n * hd], v[u * k_row:u * k_row + n * hd]
        doors.attention_scores_grouped(p1, q[u * o_row:(u + 1) * o_row], ku, qh, kvh, hd, n)
        doors.attention_softmax_rows(p1, qh, n)
        assert torch.equal(p[u * p_row:u * p_row + qh * n].view(torch.int32), p1.view(torch.int32)), u
        doors.attention_mix(o1, p1, vu, qh, kvh, hd, n, over)
        assert torch.equal(o[u * o_row:(u + 1) * o_row].view(torch.int16), o1.view(torch.int16)), u
    assert not doors.launch_failed()
