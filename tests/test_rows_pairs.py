"""One-row and many-row door pairs agree bit for bit — the reference's own requirement of a family
(engine/src/silicon_families/add_a_family.md:51-55, the pairs its on-device verb test names), checked on this
library's kernels in the CPU emulation (tests/emu):

- attention_weights_rows + attention_residual_mix_rows (gpu.cuh:195-196) against attention_weights +
  attention_residual_mix (122-123) a row at a time: row u over first + u + 1 keys;
- attention_weights_tq_rows + attention_residual_mix_tq_rows (197-198) against attention_weights_tq +
  attention_residual_mix_tq (163-164);
- attention_scores_grouped_rows + attention_softmax_lens + attention_mix_rows (222-224) against
  attention_scores_grouped + attention_softmax_rows + attention_mix (189-190, 120), row u over its own lens[u].

The weights, the residuals after each door and the fp16 answers are compared as bits.
"""
import numpy as np
import pytest

from tests.emu import emu
from tests.test_tq import make

pytestmark = pytest.mark.skipif(emu.compiler() is None, reason="no clang++ for the CPU emulation")


def _f16(rng, n):
    return rng.standard_normal(n).astype(np.float16)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_weights_rows_pair():
    qh, kvh, hd, first, rows = 8, 2, 64, 40, 5
    rng = np.random.default_rng(1)
    q = _f16(rng, rows * qh * hd)
    k = _f16(rng, (first + rows) * kvh * hd)
    v = _f16(rng, (first + rows) * kvh * hd)
    p, res_w, res, _, _ = emu.run_fp16(q, k, v, qh, kvh, hd, first=first, rows=rows)
    span, rf = first + rows, hd + 2
    for u in range(rows):
        n = first + u + 1
        ps, rws, rs, _, _ = emu.run_fp16(q[u * qh * hd:(u + 1) * qh * hd], k, v, qh, kvh, hd, length=n)
        assert np.array_equal(_bits(p[u * qh * span:u * qh * span + qh * n]), _bits(ps)), u
        assert np.array_equal(_bits(res_w[u * qh * rf:(u + 1) * qh * rf].reshape(qh, rf)[:, :2]),
                              _bits(rws.reshape(qh, rf)[:, :2])), u
        assert np.array_equal(_bits(res[u * qh * rf:(u + 1) * qh * rf]), _bits(rs)), u


@pytest.mark.parametrize("d,hd,length", [(4, 128, 300), (8, 64, 2200)])   # one split; several splits
def test_tq_rows_pair(d, hd, length):
    qh, kvh, rows = 4, 2, 3
    rng = np.random.default_rng(d + hd)
    q, codes, scales = make(rng, qh, kvh, hd, length, d, rows=rows)
    p, res_w, res, _, _ = emu.run_tq(q, codes, scales, qh, kvh, hd, length, d, rows=rows)
    rf = hd + 2
    for u in range(rows):
        ps, rws, rs, _, _ = emu.run_tq(q[u * qh * hd:(u + 1) * qh * hd], codes, scales, qh, kvh, hd, length, d)
        assert np.array_equal(_bits(p[u * qh * length:(u + 1) * qh * length]), _bits(ps)), u
        assert np.array_equal(_bits(res_w[u * qh * rf:(u + 1) * qh * rf].reshape(qh, rf)[:, :2]),
                              _bits(rws.reshape(qh, rf)[:, :2])), u
        assert np.array_equal(_bits(res[u * qh * rf:(u + 1) * qh * rf]), _bits(rs)), u


def test_grouped_rows_pair():
    qh, kvh, hd = 16, 1, 128
    lens = [300, 1, 257, 64]
    most = max(lens)
    rng = np.random.default_rng(3)
    rows = len(lens)
    q = _f16(rng, rows * qh * hd)
    k = _f16(rng, rows * most * kvh * hd)
    v = _f16(rng, rows * most * kvh * hd)
    k_row = most * kvh * hd
    p, ps_, o, _, _ = emu.run_grouped(q, k, v, qh, kvh, hd, most, lens=lens, k_row=k_row)
    for u, n in enumerate(lens):
        kk, vv = k[u * k_row:u * k_row + n * kvh * hd], v[u * k_row:u * k_row + n * kvh * hd]
        p1, s1, o1, _, _ = emu.run_grouped(q[u * qh * hd:(u + 1) * qh * hd], kk, vv, qh, kvh, hd, n)
        # a row's heads are lens[u] apart in its stretch of p (kernels.cuh:953-972)
        row_p = p[u * qh * most:u * qh * most + qh * n].reshape(qh, n)
        row_s = ps_[u * qh * most:u * qh * most + qh * n].reshape(qh, n)
        assert np.array_equal(_bits(row_p), _bits(p1.reshape(qh, n))), u
        assert np.array_equal(_bits(row_s), _bits(s1.reshape(qh, n))), u
        assert np.array_equal(o[u * qh * hd:(u + 1) * qh * hd], o1), u
