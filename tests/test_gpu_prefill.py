"""Fused causal prefill (silvann_gfx950_attention_causal_paged) against the oracle and a torch fp32 reference.

Tolerance: max-abs <= 2e-3 and cosine >= 0.9999 on the fp16 outputs. The C oracle checks chosen rows (a
causal row r is the reference's decode at position first + r over positions 0..first+r,
attention__abi.cuh:336-342); torch fp32 checks every row at full size.
"""
import numpy as np
import pytest
import torch

from silvann_amd import workloads as W
from tests.conftest import parity
from tests.gpu_util import CausalOnDevice, t, torch_causal

pytestmark = pytest.mark.gpu


def _rows_check(oracle, w, got, which):
    want, _ = oracle.causal_rows(w.q, w.k, w.v, w.pages, w.page_size, w.q_heads, w.kv_heads, w.head_dim, w.first,
                                 which)
    g = got.reshape(w.rows, -1)[np.asarray(which)]
    parity(g, want.reshape(len(which), -1))


@pytest.mark.parametrize("hd,qh,kvh,first,rows,ps", [
    (64, 8, 8, 0, 100, 0),
    (128, 32, 4, 0, 257, 0),
    (256, 16, 2, 0, 130, 0),
    (128, 16, 2, 300, 64, 32),
    (256, 16, 2, 77, 95, 64),
    (128, 6, 2, 10, 70, 0),      # group 3: one head a wave, 128 rows a workgroup
    (64, 4, 2, 5, 200, 0),       # group 2
])
def test_small_shapes_against_oracle(dev, oracle, hd, qh, kvh, first, rows, ps):
    w = W.causal("small", qh, kvh, hd, first, rows, page_size=ps, seed=hd + rows)
    print(f"case: causal hd{hd} qh{qh} kvh{kvh} first{first} rows{rows} ps{ps}", flush=True)
    got = CausalOnDevice(w, dev).run().cpu().numpy()
    _rows_check(oracle, w, got, list(range(rows)))


def test_config3_full(dev, oracle):
    w = W.config3()
    print("case: C3 causal 4096", flush=True)
    d = CausalOnDevice(w, dev)
    got = d.run()
    want = torch_causal(d.q, d.k, d.v, w.q_heads, w.kv_heads, w.head_dim, w.first, w.rows)
    parity(got.cpu().float().numpy(), want.cpu().numpy())
    _rows_check(oracle, w, got.cpu().numpy(), [0, 1, 31, 32, 63, 64, 255, 2047, 4095])


def test_config4_full(dev, oracle):
    w = W.config4()
    print("case: C4 causal 2048 over 100000 paged", flush=True)
    d = CausalOnDevice(w, dev)
    got = d.run()
    k, v = w.gathered()
    want = torch_causal(d.q, t(k, dev), t(v, dev), w.q_heads, w.kv_heads, w.head_dim, w.first, w.rows)
    parity(got.cpu().float().numpy(), want.cpu().numpy())
    _rows_check(oracle, w, got.cpu().numpy(), [0, 2047])


def test_page_permutation_bit_exact(dev):
    a = W.causal("perm", 16, 2, 128, 1000, 300, page_size=64, seed=41, permute=True)
    b = W.causal("ident", 16, 2, 128, 1000, 300, page_size=64, seed=41, permute=False)
    row = a.kv_heads * a.head_dim
    for j in range(len(a.pages)):
        pa, pb = int(a.pages[j]), int(b.pages[j])
        b.k[pb * 64 * row:(pb + 1) * 64 * row] = a.k[pa * 64 * row:(pa + 1) * 64 * row]
        b.v[pb * 64 * row:(pb + 1) * 64 * row] = a.v[pa * 64 * row:(pa + 1) * 64 * row]
    b.q[:] = a.q
    ga = CausalOnDevice(a, dev).run().cpu().numpy().view(np.uint16)
    gb = CausalOnDevice(b, dev).run().cpu().numpy().view(np.uint16)
    assert np.array_equal(ga, gb)


def test_row_equals_decode_at_its_position(dev):
    """Causal row r is decode at position first + r (attention__abi.cuh:341-342), through the two doors."""
    from tests.gpu_util import DecodeOnDevice
    w = W.causal("rowdec", 16, 2, 256, 500, 64, page_size=0, seed=43)
    got = CausalOnDevice(w, dev).run().cpu().numpy().reshape(w.rows, -1)
    row = w.kv_heads * w.head_dim
    for r in (0, 37, 63):
        n = w.first + r + 1
        dw = W.Decode("d", 16, 2, 256, np.array([n], np.uint32), 0, None, 0, n * row,
                      w.q.reshape(w.rows, -1)[r].copy(), w.k[: n * row].copy(), w.v[: n * row].copy())
        dg = DecodeOnDevice(dw, dev).run().cpu().numpy()
        parity(got[r], dg, atol=2e-3)
