"""Split-K paged decode (silvann_gfx950_attention_decode_paged) against the oracle and invariants.

Tolerance (the north star's, on fp16 outputs): max-abs <= 2e-3 and cosine >= 0.9999. Page-table
handling: bit-exact (the answer under a permuted page table equals the answer over the identity layout).
"""
import numpy as np
import pytest
import torch

from silvann_amd import workloads as W
from tests.conftest import parity
from tests.gpu_util import DecodeOnDevice, torch_decode_row

pytestmark = pytest.mark.gpu


def _oracle_decode(oracle, w):
    o, over = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, w.q_heads,
                                  w.kv_heads, w.head_dim, w.rows)
    return o, over


def test_config1_against_oracle(dev, oracle):
    w = W.config1()
    print("case: C1 decode 16q/2kv hd256 len2048", flush=True)
    got = DecodeOnDevice(w, dev).run().cpu().numpy()
    want, _ = _oracle_decode(oracle, w)
    parity(got, want)


@pytest.mark.parametrize("hd,qh,kvh", [(64, 8, 8), (128, 32, 4), (256, 16, 2), (128, 64, 1), (256, 24, 8)])
def test_small_shapes_against_oracle(dev, oracle, hd, qh, kvh):
    lens = [1, 31, 32, 33, 200, 777, 1500]
    w = W.decode("small", qh, kvh, hd, lens, page_size=32, seed=hd + qh)
    print(f"case: decode small hd{hd} qh{qh} kvh{kvh} paged32", flush=True)
    got = DecodeOnDevice(w, dev).run().cpu().numpy()
    want, _ = _oracle_decode(oracle, w)
    parity(got, want)


def test_contiguous_rows_against_oracle(dev, oracle):
    w = W.decode("contig", 16, 2, 128, [5, 64, 129, 1000], page_size=0, seed=11)
    print("case: decode contiguous rows", flush=True)
    got = DecodeOnDevice(w, dev).run().cpu().numpy()
    want, _ = _oracle_decode(oracle, w)
    parity(got, want)


def test_zero_length_row_answers_zero(dev):
    w = W.decode("zero", 16, 2, 128, [300, 0, 40], page_size=32, seed=12)
    print("case: decode zero-length row", flush=True)
    got = DecodeOnDevice(w, dev).run().view(3, -1).cpu().float().numpy()
    assert np.all(got[1] == 0)
    assert np.all(np.isfinite(got))


def test_single_position_gives_v(dev):
    """Closed form: one cached position's softmax weight is 1, so every head's answer is its kv head's v."""
    w = W.decode("one", 16, 2, 256, [1], page_size=0, seed=13)
    got = DecodeOnDevice(w, dev).run().cpu().numpy().reshape(16, 256)
    v = w.v.reshape(2, 256)
    for h in range(16):
        assert np.array_equal(got[h].view(np.uint16), v[h // 8].view(np.uint16))


def test_page_permutation_bit_exact(dev):
    """The same logical cache through a permuted page table and through the identity gives the same bits."""
    lens = [3000, 256, 1, 4097]
    a = W.decode("perm", 32, 4, 128, lens, page_size=256, seed=21, permute=True)
    b = W.decode("ident", 32, 4, 128, lens, page_size=256, seed=21, permute=False)
    # lay b's pool out so that its logical cache equals a's
    row = a.kv_heads * a.head_dim
    for u in range(a.rows):
        n = (int(lens[u]) + 255) // 256
        for j in range(n):
            pa, pb = int(a.pages[u * a.pages_row + j]), int(b.pages[u * b.pages_row + j])
            b.k[pb * 256 * row:(pb + 1) * 256 * row] = a.k[pa * 256 * row:(pa + 1) * 256 * row]
            b.v[pb * 256 * row:(pb + 1) * 256 * row] = a.v[pa * 256 * row:(pa + 1) * 256 * row]
    b.q[:] = a.q
    print("case: decode page permutation", flush=True)
    ga = DecodeOnDevice(a, dev).run().cpu().numpy().view(np.uint16)
    gb = DecodeOnDevice(b, dev).run().cpu().numpy().view(np.uint16)
    assert np.array_equal(ga, gb)


def test_config2_full_against_torch_and_oracle_rows(dev, oracle):
    w = W.config2()
    print(f"case: C2 full, sum(lens)={int(w.lens.sum())}", flush=True)
    d = DecodeOnDevice(w, dev)
    got = d.run().view(w.rows, -1)
    for u in range(w.rows):
        k, v = w.gathered(u)
        want = torch_decode_row(d.q.view(w.rows, -1)[u], torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                                w.q_heads, w.kv_heads, w.head_dim)
        parity(got[u].cpu().float().numpy(), want.cpu().numpy())
    # the C oracle on two of the rows
    for u in (0, 17):
        k, v = w.gathered(u)
        p = oracle.scores(w.q.reshape(w.rows, -1)[u], k, w.q_heads, w.kv_heads, w.head_dim, int(w.lens[u]))
        o, _ = oracle.mix(p, v, w.q_heads, w.kv_heads, w.head_dim, int(w.lens[u]))
        parity(got[u].cpu().numpy(), o)


def test_config5_full_against_oracle(dev, oracle):
    w = W.config5()
    print("case: C5 full 262144 positions", flush=True)
    got = DecodeOnDevice(w, dev).run().cpu().numpy()
    want, _ = _oracle_decode(oracle, w)
    parity(got, want)


def test_repeat_is_deterministic(dev):
    w = W.decode("det", 16, 2, 256, [20000], page_size=256, seed=31)
    d = DecodeOnDevice(w, dev)
    a = d.run().clone()
    b = d.run().clone()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
