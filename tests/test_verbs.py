"""The verbs' operand checks on the host (no GPU): each refusal raises the reference's fault word before
any door is called (the operands here are CPU tensors, so a door call would fail loudly instead).

Words: OPCT for a non-dimension (attention__abi.cuh:30-34), NPBN for operands out of bounds
(attention__abi.cuh:140-150, 190-199), NARM for a scores buffer too small for one row (attention.cuh:46),
NATB for the rows verb's own argument checks.
"""
import pytest
import torch

from silvann_amd import verbs
from silvann_amd.verbs import FAULT_BOUNDS, FAULT_ROOM, FAULT_TYPE, Fault


def h(n):
    return torch.zeros(n, dtype=torch.float16)


def f(n):
    return torch.zeros(n, dtype=torch.float32)


def refuses(word, fn, *args, **kw):
    with pytest.raises(Fault) as e:
        fn(*args, **kw)
    assert e.value.word == word, hex(e.value.word)


def test_decode_checks():
    qh, kvh, hd, to = 8, 2, 64, 10
    q, k, v, s, o = h(qh * hd), h(to * kvh * hd), h(to * kvh * hd), f(qh * to), h(qh * hd)
    refuses(FAULT_TYPE, verbs.decode, q, k, v, s, o, 0, kvh, hd, 0, to, None)            # zero heads
    refuses(FAULT_TYPE, verbs.decode, q, k, v, s, o, qh, kvh, hd, 0, (1 << 20) + 1, None)  # past DIM_MAX
    refuses(FAULT_TYPE, verbs.decode, q, k, v, s, o, qh, kvh, hd, -1, to, None)           # negative from
    refuses(FAULT_BOUNDS, verbs.decode, q, k, v, s, o, qh, kvh, hd, to, to, None)         # empty range
    refuses(FAULT_BOUNDS, verbs.decode, q, k, v, s, o, 6, 4, hd, 0, to, None)             # 6 % 4
    refuses(FAULT_BOUNDS, verbs.decode, q, h(to * kvh * hd - 1), v, s, o, qh, kvh, hd, 0, to, None)
    refuses(FAULT_BOUNDS, verbs.decode, q, k, v, f(qh * to - 1), o, qh, kvh, hd, 0, to, None)   # 2·qh·len halves
    refuses(FAULT_BOUNDS, verbs.decode, h(qh * hd - 1), k, v, s, o, qh, kvh, hd, 0, to, None)


def test_residual_merge_finish_checks():
    qh, kvh, hd, to = 4, 2, 32, 5
    q, k, v, s = h(qh * hd), h(to * kvh * hd), h(to * kvh * hd), f(qh * to)
    small = f(qh * (hd + 2) - 1)   # the residual needs 2·q_heads·(hd + 2) halves of room
    refuses(FAULT_BOUNDS, verbs.residual, q, k, v, s, small, qh, kvh, hd, 0, to)
    refuses(FAULT_BOUNDS, verbs.merge, small, small, small, qh, hd)
    refuses(FAULT_BOUNDS, verbs.finish, f(qh * (hd + 2)), h(qh * hd - 1), qh, hd, None)


def test_rows_attention_checks():
    qh, kvh, hd, first, rows = 4, 2, 32, 3, 5
    n = first + rows
    q, kv, att = h(rows * qh * hd), h(n * kvh * hd), h(rows * qh * hd)
    natb = verbs.word("NATB")
    refuses(natb, verbs.rows_attention, q, kv, kv, f(qh * n), att, qh, kvh, hd, -1, rows, None)
    refuses(natb, verbs.rows_attention, q, kv, kv, f(qh * n), att, qh, kvh, 9, first, rows, None)   # odd hd
    refuses(FAULT_ROOM, verbs.rows_attention, q, kv, kv, f(qh * n - 1), att, qh, kvh, hd, first, rows, None)
    refuses(FAULT_ROOM, verbs.rows_attention, q, h(n * kvh * hd - 1), kv, f(qh * n), att, qh, kvh, hd, first,
            rows, None)


def test_paged_checks():
    qh, kvh, hd = 8, 2, 128
    q, o = h(2 * qh * hd), h(2 * qh * hd)
    lens = torch.tensor([40, 70], dtype=torch.int32)
    pages = torch.zeros(10, dtype=torch.int32)
    kv = h(1)
    refuses(FAULT_BOUNDS, verbs.decode_paged, q, kv, kv, pages, lens, o, qh, kvh, 96, 70, page_size=16,
            pages_row=5)                                                                       # head_dim 96
    refuses(FAULT_BOUNDS, verbs.decode_paged, q, kv, kv, pages, lens, o, qh, kvh, hd, 70, page_size=24,
            pages_row=5)                                                                       # page 24
    refuses(FAULT_BOUNDS, verbs.decode_paged, q, kv, kv, pages, lens, o, qh, kvh, hd, 70, page_size=16,
            pages_row=6)                                                                       # table short
    refuses(FAULT_BOUNDS, verbs.causal_paged, q, kv, kv, pages, o, qh, kvh, hd, 0, 2, page_size=48)
    refuses(FAULT_BOUNDS, verbs.causal_paged, q, kv, kv, pages, o, qh, kvh, hd, (1 << 31) - 1, 2, page_size=32)
    refuses(FAULT_BOUNDS, verbs.causal_paged, q, kv, kv, None, o, qh, kvh, hd, 0, 2)          # cache too small
    refuses(FAULT_BOUNDS, verbs.causal_paged, q, kv, kv, None, o, 6, 4, hd, 0, 2)             # 6 % 4


def test_residual_tq_checks():
    """attention__abi.cuh:245-266: width 4 or 8 and whole groups (OPCT), then every operand's room (NPBN)."""
    qh, kvh, hd, d, n = 8, 2, 64, 4, 10
    rb = verbs.tq_row_bytes(d, hd)
    codes = lambda b: torch.zeros(b, dtype=torch.uint8)  # noqa: E731
    q, kc, ks, vc, vs = h(qh * hd), codes(n * kvh * rb), h(n * kvh), codes(n * kvh * rb), h(n * kvh)
    s, r = f(qh * n), f(qh * (hd + 2))
    args = (q, kc, ks, vc, vs, s, r)
    refuses(FAULT_TYPE, verbs.residual_tq, *args, qh, kvh, hd, 3, n)          # a width the tiers do not use
    refuses(FAULT_TYPE, verbs.residual_tq, *args, 6, 4, hd, d, n)             # 6 % 4
    refuses(FAULT_TYPE, verbs.residual_tq, *args, qh, kvh, hd, d, 0)          # no rows
    refuses(FAULT_BOUNDS, verbs.residual_tq, h(qh * hd - 1), kc, ks, vc, vs, s, r, qh, kvh, hd, d, n)
    refuses(FAULT_BOUNDS, verbs.residual_tq, q, kc, h(n * kvh - 1), vc, vs, s, r, qh, kvh, hd, d, n)
    refuses(FAULT_BOUNDS, verbs.residual_tq, q, kc, ks, vc, vs, f(qh * n - 1), r, qh, kvh, hd, d, n)
    refuses(FAULT_BOUNDS, verbs.residual_tq, q, kc, ks, vc, vs, s, f(qh * (hd + 2) - 1), qh, kvh, hd, d, n)
    # the codes' bytes against their room in halves, as the reference compares them
    refuses(FAULT_BOUNDS, verbs.residual_tq, q, codes(n * kvh * rb // 2 - 2), ks, vc, vs, s, r, qh, kvh, hd, d, n)
