"""The page-aware cache writer (silvann_gfx950_attention_cache_write_paged, row 141) on gfx950, through the C ABI.

Bit for bit against the oracle (which is bit for bit the reference family's rope_rows, tests/test_cache.py): the
caches after the write, every slot, and the fault word. Then the writer feeding the causal row: a chunk written
into a paged cache and attended there answers what the oracle gives over the cache it wrote.
"""
import numpy as np
import pytest
import torch

from silvann_amd import doors, verbs
from tests.conftest import parity
from tests.gpu_util import t
from tests.test_cache import _write_case

pytestmark = pytest.mark.gpu


def _dev(c, dev):
    return dict(k_cache=t(c["kc"], dev), v_cache=t(c["vc"], dev), pages=None if c["pages"] is None else t(c["pages"], dev),
                positions=t(c["positions"], dev), k=t(c["k"], dev), v=t(c["v"], dev),
                cs=None if c["cs"] is None else t(c["cs"], dev))


@pytest.mark.parametrize("kvh,hd,rot,lens,rps,ps,cap,paged", [
    (2, 128, 128, [5, 700], 33, 64, 1024, True),
    (8, 64, 0, [0, 1, 2, 3, 900, 31], 1, 16, 1000, True),
    (2, 256, 64, [100], 50, 0, 200, False),
    (3, 72, 18, [4, 40], 9, 32, 64, True),
    (2, 64, 64, [90, 10], 20, 32, 100, True),
    (4, 128, 128, list(range(0, 4000, 125)), 1, 256, 4096, True),   # a decode batch of 32 sequences
])
def test_writer_against_oracle(dev, oracle, kvh, hd, rot, lens, rps, ps, cap, paged):
    print(f"case: cache_write kvh{kvh} hd{hd} rot{rot} seqs{len(lens)} rps{rps} ps{ps} cap{cap}", flush=True)
    rng = np.random.default_rng(kvh + hd + rot + rps)
    c = _write_case(rng, kvh, hd, rot, lens, rps, ps, cap, paged)
    c["k"][7] = np.float16(65000).view(np.uint16)
    wk, wv, wo = oracle.cache_write_paged(**c)
    d = _dev(c, dev)
    over = verbs.cache_write_paged(d["k_cache"], d["v_cache"], d["pages"], d["positions"], d["k"], d["v"], d["cs"], kvh,
                                   hd, c["rows"], rps, cap, page_size=c["page_size"], pages_row=c["pages_row"],
                                   rot=rot or None)
    assert np.array_equal(d["k_cache"].cpu().numpy(), wk)
    assert np.array_equal(d["v_cache"].cpu().numpy(), wv)
    assert (int(over.item()) & 0xFFFFFFFF) == wo
    assert not doors.launch_failed()


def test_writer_feeds_the_causal_row(dev, oracle):
    """A 200-row chunk after a 300-position prefix: its keys turned and written into a permuted paged cache, then
    attended causally there (row 138) — the oracle's causal rows over the oracle-written cache."""
    qh, kvh, hd, first, T, ps = 16, 2, 256, 300, 200, 64
    print("case: cache_write then causal_paged", flush=True)
    rng = np.random.default_rng(21)
    c = _write_case(rng, kvh, hd, hd, [first], T, ps, 1024, True)
    c["kc"] = rng.standard_normal(c["kc"].size).astype(np.float16).view(np.uint16)   # the prefix's rows
    c["vc"] = rng.standard_normal(c["vc"].size).astype(np.float16).view(np.uint16)
    wk, wv, _ = oracle.cache_write_paged(**c)
    d = _dev(c, dev)
    verbs.cache_write_paged(d["k_cache"], d["v_cache"], d["pages"], d["positions"], d["k"], d["v"], d["cs"], kvh, hd,
                            T, T, 1024, page_size=ps, pages_row=c["pages_row"])
    q = rng.standard_normal(T * qh * hd).astype(np.float16)
    out = torch.zeros(T * qh * hd, dtype=torch.float16, device=dev)
    verbs.causal_paged(t(q, dev), d["k_cache"], d["v_cache"], d["pages"], out, qh, kvh, hd, first, T, page_size=ps)
    which = [0, 1, 63, 64, 150, T - 1]
    want, _ = oracle.causal_rows(q, wk.view(np.float16), wv.view(np.float16), c["pages"], ps, qh, kvh, hd, first,
                                 which)
    got = out.cpu().numpy().reshape(T, qh * hd)[which].ravel()
    parity(got, want)
    assert not doors.launch_failed()


def test_writer_refuses_an_odd_turn(dev):
    k = torch.zeros(4 * 64, dtype=torch.float16, device=dev)
    cache = torch.zeros(64 * 64, dtype=torch.float16, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    cs = torch.zeros(64, dtype=torch.float32, device=dev)
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    doors.attention_cache_write_paged(cache, cache, None, 0, 0, 64, pos, 4, k, k, cs, 7, 4, 1, 64, over)
    torch.cuda.synchronize()
    assert doors.launch_failed()
    assert int(over.item()) == 0


def test_rope_rows_against_oracle(dev, oracle):
    """rope_rows (nn row 46) on the GPU, bit for bit the oracle's (which is the reference family's door)."""
    from tests.test_cache import angles
    rows, heads, hd, rot, row_stride = 300, 16, 128, 64, 16 * 128 + 8
    print("case: rope_rows", flush=True)
    rng = np.random.default_rng(4)
    x = rng.standard_normal(rows * row_stride).astype(np.float16).view(np.uint16)
    x[11] = np.float16(65000).view(np.uint16)
    cs = angles(rng.integers(0, 300000, rows), rot)
    want, wo = oracle.rope_rows(x, cs, rows, heads, hd, row_stride, rot)
    xd = t(x, dev)
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    doors.rope_rows(xd, xd, t(cs, dev), rows, heads, hd, row_stride, rot, over)
    assert np.array_equal(xd.cpu().numpy(), want)
    assert (int(over.item()) & 0xFFFFFFFF) == wo
    assert not doors.launch_failed()
