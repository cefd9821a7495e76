"""The page-aware cache writer (silvann_gfx950_attention_cache_write_paged, appended row 141) on the CPU.

- The oracle's `rope_rows` against the reference family's own door (oracle/_ref, nn row 46, gpu.cuh:140), bit for
  bit, full and partial turns, with overflow; and against what the mathematics fixes: the angle 0 is the identity,
  a quarter turn is (a, b) -> (-b, a) exactly, and the turn agrees with a float64 rotation to fp16 rounding.
- The oracle's writer: a paged write, gathered through the page table, is bit for bit the contiguous write; each
  row's key is rope_rows of it and its value a copy; slots no row maps to are untouched; a position past the
  capacity writes nothing and leaves NPBN.
- The library's kernel in the CPU emulation (tests/emu) against the oracle, bit for bit (integer placement and
  the same fp32 arithmetic), on both the 16-byte and the element-wise forms.
"""
import numpy as np
import pytest

FAULT_BOUNDS = 0x4E50424E


def angles(positions, rot, theta=1e6):
    """cos then sin of each position's rot/2 angles, fp32 (HF's rotary frequencies theta^(-2i/rot))."""
    i = np.arange(rot // 2, dtype=np.float64)
    ang = np.asarray(positions, np.float64)[:, None] * theta ** (-2.0 * i / rot)[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32).ravel()


@pytest.mark.parametrize("rows,heads,hd,rot", [(13, 2, 128, 128), (7, 4, 256, 64), (5, 3, 72, 18)])
def test_oracle_rope_rows_is_the_reference(ref, oracle, rows, heads, hd, rot):
    rng = np.random.default_rng(rows + hd + rot)
    x = rng.standard_normal(rows * heads * hd).astype(np.float16).view(np.uint16)
    x[3] = np.float16(60000).view(np.uint16)   # a turn that may overflow
    cs = angles(rng.integers(0, 200000, rows), rot)
    want, wo = ref.rope_rows(x, cs, rows, heads, hd, heads * hd, rot)
    got, go = oracle.rope_rows(x, cs, rows, heads, hd, heads * hd, rot)
    assert np.array_equal(got, want)
    assert go == wo


def test_oracle_rope_rows_closed_forms(oracle):
    rows, heads, hd = 3, 2, 64
    rng = np.random.default_rng(5)
    x = rng.standard_normal(rows * heads * hd).astype(np.float16).view(np.uint16)
    half = hd // 2
    ident = np.concatenate([np.ones(half), np.zeros(half)]).astype(np.float32)
    got, _ = oracle.rope_rows(x, np.tile(ident, rows), rows, heads, hd, heads * hd, hd)
    assert np.array_equal(got, x)
    quarter = np.concatenate([np.zeros(half), np.ones(half)]).astype(np.float32)
    got, _ = oracle.rope_rows(x, np.tile(quarter, rows), rows, heads, hd, heads * hd, hd)
    xs = x.view(np.float16).reshape(rows, heads, 2, half)
    gs = got.view(np.float16).reshape(rows, heads, 2, half)
    assert np.array_equal(gs[:, :, 0], -xs[:, :, 1]) and np.array_equal(gs[:, :, 1], xs[:, :, 0])
    cs = angles([1, 1000, 77777], hd)
    got, _ = oracle.rope_rows(x, cs, rows, heads, hd, heads * hd, hd)
    c = cs.reshape(rows, 1, 2, half).astype(np.float64)
    xd = xs.astype(np.float64)
    want = np.stack([xd[:, :, 0] * c[:, :, 0] - xd[:, :, 1] * c[:, :, 1],
                     xd[:, :, 1] * c[:, :, 0] + xd[:, :, 0] * c[:, :, 1]], axis=2)
    err = np.abs(got.view(np.float16).reshape(want.shape).astype(np.float64) - want)
    assert np.all(err <= np.abs(want) * 2.0 ** -10 + 2.0 ** -24)   # within half an fp16 ulp, plus fp32 rounding


def _write_case(rng, kvh, hd, rot, lens_before, rows_per_seq, page_size, capacity, paged=True):
    """Sequences with `lens_before[u]` positions each, rows_per_seq new rows each; a pool of permuted pages."""
    nseq = len(lens_before)
    rows = nseq * rows_per_seq
    row = kvh * hd
    if paged:
        per = (capacity + page_size - 1) // page_size
        pool = nseq * per + 3
        pages = rng.permutation(pool)[: nseq * per].astype(np.uint32)
        slots = pool * page_size
    else:
        per, pages, slots = 0, None, nseq * capacity
    kc = rng.integers(0, 65536, slots * row, dtype=np.uint16)   # whatever the caches held
    vc = rng.integers(0, 65536, slots * row, dtype=np.uint16)
    k = rng.standard_normal(rows * row).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(rows * row).astype(np.float16).view(np.uint16)
    positions = np.asarray(lens_before, np.uint32)
    pos_rows = np.repeat(positions, rows_per_seq) + np.tile(np.arange(rows_per_seq), nseq)
    cs = angles(pos_rows, rot) if rot else None
    return dict(kc=kc, vc=vc, pages=pages, pages_row=per, page_size=page_size if paged else 0, capacity=capacity,
                positions=positions, rows_per_seq=rows_per_seq, k=k, v=v, cs=cs, rot=rot, rows=rows, kvh=kvh, hd=hd)


def _slots(c):
    """Each row's slot (None past capacity)."""
    out = []
    for r in range(c["rows"]):
        u, p = r // c["rows_per_seq"], int(c["positions"][r // c["rows_per_seq"]]) + r % c["rows_per_seq"]
        if p >= c["capacity"]:
            out.append(None)
        elif c["pages"] is None:
            out.append(u * c["capacity"] + p)
        else:
            out.append(int(c["pages"][u * c["pages_row"] + p // c["page_size"]]) * c["page_size"] + p % c["page_size"])
    return out


def test_oracle_writer(oracle):
    rng = np.random.default_rng(9)
    c = _write_case(rng, 2, 128, 64, [0, 300, 17], 40, 32, 512)
    kc, vc, over = oracle.cache_write_paged(**c)
    assert over == 0
    row = c["kvh"] * c["hd"]
    want_k, _ = oracle.rope_rows(c["k"], c["cs"], c["rows"], c["kvh"], c["hd"], row, c["rot"])
    written = np.zeros(len(kc) // row, bool)
    for r, s in enumerate(_slots(c)):
        assert np.array_equal(kc[s * row:(s + 1) * row], want_k[r * row:(r + 1) * row])
        assert np.array_equal(vc[s * row:(s + 1) * row], c["v"][r * row:(r + 1) * row])
        written[s] = True
    keep = np.repeat(~written, row)
    assert np.array_equal(kc[keep], c["kc"][keep]) and np.array_equal(vc[keep], c["vc"][keep])
    # the same rows into contiguous caches, gathered back from the pages: the same bits
    cc = dict(c, pages=None, pages_row=0, page_size=0)
    cc["kc"] = np.zeros(3 * c["capacity"] * row, np.uint16)
    cc["vc"] = np.zeros_like(cc["kc"])
    kc2, vc2, _ = oracle.cache_write_paged(**cc)
    for u in range(3):
        for p in range(int(c["positions"][u]), int(c["positions"][u]) + c["rows_per_seq"]):
            s = int(c["pages"][u * c["pages_row"] + p // 32]) * 32 + p % 32
            t = u * c["capacity"] + p
            assert np.array_equal(kc[s * row:(s + 1) * row], kc2[t * row:(t + 1) * row])
            assert np.array_equal(vc[s * row:(s + 1) * row], vc2[t * row:(t + 1) * row])


def test_oracle_writer_past_capacity(oracle):
    rng = np.random.default_rng(10)
    c = _write_case(rng, 2, 64, 64, [90, 10], 20, 32, 100)   # sequence 0's rows 10..19 are past 100 positions
    kc, vc, over = oracle.cache_write_paged(**c)
    assert over == FAULT_BOUNDS
    row = c["kvh"] * c["hd"]
    touched = {s for s in _slots(c) if s is not None}
    assert len(touched) == 30
    for s in range(len(kc) // row):
        if s not in touched:
            assert np.array_equal(kc[s * row:(s + 1) * row], c["kc"][s * row:(s + 1) * row])


# ── the library's kernel in the CPU emulation ────────────────────────────────────────────────────────────

@pytest.mark.parametrize("kvh,hd,rot,lens,rps,ps,cap,paged", [
    (2, 128, 128, [5, 700], 33, 64, 1024, True),     # a chunk a sequence, 16-byte units, full turn
    (8, 64, 0, [0, 1, 2, 3, 900, 31], 1, 16, 1000, True),   # a decode batch, no angles
    (2, 256, 64, [100], 50, 0, 200, False),          # contiguous, partial turn
    (3, 72, 18, [4, 40], 9, 32, 64, True),           # head_dim 72, turn 18: the element-wise form
    (2, 64, 64, [90, 10], 20, 32, 100, True),        # rows past the capacity
])
def test_emulated_writer(oracle, kvh, hd, rot, lens, rps, ps, cap, paged):
    from tests.emu import emu
    if emu.compiler() is None:
        pytest.skip("no clang++ for the CPU emulation")
    rng = np.random.default_rng(kvh + hd + rot + rps)
    c = _write_case(rng, kvh, hd, rot, lens, rps, ps, cap, paged)
    c["k"][7] = np.float16(65000).view(np.uint16)
    wk, wv, wo = oracle.cache_write_paged(**c)
    gk, gv, go, _ = emu.run_cache_write(**c)
    assert np.array_equal(gk, wk)
    assert np.array_equal(gv, wv)
    assert go == wo
    if rot == 0:
        assert go == 0


@pytest.mark.parametrize("rows,heads,hd,rot,row_stride", [(13, 2, 128, 128, 256), (5, 3, 72, 18, 3 * 72 + 8)])
def test_emulated_rope_rows(oracle, rows, heads, hd, rot, row_stride):
    """rope_rows (nn row 46) in the emulation against the oracle — itself the reference family's door to the bit."""
    from tests.emu import emu
    if emu.compiler() is None:
        pytest.skip("no clang++ for the CPU emulation")
    rng = np.random.default_rng(rows + hd)
    x = rng.standard_normal(rows * row_stride).astype(np.float16).view(np.uint16)
    x[5] = np.float16(65000).view(np.uint16)
    cs = angles(rng.integers(0, 300000, rows), rot)
    want, wo = oracle.rope_rows(x, cs, rows, heads, hd, row_stride, rot)
    got, go, _ = emu.run_rope_rows(x, cs, rows, heads, hd, row_stride, rot)
    assert np.array_equal(got, want)
    assert go == wo
