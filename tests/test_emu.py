"""The library's kernel sources run in the CPU emulation (tests/emu) against the oracle — no GPU needed.

The emulation (tests/emu/emu_rt.hpp) runs every lane of a workgroup as a host thread with the gfx950
operand layouts of the MFMA and the transposing LDS read; direct-to-LDS loads land only when the issuing
lane's s_waitcnt lets them (their destination reads NaN before that), and every buffer sits against a guard
page. So these tests check the kernels' arithmetic, their waits and barriers, and that every access stays
inside its buffer, through the same C entry points the GPU tests call. The bar is the GPU tests' bar:
max-abs <= 2e-3 and cosine >= 0.9999 on the fp16 outputs (tests/conftest.py::parity). They do not measure
anything a GPU would: timing, and hardware behaviour the emulation does not model.

Shapes are small (the emulation runs a few workgroups a second).
"""
import numpy as np
import pytest

from silvann_amd import workloads as W
from tests.conftest import parity, residual_parity
from tests.emu import emu

pytestmark = pytest.mark.skipif(emu.compiler() is None, reason="no clang++ for the CPU emulation")

PIPE = {"SILVANN_GFX950_PREFILL": "pipe"}
DUO = {"SILVANN_GFX950_PREFILL": "duo"}


def _causal(oracle, hd, qh, kvh, first, rows, ps, env=None):
    w = W.causal("emu", qh, kvh, hd, first, rows, page_size=ps, seed=hd + rows)
    got, over, _ = emu.run_causal(w, env)
    want, _ = oracle.causal_rows(w.q, w.k, w.v, w.pages, w.page_size, qh, kvh, hd, first, list(range(rows)))
    parity(got, want)
    assert over == 0


@pytest.mark.parametrize("hd,qh,kvh,first,rows,ps", [
    (128, 6, 2, 10, 70, 0),      # group 3: one head a wave, waves on different rows
    (256, 16, 2, 77, 95, 64),    # paged, page table in LDS, the steady loop at head_dim 256
    (64, 8, 1, 300, 256, 32),    # 8 workgroups of 8 row tiles: the XCD-aware order permutes them
])
def test_causal_default_kernel(oracle, hd, qh, kvh, first, rows, ps):
    _causal(oracle, hd, qh, kvh, first, rows, ps)


@pytest.mark.parametrize("hd,qh,kvh,first,rows,ps", [
    (256, 16, 2, 0, 130, 0),     # paired row tiles; the first tile load of K 4 must wait for S(0)
    (256, 6, 2, 37, 90, 0),      # one head a wave: waves with different steady lengths
    (256, 4, 2, 50, 100, 32),    # two heads a wave, 32-position pages
])
def test_causal_pipe_kernel(oracle, hd, qh, kvh, first, rows, ps):
    _causal(oracle, hd, qh, kvh, first, rows, ps, env=PIPE)


@pytest.mark.parametrize("hd,qh,kvh,first,rows,ps", [
    (256, 16, 2, 0, 130, 0),     # paired row tiles; an odd tile count leaves the odd waves a lone last tile
    (256, 8, 2, 37, 90, 64),     # paged, page table in LDS; a prefix longer than a tile
    (128, 4, 1, 300, 40, 32),    # unpaired (prefix past the chunk); 32-position pages
    (128, 8, 1, 5, 1, 0),        # one row: one tile, the odd waves idle; the merge over an empty partner
    (256, 8, 2, 1, 33, 96),      # the odd waves' first tile past most rows' positions: rows with no key seen yet
])
def test_causal_duo_kernel(oracle, hd, qh, kvh, first, rows, ps):
    """causal_duo (two waves a SIMD over alternate key tiles, merged through LDS) against the oracle."""
    _causal(oracle, hd, qh, kvh, first, rows, ps, env=DUO)


@pytest.mark.parametrize("hd,qh,kvh,first,rows,ps", [
    (256, 16, 2, 77, 95, 64),    # paged, page table in LDS
    (128, 4, 1, 1, 33, 0),       # the odd waves' first tile past most rows' positions
    (256, 8, 2, 300, 40, 32),    # unpaired: a prefix longer than the chunk
])
def test_causal_duo_residual_kernel(oracle, hd, qh, kvh, first, rows, ps):
    """Row 140 through causal_duo (SILVANN_GFX950_PREFILL=duo): the two waves' residuals merged against the true
    max of both, against the oracle's attention_weights_rows + attention_residual_mix_rows."""
    w = W.causal("emu", qh, kvh, hd, first, rows, page_size=ps, seed=hd + rows + 5)
    got, over, _ = emu.run_causal_res(w, DUO)
    k, v = w.gathered()
    p, res = oracle.weights_rows(w.q, k, qh, kvh, hd, first, rows)
    residual_parity(got, oracle.residual_mix_rows(res, p, v, qh, kvh, hd, first, rows), hd)
    assert over == 0


@pytest.mark.parametrize("qh,kvh,hd,lens,ps", [
    (16, 2, 256, [700, 2048], 256),        # paged rows of different lengths
    (8, 2, 128, [1, 17, 300], 0),          # contiguous, a one-position row
    (4, 4, 64, [33, 250], 16),             # pages shorter than a tile: one lookup a 16-key group
    # the plan's order (full splits, then the shorter last ones, longest first) at a 256-position chunk: exact
    # multiples (no short split), rows shorter than a chunk (only a short one), empty rows
    (8, 2, 128, [256, 512, 300, 0, 1, 255, 257, 1024, 0, 769], 0),
    (4, 1, 64, [(i * 37) % 160 for i in range(260)], 32),   # more rows than the plan's 256 threads
])
def test_decode(oracle, qh, kvh, hd, lens, ps):
    w = W.decode("emu", qh, kvh, hd, lens, page_size=ps, seed=hd + len(lens))
    got, over, _ = emu.run_decode(w)
    want, _ = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, kvh, hd,
                                  w.rows)
    parity(got, want)
    assert over == 0


@pytest.mark.parametrize("hd,qh,kvh,first,rows,ps", [
    (256, 16, 2, 77, 95, 64),    # paged, page table in LDS, the steady loop at head_dim 256
    (128, 6, 2, 10, 70, 0),      # group 3: one head a wave
    (64, 8, 2, 300, 40, 32),     # a prefix longer than the chunk: row tiles unpaired
])
def test_causal_residual_kernel(oracle, hd, qh, kvh, first, rows, ps):
    """attention_causal_residual_paged (row 140) against the oracle's attention_weights_rows +
    attention_residual_mix_rows over the gathered cache, the pair it replaces."""
    w = W.causal("emu", qh, kvh, hd, first, rows, page_size=ps, seed=hd + rows + 1)
    got, over, _ = emu.run_causal_res(w)
    k, v = w.gathered()
    p, res = oracle.weights_rows(w.q, k, qh, kvh, hd, first, rows)
    want = oracle.residual_mix_rows(res, p, v, qh, kvh, hd, first, rows)
    residual_parity(got, want, hd)
    assert over == 0


@pytest.mark.parametrize("qh,lens,ps,shared", [
    (64, [130, 41], 0, True),       # latent attention's shape: 64 heads, one kv head, keys = values, 512 wide
    (20, [97], 64, True),           # two head blocks, the second part-full; paged
    (8, [70, 33], 16, True),        # pages shorter than a tile: one lookup a 16-key group
    (16, [130, 1], 0, False),       # head_dim 512 with values of their own
])
def test_decode_head_dim_512(oracle, qh, lens, ps, shared):
    """Row 137 at head_dim 512 (the shared-tile form when k == v) against the oracle's decode over the same cache."""
    w = W.decode("emu", qh, 1, 512, lens, page_size=ps, seed=qh + len(lens))
    got, over, _ = emu.run_decode(w, shared=shared)
    v = w.k if shared else w.v
    want, _ = oracle.decode_paged(w.q, w.k, v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, 1, 512, w.rows)
    parity(got, want)
    assert over == 0


@pytest.mark.parametrize("qh,kvh,lens,ps", [
    (64, 1, [130, 41], 0),             # latent attention's shape: one workgroup a split for all four head blocks
    (80, 1, [300, 7, 0], 64),          # five head blocks: a second workgroup with one working wave; paged; an empty row
    (20, 2, [97, 1200], 16),           # two kv heads of 10 heads; pages shorter than a tile; several splits a row
    (16, 1, [5000], 0),                # one head block (three waves idle), a ring of many tiles
])
def test_decode_latent_wide(oracle, qh, kvh, lens, ps):
    """Row 137 at head_dim 512 with the keys the values in its wide form (SILVANN_GFX950_DECODE_LATENT=wide): a
    workgroup's four waves take four head blocks of one split over a shared ring of latent tiles. The oracle's decode
    over the same cache."""
    w = W.decode("emu", qh, kvh, 512, lens, page_size=ps, seed=qh + len(lens) + 5)
    got, over, log = emu.run_decode(w, shared=True, env={"SILVANN_GFX950_DECODE_LATENT": "wide", "EMU_LAUNCHES": "1"})
    want, _ = oracle.decode_paged(w.q, w.k, w.k, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, kvh, 512,
                                  w.rows)
    parity(got, want)
    assert over == 0
    assert any("decode_latent" in ln for ln in log.splitlines() if ln.startswith("emu launch ")), log[-500:]


FUSED = {"SILVANN_GFX950_DECODE_FUSED": "1"}


@pytest.mark.parametrize("qh,kvh,hd,lens,ps", [
    (16, 2, 256, [700, 2048, 0], 256),     # a row with no positions: its answers are zeros
    (8, 2, 128, [1, 17, 3000], 0),         # a row of many splits beside one-split rows
    (4, 4, 64, [33, 250], 16),             # pages shorter than a tile
])
def test_decode_fused_finish(oracle, qh, kvh, hd, lens, ps):
    """Row 137 with the fused finish (the last split of a row and head block merges the others): the same
    answers as the oracle's decode, every split counted once — the scratch starts as garbage."""
    w = W.decode("emu", qh, kvh, hd, lens, page_size=ps, seed=hd + len(lens) + 3)
    got, over, _ = emu.run_decode(w, env=FUSED)
    want, _ = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, kvh, hd,
                                  w.rows)
    parity(got, want)
    assert over == 0


@pytest.mark.parametrize("qh,kvh,hd,lens,ps", [
    (16, 2, 256, [700, 2048], 256),
    (8, 2, 128, [1, 17, 300], 0),
    (4, 4, 64, [33, 250], 16),
])
def test_decode_transposing_reads(oracle, qh, kvh, hd, lens, ps):
    """Row 137 at head_dim <= 256 with the transposing V^T read (SILVANN_GFX950_DECODE_VTR=1, the candidate the
    head_dim-512 kernels use) against the oracle."""
    w = W.decode("emu", qh, kvh, hd, lens, page_size=ps, seed=hd + len(lens) + 7)
    got, over, _ = emu.run_decode(w, env={"SILVANN_GFX950_DECODE_VTR": "1"})
    want, _ = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, kvh, hd,
                                  w.rows)
    parity(got, want)
    assert over == 0


INLINE = {"SILVANN_GFX950_DECODE_INLINE": "1", "EMU_LAUNCHES": "1"}


@pytest.mark.parametrize("qh,kvh,hd,lens,ps", [
    (16, 2, 256, [700, 0, 2048, 0], 256),                  # empty rows between and last
    (8, 2, 128, [0, 1, 17, 3000, 5], 0),                   # an empty first row; many splits beside one-split rows
    (4, 1, 64, [(37 * i) % 150 for i in range(64)], 16),   # 64 rows (the inline plan's most), pages shorter than a tile
])
def test_decode_inline_plan(oracle, qh, kvh, hd, lens, ps):
    """Row 137 with its plan made inside decode_split (SILVANN_GFX950_DECODE_INLINE=1: each wave's prefix scan of
    the rows' split counts, an item's row found by ballot) against the oracle, with no plan launch."""
    w = W.decode("emu", qh, kvh, hd, lens, page_size=ps, seed=hd + len(lens) + 11)
    got, over, log = emu.run_decode(w, env=INLINE)
    want, _ = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, kvh, hd,
                                  w.rows)
    parity(got, want)
    assert over == 0
    launched = [ln for ln in log.splitlines() if ln.startswith("emu launch ")]
    assert len(launched) == 2 and "decode_split" in launched[0] and "decode_merge" in launched[1], launched


@pytest.mark.parametrize("qh,kvh,hd,lens,ps", [
    (16, 2, 256, [700, 0, 2048, 0], 256),                  # empty rows: zero answers from workgroup 0
    (8, 2, 128, [1, 17, 3000], 0),                         # a row of many splits beside one-split rows
    (4, 1, 64, [(37 * i) % 150 for i in range(64)], 16),   # 64 rows, pages shorter than a tile
])
@pytest.mark.parametrize("repeat", [False, True])
def test_decode_one_launch(oracle, qh, kvh, hd, lens, ps, repeat):
    """Row 137 as one launch (SILVANN_GFX950_DECODE_FUSED=1 with SILVANN_GFX950_DECODE_INLINE=1): the plan made in the
    kernel, the finish fused, its counts tagged with the call's tag over a scratch that starts as garbage — or, with
    `repeat`, over the complete counts a first call left (counted again as zero: another tag) — the oracle's
    answers, and only decode_split in the launch log."""
    w = W.decode("emu", qh, kvh, hd, lens, page_size=ps, seed=hd + len(lens) + 13)
    env = {**FUSED, **INLINE, **({"EMU_REPEAT": "1"} if repeat else {})}
    got, over, log = emu.run_decode(w, env=env)
    want, _ = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, qh, kvh, hd,
                                  w.rows)
    parity(got, want)
    assert over == 0
    launched = [ln for ln in log.splitlines() if ln.startswith("emu launch ")]
    assert len(launched) == 1 + repeat and all("decode_split" in x for x in launched), launched


@pytest.mark.parametrize("inline,repeat", [(False, False), (True, False), (True, True)])
def test_decode_fused_finish_in_two_levels(oracle, inline, repeat):
    """Rows of more than 32 splits (40 and 34 here, beside a one-split row) with the fused finish: each group of 32
    splits is merged by its last split into the group's first slot, and the group that completes the row finishes
    it, so no workgroup reads every split's residual. No merge launch; with the inline plan, one launch — also over
    the counts a first call left (`repeat`). The answers are the oracle's."""
    w = W.decode("emu", 4, 4, 64, [20000, 300, 17000], page_size=0, seed=77)
    env = {**FUSED, **(INLINE if inline else {"EMU_LAUNCHES": "1"}), **({"EMU_REPEAT": "1"} if repeat else {})}
    got, over, log = emu.run_decode(w, env=env)
    want, _ = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, w.k_row, w.lens, 4, 4, 64,
                                  w.rows)
    parity(got, want)
    assert over == 0
    launched = [ln for ln in log.splitlines() if ln.startswith("emu launch ")]
    splits = [x for x in launched if "decode_split" in x]
    assert not any("decode_merge" in x for x in launched), launched
    assert len(splits) == 1 + repeat and len(launched) == (1 + repeat) * (1 if inline else 2), launched
