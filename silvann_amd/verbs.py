"""The host side of the reference's attention verbs, over this library's doors.

Each verb checks its operands the way the reference's verb does and refuses with the same fault word,
then calls the doors in the same order with the same pointers (packages/nn/cpu/opcodes/attention__abi.cuh).
A buffer is a torch tensor on the GPU; its "room" is its size in halves, as `nn__primitives__room` counts
(packages/nn/cpu/primitives__header.cuh:38-55). Integers are Python ints. A refusal raises `Fault`
carrying the word; nothing is launched.

The two paged verbs are new (the reference has no page table): `decode_paged` and `causal_paged`, the
split-K decode and the fused causal prefill, with the same kind of checks.

The reference's verbs call their doors as chains (`decode`: scores then mix; `residual`: weights then residual_mix;
`rows_attention`: causal scores, softmax, mix; `residual_tq`; the window's pairs); the library defers a chain's first
door and runs the chain fused, so these verbs reach the fast kernels with the reference's own call sequence.
"""
from __future__ import annotations

import torch

from . import doors

FAULT_TYPE = 0x4F504354      # "OPCT" packages/sys/contracts/objects/opcodes.cuh:6
FAULT_BOUNDS = 0x4E50424E    # "NPBN" packages/nn/contracts/objects/primitives.cuh:5
FAULT_OVERFLOW = 0x4E504F56  # "NPOV" primitives.cuh:57
FAULT_ROOM = 0x4E41524D      # "NARM" packages/nn/contracts/objects/attention.cuh:46
DIM_MAX = 1 << 20            # attention__abi.cuh:28 NN__ATTENTION__DIM_MAX
ELEMENT_BYTES = 2            # primitives.cuh:82


class Fault(RuntimeError):
    def __init__(self, word: int):
        self.word = word
        super().__init__(f"fault {word.to_bytes(4, 'big').decode(errors='replace')} (0x{word:08X})")


def word(name: str) -> int:
    return int.from_bytes(name.encode(), "big")


def room(t: torch.Tensor) -> int:
    return t.numel() * t.element_size() // ELEMENT_BYTES


def _dim(x) -> int:
    """attention__abi.cuh:30-34: an integer in (0, DIM_MAX]."""
    if not isinstance(x, int) or isinstance(x, bool) or x == 0 or x > DIM_MAX or x < 0:
        raise Fault(FAULT_TYPE)
    return x


def _fits(n: int, r: int) -> bool:
    return n <= r


def check_fault(over: torch.Tensor) -> None:
    """Raise the fault a door left in the fault word, as the engine does at the next apply."""
    w = int(over.view(torch.int32)[0].item()) & 0xFFFFFFFF
    if w:
        raise Fault(w)


def decode(q, k, v, scores, out, q_heads, kv_heads, head_dim, from_, to, over):
    """`(nn__attention__decode q k v scores out q_heads kv_heads head_dim from to)` — attention__abi.cuh:129-160."""
    q_heads, kv_heads, head_dim, to = _dim(q_heads), _dim(kv_heads), _dim(head_dim), _dim(to)
    if not isinstance(from_, int) or from_ < 0:
        raise Fault(FAULT_TYPE)
    row = kv_heads * head_dim
    if from_ >= to:
        raise Fault(FAULT_BOUNDS)
    length, cached = to - from_, to * row
    if (q_heads % kv_heads or not _fits(q_heads * head_dim, room(q)) or not _fits(q_heads * head_dim, room(out))
            or not _fits(cached, room(k)) or not _fits(cached, room(v))
            or not _fits(2 * q_heads * length, room(scores))):
        raise Fault(FAULT_BOUNDS)
    skip = from_ * row * ELEMENT_BYTES
    doors.attention_scores(scores, q, k.data_ptr() + skip, q_heads, kv_heads, head_dim, length)
    doors.attention_mix(out, scores, v.data_ptr() + skip, q_heads, kv_heads, head_dim, length, over)
    return out


def _residual_fits(t, q_heads, head_dim) -> bool:
    return _fits(2 * q_heads * (head_dim + 2), room(t))


def residual(q, k, v, scores, res, q_heads, kv_heads, head_dim, from_, to):
    """`(nn__attention__residual …)` — attention__abi.cuh:177-208."""
    q_heads, kv_heads, head_dim, to = _dim(q_heads), _dim(kv_heads), _dim(head_dim), _dim(to)
    if not isinstance(from_, int) or from_ < 0:
        raise Fault(FAULT_TYPE)
    row = kv_heads * head_dim
    if from_ >= to:
        raise Fault(FAULT_BOUNDS)
    length, cached = to - from_, to * row
    if (q_heads % kv_heads or not _fits(q_heads * head_dim, room(q)) or not _fits(cached, room(k))
            or not _fits(cached, room(v)) or not _fits(2 * q_heads * length, room(scores))
            or not _residual_fits(res, q_heads, head_dim)):
        raise Fault(FAULT_BOUNDS)
    skip = from_ * row * ELEMENT_BYTES
    doors.attention_weights(scores, res, q, k.data_ptr() + skip, q_heads, kv_heads, head_dim, length)
    doors.attention_residual_mix(res, scores, v.data_ptr() + skip, q_heads, kv_heads, head_dim, length)
    return res


def tq_row_bytes(d: int, cols: int) -> int:
    """kernels.cuh:2814-2817: a TurboQuant row of `cols` values is whole 16-bit containers of 16 / d codes."""
    per = 16 // d
    return (cols + per - 1) // per * 2


def residual_tq(q, k_codes, k_scales, v_codes, v_scales, scores, res, q_heads, kv_heads, head_dim, d, count):
    """`(nn__attention__residual_tq q kc ks vc vs scores res q_heads kv_heads head_dim d count)` —
    attention__abi.cuh:245-272: a residual over `count` TurboQuant key and value rows (width d, 4 or 8), the
    query already rotated. The scores hold no weights afterwards (the mix keeps its sums there)."""
    q_heads, kv_heads, head_dim = _dim(q_heads), _dim(kv_heads), _dim(head_dim)
    d, count = _dim(d), _dim(count)
    if d not in (4, 8) or q_heads % kv_heads:
        raise Fault(FAULT_TYPE)
    rows = count * kv_heads
    code_bytes = rows * tq_row_bytes(d, head_dim)
    # the reference compares the codes' bytes with their buffers' room as it counts it (attention__abi.cuh:262-265)
    if (not _fits(q_heads * head_dim, room(q)) or code_bytes > room(k_codes) or not _fits(rows, room(k_scales))
            or code_bytes > room(v_codes) or not _fits(rows, room(v_scales))
            or not _fits(2 * q_heads * count, room(scores)) or not _residual_fits(res, q_heads, head_dim)):
        raise Fault(FAULT_BOUNDS)
    doors.attention_weights_tq(scores, res, q, k_codes, k_scales, q_heads, kv_heads, head_dim, count, d)
    doors.attention_residual_mix_tq(res, scores, v_codes, v_scales, q_heads, kv_heads, head_dim, count, d)
    return res


def residual_tq_scratch_bytes(q_heads, kv_heads, head_dim, count, d, rows=1) -> int:
    return int(doors.attention_residual_tq_scratch(q_heads, kv_heads, head_dim, count, d, rows))


def residual_tq_fused(q, k_codes, k_scales, v_codes, v_scales, res, scratch, q_heads, kv_heads, head_dim, d, count,
                      rows=1):
    """`residual_tq`'s answer through the fused row (attention_residual_tq): the same operand checks
    (attention__abi.cuh:245-266), no weights materialised, `rows` query rows over the same keys (the tiered
    prefill window, prefill__abi.cuh:437-440). `scratch` holds residual_tq_scratch_bytes(...) bytes."""
    q_heads, kv_heads, head_dim = _dim(q_heads), _dim(kv_heads), _dim(head_dim)
    d, count, rows = _dim(d), _dim(count), _dim(rows)
    if d not in (4, 8) or q_heads % kv_heads or head_dim not in (64, 128, 256):
        raise Fault(FAULT_TYPE)
    n = count * kv_heads
    code_bytes = n * tq_row_bytes(d, head_dim)
    if (not _fits(rows * q_heads * head_dim, room(q)) or code_bytes > room(k_codes) or not _fits(n, room(k_scales))
            or code_bytes > room(v_codes) or not _fits(n, room(v_scales))
            or not _fits(2 * rows * q_heads * (head_dim + 2), room(res))
            or scratch.numel() * scratch.element_size()
            < residual_tq_scratch_bytes(q_heads, kv_heads, head_dim, count, d, rows)):
        raise Fault(FAULT_BOUNDS)
    doors.attention_residual_tq(res, q, k_codes, k_scales, v_codes, v_scales, q_heads, kv_heads, head_dim, count, d,
                                rows, scratch)
    return res


def merge(a, b, into, q_heads, head_dim):
    """`(nn__attention__merge a b into q_heads head_dim)` — attention__abi.cuh:212-227."""
    q_heads, head_dim = _dim(q_heads), _dim(head_dim)
    if not (_residual_fits(a, q_heads, head_dim) and _residual_fits(b, q_heads, head_dim)
            and _residual_fits(into, q_heads, head_dim)):
        raise Fault(FAULT_BOUNDS)
    doors.attention_merge(into, a, b, q_heads, head_dim)
    return into


def finish(res, out, q_heads, head_dim, over):
    """`(nn__attention__finish res out q_heads head_dim)` — attention__abi.cuh:230-243."""
    q_heads, head_dim = _dim(q_heads), _dim(head_dim)
    if not _residual_fits(res, q_heads, head_dim) or not _fits(q_heads * head_dim, room(out)):
        raise Fault(FAULT_BOUNDS)
    doors.attention_finish(out, res, q_heads, head_dim, over)
    return out


def rows_attention(q, keys, values, scores, att, q_heads, kv_heads, head_dim, first, rows, over):
    """The attention of `nn__attention__rows` (attention__abi.cuh:345-421, the part at 370 and 407-414):
    queries `q` for positions first .. first+rows-1 (their keys and values already in the cache) attend the
    cache causally, as many rows a pass as the scores' room holds — causal_scores_grouped, causal_softmax,
    causal_mix — into `att`. The verb's own limits on the whole layer (ROWS_MAX, the 512-blocks) belong to its
    projections and are not this part's."""
    q_heads, kv_heads, head_dim = _dim(q_heads), _dim(kv_heads), _dim(head_dim)
    if not isinstance(first, int) or first < 0 or first >= (1 << 32) or not isinstance(rows, int) or rows <= 0:
        raise Fault(word("NATB"))
    qw, kvw, to = q_heads * head_dim, kv_heads * head_dim, first + rows
    if head_dim % 2 or q_heads % kv_heads:
        raise Fault(word("NATB"))
    if (not _fits(rows * qw, room(q)) or not _fits(rows * qw, room(att)) or not _fits(to * kvw, room(keys))
            or not _fits(to * kvw, room(values)) or scores.numel() * scores.element_size() // 4 < q_heads * to):
        raise Fault(FAULT_ROOM)
    per = scores.numel() * scores.element_size() // 4 // (q_heads * to)
    npass = min(rows, per)
    r0 = 0
    while r0 < rows:
        n = min(npass, rows - r0)
        doors.attention_causal_scores_grouped(scores, q.data_ptr() + 2 * r0 * qw, keys, q_heads, kv_heads, head_dim,
                                              first + r0, n)
        doors.attention_causal_softmax(scores, q_heads, first + r0, n)
        doors.attention_causal_mix(att.data_ptr() + 2 * r0 * qw, scores, values, q_heads, kv_heads, head_dim,
                                   first + r0, n, over)
        r0 += n
    return att


def decode_paged_scratch_bytes(q_heads, kv_heads, head_dim, most, rows) -> int:
    return int(doors.attention_decode_paged_scratch(q_heads, kv_heads, head_dim, most, rows))


def decode_paged(q, k, v, pages, lens, out, q_heads, kv_heads, head_dim, most, page_size=0, pages_row=0, k_row=0,
                 scratch=None, over=None):
    """One query position a row over its own (paged) cache — the split-K decode door. `pages` None: each row's
    cache is contiguous at k + u·k_row. `lens` a uint32 GPU tensor of the rows' lengths, `most` ≥ every one."""
    q_heads, kv_heads, head_dim, most = _dim(q_heads), _dim(kv_heads), _dim(head_dim), _dim(most)
    rows = lens.numel()
    if rows == 0 or q_heads % kv_heads or head_dim not in (64, 128, 256):
        raise Fault(FAULT_BOUNDS)
    if not _fits(rows * q_heads * head_dim, room(q)) or not _fits(rows * q_heads * head_dim, room(out)):
        raise Fault(FAULT_BOUNDS)
    if pages is not None:
        if page_size <= 0 or page_size % 16 or pages_row * (rows - 1) + (most + page_size - 1) // page_size > pages.numel():
            raise Fault(FAULT_BOUNDS)
    need = decode_paged_scratch_bytes(q_heads, kv_heads, head_dim, most, rows)
    if scratch is None:
        scratch = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
    elif scratch.numel() * scratch.element_size() < need:
        raise Fault(FAULT_BOUNDS)
    if over is None:
        over = torch.zeros(1, dtype=torch.int32, device=q.device)
    doors.attention_decode_paged(out, q, k, v, pages, pages_row, page_size, k_row, lens, q_heads, kv_heads, head_dim,
                                 most, rows, scratch, over)
    return out


def causal_paged(q, k, v, pages, out, q_heads, kv_heads, head_dim, first, rows, page_size=0, over=None):
    """Causal prefill of positions first .. first+rows-1 over the (paged) cache — the fused MFMA door."""
    q_heads, kv_heads, head_dim = _dim(q_heads), _dim(kv_heads), _dim(head_dim)
    if (not isinstance(first, int) or first < 0 or not isinstance(rows, int) or rows <= 0 or q_heads % kv_heads
            or head_dim not in (64, 128, 256)):
        raise Fault(FAULT_BOUNDS)
    qw, kvw, to = q_heads * head_dim, kv_heads * head_dim, first + rows
    if to >= 1 << 31 or not _fits(rows * qw, room(q)) or not _fits(rows * qw, room(out)):
        raise Fault(FAULT_BOUNDS)
    if pages is None:
        if not _fits(to * kvw, room(k)) or not _fits(to * kvw, room(v)):
            raise Fault(FAULT_BOUNDS)
    elif page_size <= 0 or page_size % 32 or (to + page_size - 1) // page_size > pages.numel():
        raise Fault(FAULT_BOUNDS)
    if over is None:
        over = torch.zeros(1, dtype=torch.int32, device=q.device)
    doors.attention_causal_paged(out, q, k, v, pages, page_size, q_heads, kv_heads, head_dim, first, rows, over)
    return out


def causal_residual_paged(q, k, v, pages, res, q_heads, kv_heads, head_dim, first, rows, page_size=0):
    """The residuals {m, l, acc} of positions first .. first+rows-1 over the (paged) cache, row r's at
    res + r·q_heads·(head_dim + 2) — what weights_rows + residual_mix_rows leave (doors.cuh:201-204,417-432),
    in one launch of the fused MFMA door (row 140). The same checks as causal_paged."""
    q_heads, kv_heads, head_dim = _dim(q_heads), _dim(kv_heads), _dim(head_dim)
    if (not isinstance(first, int) or first < 0 or not isinstance(rows, int) or rows <= 0 or q_heads % kv_heads
            or head_dim not in (64, 128, 256)):
        raise Fault(FAULT_BOUNDS)
    qw, kvw, to = q_heads * head_dim, kv_heads * head_dim, first + rows
    if to >= 1 << 31 or not _fits(rows * qw, room(q)) or not _fits(2 * rows * q_heads * (head_dim + 2), room(res)):
        raise Fault(FAULT_BOUNDS)
    if pages is None:
        if not _fits(to * kvw, room(k)) or not _fits(to * kvw, room(v)):
            raise Fault(FAULT_BOUNDS)
    elif page_size <= 0 or page_size % 32 or (to + page_size - 1) // page_size > pages.numel():
        raise Fault(FAULT_BOUNDS)
    doors.attention_causal_residual_paged(res, q, k, v, pages, page_size, q_heads, kv_heads, head_dim, first, rows)
    return res


# ── the tiered prefill window (ai_qwen_3 prefill__abi.cuh:409-447, step ④) ─────────────────────────────────

WARM_BITS, COLD_BITS = 8, 4   # prefill__abi.cuh:433: the warm tier's codes are 8 bits, the cold tier's 4


def _tier_ok(tier, kv_heads, head_dim, d) -> bool:
    if tier is None:
        return True
    kc, ks, vc, vs, count = tier
    n = count * kv_heads
    b = n * tq_row_bytes(d, head_dim)
    return b <= room(kc) and b <= room(vc) and _fits(n, room(ks)) and _fits(n, room(vs))


def _window_checks(q, window_k, window_v, first_w, rows, warm, cold, res, att, q_heads, kv_heads, head_dim):
    q_heads, kv_heads, head_dim = _dim(q_heads), _dim(kv_heads), _dim(head_dim)
    if not isinstance(first_w, int) or first_w < 0 or not isinstance(rows, int) or rows <= 0 or q_heads % kv_heads:
        raise Fault(FAULT_TYPE)
    qw, kvw, window = q_heads * head_dim, kv_heads * head_dim, first_w + rows
    warm = None if warm is None or warm[4] == 0 else warm
    cold = None if cold is None or cold[4] == 0 else cold
    if (not _fits(rows * qw, room(q)) or not _fits(rows * qw, room(att)) or not _fits(window * kvw, room(window_k))
            or not _fits(window * kvw, room(window_v)) or not _tier_ok(warm, kv_heads, head_dim, WARM_BITS)
            or not _tier_ok(cold, kv_heads, head_dim, COLD_BITS)
            or ((warm or cold) and not _fits(2 * 3 * rows * q_heads * (head_dim + 2), room(res)))):
        raise Fault(FAULT_BOUNDS)
    return q_heads, kv_heads, head_dim, window, warm, cold


def window_attention(q, window_k, window_v, first_w, rows, warm, cold, scores, rows_scores, res, att, q_heads,
                     kv_heads, head_dim, over):
    """Step ④ of ai_qwen_3's tiered prefill (prefill__abi.cuh:409-447) as the reference runs it, through the
    reference's doors: the chunk's `rows` query rows `q` are the last rows of the fp16 window (`first_w` positions
    before them), contiguous in `window_k` / `window_v`. With no warm or cold rows the chunk attends the window
    causally (causal_scores_grouped, causal_softmax, causal_mix, 414-418). Past that each row's residual over the
    window up to its own position (weights_rows + residual_mix_rows), over the whole warm tier (8-bit
    weights_tq_rows + residual_mix_tq_rows) and over the whole cold tier (4-bit), as many rows a pass as
    `rows_scores` holds (one row at a time in `scores` when it holds none), merged and finished into `att`.
    `warm` / `cold` are (k_codes, k_scales, v_codes, v_scales, count) or None; `res` holds three residual blocks of
    rows·q_heads·(head_dim + 2) floats (r0, r1, r2)."""
    q_heads, kv_heads, head_dim, window, warm, cold = _window_checks(
        q, window_k, window_v, first_w, rows, warm, cold, res, att, q_heads, kv_heads, head_dim)
    qw = q_heads * head_dim
    if warm is None and cold is None:
        if rows_scores.numel() * rows_scores.element_size() // 4 < rows * q_heads * window:
            raise Fault(FAULT_ROOM)
        doors.attention_causal_scores_grouped(rows_scores, q, window_k, q_heads, kv_heads, head_dim, first_w, rows)
        doors.attention_causal_softmax(rows_scores, q_heads, first_w, rows)
        doors.attention_causal_mix(att, rows_scores, window_v, q_heads, kv_heads, head_dim, first_w, rows, over)
        return att
    rw = 4 * q_heads * (head_dim + 2)                       # a row's residual, in bytes
    r0 = res.data_ptr()
    r1, r2 = r0 + rows * rw, r0 + 2 * rows * rw
    longest = max(window, warm[4] if warm else 0, cold[4] if cold else 0)
    if scores.numel() * scores.element_size() // 4 < q_heads * longest:
        raise Fault(FAULT_ROOM)
    for part, span, tier, into in ((0, window, None, r0), (1, warm[4] if warm else 0, warm, r1),
                                   (2, cold[4] if cold else 0, cold, r2)):
        if span == 0:
            continue
        fit = rows_scores.numel() * rows_scores.element_size() // 4 // (q_heads * span)
        per = 1 if fit == 0 else min(fit, rows)
        pp = scores if fit == 0 else rows_scores
        for r in range(0, rows, per):
            n = min(per, rows - r)
            qrr = q.data_ptr() + 2 * r * qw
            if part == 0:
                doors.attention_weights_rows(pp, into + r * rw, qrr, window_k, q_heads, kv_heads, head_dim, first_w + r,
                                             n)
                doors.attention_residual_mix_rows(into + r * rw, pp, window_v, q_heads, kv_heads, head_dim, first_w + r,
                                                  n)
            else:
                kc, ks, vc, vs, _ = tier
                bits = WARM_BITS if part == 1 else COLD_BITS
                doors.attention_weights_tq_rows(pp, into + r * rw, qrr, kc, ks, q_heads, kv_heads, head_dim, span, bits,
                                                n)
                doors.attention_residual_mix_tq_rows(into + r * rw, pp, vc, vs, q_heads, kv_heads, head_dim, span, bits,
                                                     n)
    if warm:
        doors.attention_merge(r0, r0, r1, rows * q_heads, head_dim)
    if cold:
        doors.attention_merge(r0, r0, r2, rows * q_heads, head_dim)
    doors.attention_finish(att, r0, rows * q_heads, head_dim, over)
    return att


def window_scratch_bytes(q_heads, kv_heads, head_dim, rows, warm_count, cold_count) -> int:
    """Scratch window_attention_fused needs: the larger of the two tiers' fused-residual scratch (they run one
    after the other on the stream)."""
    need = 0
    for count, d in ((warm_count, WARM_BITS), (cold_count, COLD_BITS)):
        if count:
            need = max(need, residual_tq_scratch_bytes(q_heads, kv_heads, head_dim, count, d, rows))
    return need


def window_attention_fused(q, window_k, window_v, first_w, rows, warm, cold, res, scratch, att, q_heads, kv_heads,
                           head_dim, over):
    """window_attention's answer through the fused rows: the window part is one causal launch on MFMA (row 138
    straight into `att` when there are no tiers, else row 140's residuals), each tier one fused TurboQuant
    residual (row 139) over all the chunk's rows; then the reference's merge and finish. No weights are
    materialised. head_dim 64, 128 or 256; `scratch` holds window_scratch_bytes(...) bytes."""
    q_heads, kv_heads, head_dim, window, warm, cold = _window_checks(
        q, window_k, window_v, first_w, rows, warm, cold, res, att, q_heads, kv_heads, head_dim)
    if head_dim not in (64, 128, 256) or window >= 1 << 31:
        raise Fault(FAULT_TYPE)
    if warm is None and cold is None:
        doors.attention_causal_paged(att, q, window_k, window_v, None, 0, q_heads, kv_heads, head_dim, first_w, rows,
                                     over)
        return att
    need = window_scratch_bytes(q_heads, kv_heads, head_dim, rows, warm[4] if warm else 0, cold[4] if cold else 0)
    if scratch is None or scratch.numel() * scratch.element_size() < need:
        raise Fault(FAULT_BOUNDS)
    rw = 4 * q_heads * (head_dim + 2)
    r0 = res.data_ptr()
    r1, r2 = r0 + rows * rw, r0 + 2 * rows * rw
    doors.attention_causal_residual_paged(r0, q, window_k, window_v, None, 0, q_heads, kv_heads, head_dim, first_w, rows)
    for tier, into, bits in ((warm, r1, WARM_BITS), (cold, r2, COLD_BITS)):
        if tier:
            kc, ks, vc, vs, count = tier
            doors.attention_residual_tq(into, q, kc, ks, vc, vs, q_heads, kv_heads, head_dim, count, bits, rows, scratch)
    if warm:
        doors.attention_merge(r0, r0, r1, rows * q_heads, head_dim)
    if cold:
        doors.attention_merge(r0, r0, r2, rows * q_heads, head_dim)
    doors.attention_finish(att, r0, rows * q_heads, head_dim, over)
    return att


# ── the page-aware cache writer ──────────────────────────────────────────────────────────────────────────


def cache_write_paged(k_cache, v_cache, pages, positions, k, v, cs, kv_heads, head_dim, rows, rows_per_seq,
                      capacity, page_size=0, pages_row=0, rot=None, over=None):
    """New key and value rows into their slots (row 141): what the reference's rows verb does with `rope_rows`
    pointed at the contiguous cache and the value projection's placement (attention__abi.cuh:398-406), over a paged
    cache. `positions` a uint32 GPU tensor, a sequence's first new position each; `cs` the rows' angles (rot/2
    cosines then rot/2 sines a row, fp32) or None; `rot` defaults to head_dim. A row at or past `capacity` leaves
    NPBN in the fault word (check_fault raises it)."""
    kv_heads, head_dim, rows, rows_per_seq = _dim(kv_heads), _dim(head_dim), _dim(rows), _dim(rows_per_seq)
    if not isinstance(capacity, int) or capacity <= 0 or capacity >= 1 << 32:
        raise Fault(FAULT_BOUNDS)
    rot = head_dim if rot is None else rot
    if cs is not None and (rot % 2 or rot > head_dim or rot <= 0):
        raise Fault(FAULT_TYPE)
    row = kv_heads * head_dim
    nseq = (rows + rows_per_seq - 1) // rows_per_seq
    if (not _fits(rows * row, room(k)) or not _fits(rows * row, room(v)) or positions.numel() < nseq
            or (cs is not None and cs.numel() < rows * rot)):
        raise Fault(FAULT_BOUNDS)
    if pages is None:
        if not _fits(nseq * capacity * row, room(k_cache)) or not _fits(nseq * capacity * row, room(v_cache)):
            raise Fault(FAULT_BOUNDS)
    elif (page_size <= 0 or pages_row < (capacity + page_size - 1) // page_size
          or pages.numel() < (nseq - 1) * pages_row + (capacity + page_size - 1) // page_size):
        raise Fault(FAULT_BOUNDS)
    if over is None:
        over = torch.zeros(1, dtype=torch.int32, device=k.device)
    doors.attention_cache_write_paged(k_cache, v_cache, pages, pages_row, page_size, capacity, positions, rows_per_seq,
                                      k, v, cs, rot if cs is not None else 0, rows, kv_heads, head_dim, over)
    return over


# ── multi-head latent attention (GLM 5.3, DeepSeek) ──────────────────────────────────────────────────────────

def latent_attention(q, latents, lens, out, heads, latent_dim, most, k_row=0, scratch=None, over=None):
    """The latent attention of GLM 5.3's MLA (ai_z__glm_5_3/cpu/opcodes/layer__abi.cuh:283-289 for one query,
    1037-1043 for a block of rows over their gathered sets): `heads` query heads over one cache of latents that are
    both the keys and the values — scores_grouped(_rows) + softmax_rows / softmax_lens + mix(_rows) with one kv head
    — in one pass of the split-K decode door (row 137) with k = v, each latent read once. Row u's `heads` queries at
    q + u·heads·latent_dim attend latents 0 .. lens[u]-1 at latents + u·k_row; its answers go to
    out + u·heads·latent_dim. `lens` a uint32 GPU tensor, `most` ≥ every one."""
    heads, latent_dim, most = _dim(heads), _dim(latent_dim), _dim(most)
    rows = lens.numel()
    if rows == 0 or latent_dim not in (64, 128, 256, 512):
        raise Fault(FAULT_TYPE)
    if (not _fits(rows * heads * latent_dim, room(q)) or not _fits(rows * heads * latent_dim, room(out))
            or not _fits((rows - 1) * k_row + most * latent_dim, room(latents))):
        raise Fault(FAULT_BOUNDS)
    need = decode_paged_scratch_bytes(heads, 1, latent_dim, most, rows)
    if scratch is None:
        scratch = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
    elif scratch.numel() * scratch.element_size() < need:
        raise Fault(FAULT_BOUNDS)
    if over is None:
        over = torch.zeros(1, dtype=torch.int32, device=q.device)
    doors.attention_decode_paged(out, q, latents, latents, None, 0, 0, k_row, lens, heads, 1, latent_dim, most, rows,
                                 scratch, over)
    return out
