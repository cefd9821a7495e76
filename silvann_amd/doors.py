"""The C-ABI doors, called with torch tensors for device memory.

Each function is the C entry point of the same name (include/silvann_gfx950_attention.h) with tensors in
place of pointers: a tensor is passed as its data pointer, `None` as NULL. No checks beyond that — the
reference's doors take operands their verbs already validated (packages/nn/contracts/abi/gpu.cuh:86-92);
`silvann_amd.verbs` holds the checks.
"""
from __future__ import annotations

from . import _lib


def _a(x):
    if x is None:
        return None
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    return int(x)


def _door(name):
    full = "silvann_gfx950_" + name

    def call(*args):
        return getattr(_lib.lib(), full)(*[_a(a) for a in args])

    call.__name__ = name
    call.__doc__ = f"C entry point {full}"
    return call


attention_scores = _door("attention_scores")
attention_mix = _door("attention_mix")
attention_weights = _door("attention_weights")
attention_residual_mix = _door("attention_residual_mix")
attention_merge = _door("attention_merge")
attention_finish = _door("attention_finish")
attention_causal_scores = _door("attention_causal_scores")
attention_causal_mix = _door("attention_causal_mix")
attention_weights_tq = _door("attention_weights_tq")
attention_residual_mix_tq = _door("attention_residual_mix_tq")
attention_scores_grouped = _door("attention_scores_grouped")
attention_softmax_rows = _door("attention_softmax_rows")
attention_causal_scores_grouped = _door("attention_causal_scores_grouped")
attention_causal_softmax = _door("attention_causal_softmax")
attention_softmax_sink = _door("attention_softmax_sink")
attention_weights_rows = _door("attention_weights_rows")
attention_residual_mix_rows = _door("attention_residual_mix_rows")
attention_weights_tq_rows = _door("attention_weights_tq_rows")
attention_residual_mix_tq_rows = _door("attention_residual_mix_tq_rows")
attention_scores_grouped_rows = _door("attention_scores_grouped_rows")
attention_softmax_lens = _door("attention_softmax_lens")
attention_mix_rows = _door("attention_mix_rows")
rope_rows = _door("rope_rows")
attention_decode_paged = _door("attention_decode_paged")
attention_decode_paged_scratch = _door("attention_decode_paged_scratch")
attention_causal_paged = _door("attention_causal_paged")
attention_causal_residual_paged = _door("attention_causal_residual_paged")
attention_residual_tq = _door("attention_residual_tq")
attention_cache_write_paged = _door("attention_cache_write_paged")
attention_residual_tq_scratch = _door("attention_residual_tq_scratch")


def set_stream(stream) -> None:
    """Queue this thread's doors on `stream` (a torch.cuda.Stream, a raw hipStream_t int, or None)."""
    raw = None if stream is None else getattr(stream, "cuda_stream", stream)
    _lib.lib().silvann_gfx950_set_stream(raw)


def flush() -> None:
    """Run a deferred chain door now (its weights are then in its buffer)."""
    _lib.lib().silvann_gfx950_flush()


def set_defer(on: bool) -> None:
    """Deferral of chain doors on this thread (default on; SILVANN_GFX950_DEFER=0 makes off the default)."""
    _lib.lib().silvann_gfx950_set_defer(1 if on else 0)


def launch_failed() -> bool:
    return bool(_lib.lib().silvann_gfx950_launch_failed())


def version() -> str:
    return _lib.lib().silvann_gfx950_version().decode()
