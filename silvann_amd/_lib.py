"""Loads libsilvann_gfx950_attention.so and types its C entry points.

The library is the product: there is no fallback. If it is not built, `lib()` raises — on a GPU box a
missing extension is an error, never a silent CPU path.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libsilvann_gfx950_attention.so"
HEADER = PKG.parent / "include" / "silvann_gfx950_attention.h"

_u64, _p, _u32p = C.c_uint64, C.c_void_p, C.c_void_p

# argument types of every entry point, in header order
SIGNATURES = {
    "silvann_gfx950_attention_scores": [_p, _p, _p, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_mix": [_p, _p, _p, _u64, _u64, _u64, _u64, _p],
    "silvann_gfx950_attention_weights": [_p, _p, _p, _p, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_residual_mix": [_p, _p, _p, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_merge": [_p, _p, _p, _u64, _u64],
    "silvann_gfx950_attention_finish": [_p, _p, _u64, _u64, _p],
    "silvann_gfx950_attention_causal_scores": [_p, _p, _p, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_causal_mix": [_p, _p, _p, _u64, _u64, _u64, _u64, _u64, _p],
    "silvann_gfx950_attention_weights_tq": [_p, _p, _p, _p, _p, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_residual_mix_tq": [_p, _p, _p, _p, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_scores_grouped": [_p, _p, _p, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_softmax_rows": [_p, _u64, _u64],
    "silvann_gfx950_attention_causal_scores_grouped": [_p, _p, _p, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_causal_softmax": [_p, _u64, _u64, _u64],
    "silvann_gfx950_attention_softmax_sink": [_p, _p, _u64, _u64],
    "silvann_gfx950_attention_weights_rows": [_p, _p, _p, _p, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_residual_mix_rows": [_p, _p, _p, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_weights_tq_rows": [_p, _p, _p, _p, _p, _u64, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_residual_mix_tq_rows": [_p, _p, _p, _p, _u64, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_scores_grouped_rows": [_p, _u64, _p, _u64, _p, _u64, _p, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_softmax_lens": [_p, _u64, _p, _u64, _u64],
    "silvann_gfx950_attention_mix_rows": [_p, _u64, _p, _u64, _p, _u64, _p, _u64, _u64, _u64, _u64, _p],
    "silvann_gfx950_rope_rows": [_p, _p, _p, _u64, _u64, _u64, _u64, _u64, _p],
    "silvann_gfx950_attention_decode_paged": [_p, _p, _p, _p, _p, _u64, _u64, _u64, _p, _u64, _u64, _u64, _u64, _u64,
                                              _p, _p],
    "silvann_gfx950_attention_decode_paged_scratch": [_u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_causal_paged": [_p, _p, _p, _p, _p, _u64, _u64, _u64, _u64, _u64, _u64, _p],
    "silvann_gfx950_attention_causal_residual_paged": [_p, _p, _p, _p, _p, _u64, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_attention_cache_write_paged": [_p, _p, _p, _u64, _u64, _u64, _p, _u64, _p, _p, _p, _u64, _u64,
                                                   _u64, _u64, _p],
    "silvann_gfx950_attention_residual_tq": [_p, _p, _p, _p, _p, _p, _u64, _u64, _u64, _u64, _u64, _u64, _p],
    "silvann_gfx950_attention_residual_tq_scratch": [_u64, _u64, _u64, _u64, _u64, _u64],
    "silvann_gfx950_set_stream": [_p],
    "silvann_gfx950_get_stream": [],
    "silvann_gfx950_flush": [],
    "silvann_gfx950_set_defer": [C.c_int],
    "silvann_gfx950_launch_failed": [],
    "silvann_gfx950_profile_enable": [C.c_int],
    "silvann_gfx950_profile_read": [C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64)],
    "silvann_gfx950_attention_install": [_p],
    "silvann_gfx950_version": [],
}
RESTYPES = {
    "silvann_gfx950_attention_decode_paged_scratch": _u64,
    "silvann_gfx950_attention_residual_tq_scratch": _u64,
    "silvann_gfx950_get_stream": _p,
    "silvann_gfx950_launch_failed": C.c_int,
    "silvann_gfx950_profile_read": C.c_int,
    "silvann_gfx950_attention_install": C.c_uint32,
    "silvann_gfx950_version": C.c_char_p,
}


class LibraryMissing(RuntimeError):
    pass


_LIB = None


def header_functions() -> list[str]:
    """Every function include/silvann_gfx950_attention.h declares."""
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:void|uint64_t|uint32_t|int|const char\*|void\*)\s+(silvann_gfx950_\w+)\s*\(", text, re.M)


def lib() -> C.CDLL:
    """The library, loaded once a process: LIB_PATH, or the build SILVANN_GFX950_LIB names (an experiment build of
    the same sources)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("SILVANN_GFX950_LIB") or LIB_PATH)
    if not path.exists():
        raise LibraryMissing(f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                             "or `python silvann_amd/build.py`")
    L = C.CDLL(str(path))
    for name, args in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = RESTYPES.get(name)
    _LIB = L
    return L
