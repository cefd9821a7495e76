"""TEST INFRASTRUCTURE: build the CPU emulation of this library's kernels and run one call of an entry point.

`build()` turns silvann_amd/csrc/{prefill,decode}.hip into host C++ (gen.py), compiles them with the
harness against emu_rt.hpp into tests/emu/_build/emu (rebuilt when any source changes), and returns its
path. `run_causal(w)` / `run_decode(w)` run a workload from silvann_amd.workloads through the library's own
C entry point in the emulation and return the fp16 answer and the fault word.
"""
from __future__ import annotations

import concurrent.futures as cf
import fcntl
import hashlib
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BUILD = HERE / "_build"
SOURCES = ["prefill.hip", "decode.hip", "doors.hip", "tq_decode.hip", "cache.hip"]
CXX_CANDIDATES = ["/opt/rocm/llvm/bin/clang++", "/opt/rocm/lib/llvm/bin/clang++", shutil.which("clang++") or ""]
FLAGS = ["-std=c++20", "-O1", "-g", "-fno-omit-frame-pointer", "-rdynamic", "-w", "-pthread"]


def compiler() -> str | None:
    for c in CXX_CANDIDATES:
        if c and Path(c).exists():
            return c
    return None


def _digest() -> str:
    from . import gen  # noqa: F401  (the transform is part of the key)
    h = hashlib.sha256()
    for f in [*(gen.CSRC / s for s in SOURCES), gen.CSRC / "common.hpp", gen.CSRC / "tq_levels.hpp",
              HERE / "emu_rt.hpp", HERE / "gen.py",
              HERE / "harness.cpp", gen.INCLUDE / "silvann_gfx950_attention.h"]:
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def build() -> Path:
    """Build under an exclusive lock: pytest-xdist workers would otherwise regenerate and compile the same files
    at once (a source rewritten while clang reads it)."""
    BUILD.mkdir(parents=True, exist_ok=True)
    with open(BUILD / ".lock", "w") as lk:
        fcntl.flock(lk, fcntl.LOCK_EX)
        try:
            return _build_locked()
        finally:
            fcntl.flock(lk, fcntl.LOCK_UN)


def _build_locked() -> Path:
    from . import gen
    cxx = compiler()
    if cxx is None:
        raise RuntimeError("no clang++ for the emulation")
    key = _digest()
    exe = BUILD / f"emu-{key}"
    if BUILD.exists():
        for old in BUILD.glob("*"):   # builds of earlier sources
            if (old.name.startswith("emu-") or old.suffix == ".o") and key not in old.name:
                old.unlink(missing_ok=True)
    if exe.exists():
        return exe
    srcs = gen.write(BUILD, SOURCES) + [HERE / "harness.cpp"]

    def cc(src: Path) -> Path:
        obj = BUILD / (src.stem + f"-{key}.o")
        subprocess.run([cxx, *FLAGS, f"-I{BUILD}", f"-I{gen.INCLUDE}", f"-I{gen.CSRC}", "-c", str(src), "-o", str(obj)],
                       check=True)
        return obj

    with cf.ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        objs = list(ex.map(cc, srcs))
    tmp = exe.with_suffix(".tmp")
    subprocess.run([cxx, *FLAGS, *map(str, objs), "-o", str(tmp)], check=True)
    os.replace(tmp, exe)
    return exe


def _run(files: dict, params: str, env: dict | None, timeout: int, outs=(("o", np.float16),)):
    exe = build()
    with tempfile.TemporaryDirectory(prefix="silvann_emu_") as d:
        for name, arr in files.items():
            if arr is not None:
                np.ascontiguousarray(arr).tofile(f"{d}/{name}.bin")
        Path(d, "params.txt").write_text(params + f" {timeout}\n")
        r = subprocess.run([str(exe), d], capture_output=True, text=True, env={**os.environ, **(env or {})},
                           timeout=timeout + 60)
        if r.returncode != 0:
            raise RuntimeError(f"emulation exited {r.returncode}:\n{r.stderr[-4000:]}")
        got = [np.fromfile(f"{d}/{name}.bin", dtype=dt) for name, dt in outs]
        over = int(np.fromfile(f"{d}/over.bin", dtype=np.uint32)[0])
        return (*got, over, r.stderr)


def run_causal(w, env: dict | None = None, timeout: int = 900):
    pages = None if w.pages is None else w.pages.astype(np.uint32)
    params = f"causal {w.q_heads} {w.kv_heads} {w.head_dim} {w.first} {w.rows} {w.page_size} 0 0"
    return _run({"q": w.q, "k": w.k, "v": w.v, "pages": pages}, params, env, timeout)


def run_causal_res(w, env: dict | None = None, timeout: int = 900):
    """attention_causal_residual_paged: the fp32 residuals {m, l, acc} of every row and head."""
    pages = None if w.pages is None else w.pages.astype(np.uint32)
    params = f"causal_res {w.q_heads} {w.kv_heads} {w.head_dim} {w.first} {w.rows} {w.page_size} 0 0"
    return _run({"q": w.q, "k": w.k, "v": w.v, "pages": pages}, params, env, timeout, outs=(("res", np.float32),))


def run_decode(w, env: dict | None = None, timeout: int = 900, shared: bool = False):
    """`shared`: the keys are the values — one buffer passed as both (w.v is not used)."""
    pages = None if w.pages is None else w.pages.astype(np.uint32)
    params = (f"decode {w.q_heads} {w.kv_heads} {w.head_dim} {w.most} {w.rows} {w.page_size} {w.pages_row} "
              f"{w.k_row}")
    return _run({"q": w.q, "k": w.k, "v": None if shared else w.v, "pages": pages, "lens": w.lens.astype(np.uint32)},
                params, env, timeout)


def run_tq(q, codes, scales, qh, kvh, hd, length, d, rows=0, timeout: int = 900):
    """weights_tq then residual_mix_tq (their _rows forms when rows > 0), each door on its own: the weights and the
    residual after the first door, and the residual after the second."""
    params = f"{'tq_rows' if rows else 'tq'} {qh} {kvh} {hd} {length} {max(rows, 1)} {d} 0 0"
    return _run({"q": q, "k": codes, "v": scales}, params, {"SILVANN_GFX950_DEFER": "0"}, timeout,
                outs=(("p", np.float32), ("res_w", np.float32), ("res", np.float32)))


def run_tq_fused(q, k_codes, k_scales, v_codes, v_scales, qh, kvh, hd, length, d, rows=1, timeout: int = 900):
    """attention_residual_tq: the residual of `rows` query rows over the TurboQuant keys and values."""
    params = f"tq_fused {qh} {kvh} {hd} {length} {rows} {d} 0 0"
    return _run({"q": q, "k": k_codes, "v": v_codes, "pages": k_scales, "lens": v_scales}, params, None, timeout,
                outs=(("res", np.float32),))


def run_cache_write(kc, vc, pages, pages_row, page_size, capacity, positions, rows_per_seq, k, v, cs, rot, rows, kvh,
                    hd, timeout: int = 900):
    """attention_cache_write_paged over copies of the caches `kc` / `vc`: the caches after it, and the fault word."""
    pages = None if pages is None else np.ascontiguousarray(pages, np.uint32)
    params = f"cache {rot} {kvh} {hd} {rows_per_seq} {rows} {page_size} {pages_row} {capacity}"
    return _run({"q": cs, "k": k, "v": v, "pages": pages, "lens": np.ascontiguousarray(positions, np.uint32),
                 "kc": kc, "vc": vc}, params, None, timeout, outs=(("kc_out", np.uint16), ("vc_out", np.uint16)))


def run_fp16(q, k, v, qh, kvh, hd, length=0, first=0, rows=0, timeout: int = 900):
    """attention_weights + attention_residual_mix over `length` keys (rows == 0), or their _rows forms for `rows`
    rows from `first`: the weights, the residual after the first door and after the second — each door on its own
    (no deferred chain: the weights are read between the doors)."""
    many = rows > 0
    params = f"{'fp16_rows' if many else 'fp16'} {qh} {kvh} {hd} {first if many else length} {rows or 1} 0 0 0"
    return _run({"q": q, "k": k, "v": v}, params, {"SILVANN_GFX950_DEFER": "0"}, timeout,
                outs=(("p", np.float32), ("res_w", np.float32), ("res", np.float32)))


def run_grouped(q, k, v, qh, kvh, hd, most, lens=None, k_row=0, timeout: int = 900):
    """attention_scores_grouped + attention_softmax_rows + attention_mix over `most` keys (lens None), or
    scores_grouped_rows + softmax_lens + mix_rows for one row a lens entry, each door on its own: raw scores,
    weights and answers."""
    many = lens is not None
    rows = len(lens) if many else 1
    params = f"{'grouped_rows' if many else 'grouped'} {qh} {kvh} {hd} {most} {rows} 0 0 {k_row}"
    files = {"q": q, "k": k, "v": v}
    if many:
        files["lens"] = np.ascontiguousarray(lens, np.uint32)
    return _run(files, params, {"SILVANN_GFX950_DEFER": "0"}, timeout,
                outs=(("p", np.float32), ("p_soft", np.float32), ("o", np.uint16)))


def run_rope_rows(x, cs, rows, heads, head_stride, row_stride, rot, timeout: int = 900):
    """rope_rows in place on a copy of x (halves as uint16): the turned rows and the fault word."""
    params = f"rope {heads} 0 {head_stride} 0 {rows} {rot} 0 {row_stride}"
    return _run({"q": x, "k": cs}, params, None, timeout, outs=(("o", np.uint16),))


def run_chain(kind, q, k, v, qh, kvh, hd, a0, a1=0, interleave=False, defer=True, timeout: int = 900,
              extra_env: dict | None = None):
    """A reference verb's door chain through the library's doors: kind "decode" (scores, mix; a0 = length),
    "weights" (weights, residual_mix; a0 = length) or "causal" (causal_scores_grouped, causal_softmax, causal_mix;
    a0 = first, a1 = rows). `interleave` puts another door inside the chain; `defer` False runs every door on its
    own; `extra_env` adds switches. Answers the fp16 answers, the weights buffer afterwards, the residual (not for
    "causal"), the fault word and the emulation's log."""
    env = {**({} if defer else {"SILVANN_GFX950_DEFER": "0"}), **(extra_env or {})} or None
    if kind == "causal":
        params = f"chain_causal {qh} {kvh} {hd} {a0} {a1} {1 if interleave else 0} 0 0"
        return _run({"q": q, "k": k, "v": v}, params, env, timeout, outs=(("o", np.float16), ("p", np.float32)))
    params = f"chain_{kind} {qh} {kvh} {hd} {a0} {1 if interleave else 0} 0 0 0"
    return _run({"q": q, "k": k, "v": v}, params, env, timeout,
                outs=(("o", np.float16), ("p", np.float32), ("res", np.float32)))


def run_chain_residual(kind, q, kcodes, kscales, vcodes, vscales, qh, kvh, hd, a0, rows=1, d=0, interleave=False,
                       defer=True, timeout: int = 900):
    """The residual chains as the verbs call them: kind "rows" (weights_rows + residual_mix_rows from a0 = first over
    `rows` rows; kcodes/vcodes are the fp16 keys and values), "tq" (weights_tq + residual_mix_tq over a0 = length
    rows of width d) or "tq_rows" (their _rows forms for `rows` query rows). The weights buffer afterwards, the
    residuals and the fault word."""
    env = None if defer else {"SILVANN_GFX950_DEFER": "0"}
    params = f"cres_{ {'rows': 'rows', 'tq': 'tq', 'tq_rows': 'tqr'}[kind]} {qh} {kvh} {hd} {a0} {rows} {d} " \
             f"{1 if interleave else 0} 0"
    files = {"q": q, "k": kcodes, "v": vcodes, "pages": kscales, "lens": vscales}
    return _run(files, params, env, timeout, outs=(("p", np.float32), ("res", np.float32)))


def run_chain_grouped(q, k, v, qh, kvh, hd, length, sink=None, interleave=False, timeout: int = 900,
                      extra_env: dict | None = None):
    """Latent attention's chain as GLM and DeepSeek call it: attention_scores_grouped, then attention_softmax_rows
    (sink None) or attention_softmax_sink, then attention_mix. `v` None: the keys are the values. The answers, the
    weights buffer afterwards and the fault word."""
    params = f"chain_grp {qh} {kvh} {hd} {length} {0 if sink is None else 1} {1 if interleave else 0} 0 0"
    files = {"q": q, "k": k, "v": v}
    if sink is not None:
        files["lens"] = np.ascontiguousarray(sink, np.uint16)
    return _run(files, params, extra_env, timeout, outs=(("o", np.float16), ("p", np.float32)))


def run_chain_grouped_rows(q, lat, lens, qh, hd, most, interleave=False, timeout: int = 900,
                           extra_env: dict | None = None):
    """GLM's block chain: attention_scores_grouped_rows, attention_softmax_lens, attention_mix_rows, one kv head, row u
    over its own `lens[u]` latents at lat + u·most·hd (keys and values). The answers, the weights buffer afterwards
    and the fault word."""
    params = f"chain_grows {qh} 1 {hd} {most} {len(lens)} {1 if interleave else 0} 0 {most * hd}"
    return _run({"q": q, "k": lat, "lens": np.ascontiguousarray(lens, np.uint32)}, params, extra_env, timeout,
                outs=(("o", np.float16), ("p", np.float32)))
