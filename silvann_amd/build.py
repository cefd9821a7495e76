"""Build the gfx950 attention library in-tree: silvann_amd/libsilvann_gfx950_attention.so, and the same objects as a
SiLVANN silicon family of their own, silvann_amd/libsilvann_gfx950_family.so.

One hipcc invocation a source file (in parallel), then one link a library. Every HIP source is compiled for gfx950
only, with packed-fp32 instruction selection switched off (the pool's rule for these boxes) and every
symbol hidden except the `extern "C"` entry points include/silvann_gfx950_attention.h declares.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsilvann_gfx950_attention.so"
FAMILY = PKG / "libsilvann_gfx950_family.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _compile(src: Path) -> Path:
    """One source to its object; hipcc's per-kernel resource report (registers, spills, LDS, occupancy) goes to
    _build/<object>.resources.txt, where tests/test_resources.py reads it."""
    obj = BUILD / (src.parent.name + "_" + src.stem + ".o" if src.parent != CSRC else src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics", "-c", str(src), "-o",
           str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    lines = [line for line in (r.stdout + r.stderr).splitlines() if noise not in line]
    report = [line for line in lines if "kernel-resource-usage" in line]
    err = "\n".join(line for line in lines if "kernel-resource-usage" not in line and "remark:" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    obj.with_suffix(".resources.txt").write_text("\n".join(report) + "\n")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _link(objs: list[Path], out: Path, extra: list[str]) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), *extra, "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {out.name} failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, out)


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    family = sorted((CSRC / "family").glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources) + len(family))) as ex:
        objs = list(ex.map(_compile, sources + family))
    lib_objs, family_objs = objs[:len(sources)], objs[len(sources):]
    _link(lib_objs, LIB, [])
    # the family: the same objects and its entry point, every other name local
    _link(lib_objs + family_objs, FAMILY, [f"-Wl,--version-script={CSRC / 'family' / 'family.map'}"])
    if verbose:
        print(f"built {LIB.relative_to(PKG.parent)} from {len(sources)} sources, "
              f"{FAMILY.relative_to(PKG.parent)} with the family entry point")
    return LIB

if __name__ == "__main__":
    build()
