"""TEST INFRASTRUCTURE: turn this library's HIP sources into host C++ for the CPU emulation (emu_rt.hpp).

The kernels are used as they are. The transformation is textual and small: the HIP runtime header and the
LDS address-space qualifier go, `<<<grid, block, lds, stream>>>(args)` launches become emu::launch calls, and
the few inline-assembly helpers (direct-to-LDS loads, a scalar load, an in-place accumulator scale) become
their host equivalents. Anything else the emulation does not know stops the build.
"""
from __future__ import annotations

import re
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent.parent / "silvann_amd" / "csrc"
INCLUDE = HERE.parent.parent / "include"
AS3 = "__attribute__((address_space(3)))"


def _sub(pattern: str, repl: str, s: str, what: str, required: bool = True) -> str:
    out, n = re.subn(pattern, repl, s, flags=re.S)
    if required and n == 0:
        raise RuntimeError(f"emulation source transform: {what} not found")
    return out


def common() -> str:
    s = (CSRC / "common.hpp").read_text()
    s = s.replace("#include <hip/hip_runtime.h>", '#include "emu_rt.hpp"')
    s = _sub(r"__device__ __forceinline__ void dma16\(const void\* src, " + re.escape(AS3) + r" void\* lds\) \{.*?\n\}",
             "inline void dma16(const void* src, void* lds) { emu_dma((const char*)src, lds); }", s, "dma16")
    s = _sub(r"__device__ __forceinline__ void dma16s\(const void\* base, uint32_t off, " + re.escape(AS3)
             + r" void\* lds\) \{.*?\n\}",
             "inline void dma16s(const void* base, uint32_t off, void* lds) {\n"
             "    emu_dma(emu_readfirstlane((const char*)base) + off, lds);\n}", s, "dma16s")
    s = _sub(r"__device__ __forceinline__ void dma16_nt\(const void\* src, " + re.escape(AS3) + r" void\* lds\) \{.*?\n\}",
             "inline void dma16_nt(const void* src, void* lds) { emu_dma((const char*)src, lds); }", s, "dma16_nt")
    if "asm" in s:
        raise RuntimeError("inline assembly left in common.hpp")
    s = s.replace("namespace silvann {", """namespace silvann {
// a direct-to-LDS load: lane l's 16 bytes land at (the wave's first lane's lds) + 16·l (M0 is wave-uniform)
inline void emu_dma(const char* src, void* lds) {
    emu::dma_issue(src, (char*)emu_readfirstlane(lds) + 16 * emu::tl_lane);
}""", 1)
    s += """
namespace silvann {
inline hipStream_t stream() { return nullptr; }
inline int emu_refused = 0;
inline void check_launch(const char*) {}
inline void prof_begin(int) {}
inline void prof_end(int) {}
inline void refuse(const char* what) { std::fprintf(stderr, "refused: %s\\n", what); emu_refused = 1; }
// the deferral state of library.hip (not built here): on unless SILVANN_GFX950_DEFER=0
inline Deferred& deferred() { static Deferred d; return d; }
inline bool defer_enabled() {
    const char* e = std::getenv("SILVANN_GFX950_DEFER");
    return !(e && std::strcmp(e, "0") == 0);
}
}
"""
    return s


def _split_top(text: str) -> list[str]:
    """`text` split at its commas outside any brackets."""
    parts, depth, cur = [], 0, ""
    for ch in text:
        if ch in "([{<":
            depth += 1
        elif ch in ")]}>":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append(cur.strip())
            cur = ""
        else:
            cur += ch
    parts.append(cur.strip())
    return parts


def _launches(s: str) -> str:
    """`kernel<<<grid, block, lds, stream>>>(args);` -> `emu::launch(grid, block, [&]{ kernel(args); });` (the
    dynamic LDS size is dropped: dynamic LDS is a static of the most a workgroup may ask for)."""
    out, i = [], 0
    while True:
        j = s.find("<<<", i)
        if j < 0:
            out.append(s[i:])
            return "".join(out)
        # the kernel name (with template arguments) ends at j; find where it starts
        k, depth = j, 0
        while k > 0:
            ch = s[k - 1]
            if ch == ">":
                depth += 1
            elif ch == "<":
                depth -= 1
            elif depth == 0 and not (ch.isalnum() or ch in "_:"):
                break
            k -= 1
        e = s.index(">>>", j)
        cfg = _split_top(s[j + 3:e])
        if s[e + 3] != "(":
            raise RuntimeError("launch without arguments")
        depth, m = 0, e + 3
        while True:
            if s[m] == "(":
                depth += 1
            elif s[m] == ")":
                depth -= 1
                if depth == 0:
                    break
            m += 1
        out.append(s[i:k])
        name = " ".join(s[k:j].split())
        out.append(f"emu::launch({cfg[0]}, {cfg[1]}, [&]{{ {s[k:j]}{s[e + 3:m + 1]}; }}, \"{name}\")")
        i = m + 1


def kernel(name: str) -> str:
    s = (CSRC / name).read_text()
    s = s.replace('#include "common.hpp"', '#include "common_emu.hpp"')
    s = re.sub(r'#include "\.\./\.\./include/([^"]+)"', lambda m: f'#include "{INCLUDE / m.group(1)}"', s)
    s = s.replace(AS3, "")
    s = re.sub(r"__attribute__\(\(amdgpu_waves_per_eu\([^)]*\)\)\)", "", s)
    # dynamic LDS: the most a workgroup may ask for, as a static (one workgroup runs at a time)
    s = re.sub(r"extern __shared__ (\w+) (\w+)\[\];", r"static \1 \2[65536 / sizeof(\1)];", s)
    s = _sub(r"(__device__ __forceinline__ uint32_t scalar_load\(const uint32_t\* p\) \{).*?\n\}",
             r"\1 return *emu_readfirstlane(p); }", s, "scalar_load", required=False)
    s = _sub(r"(__device__ __forceinline__ void scale_acc\(float& x, float c\) \{).*?\n\}", r"\1 x *= c; }", s,
             "scale_acc", required=False)
    s = _sub(r"(__device__ __forceinline__ void dma16s_gap\(const void\* base, uint32_t off, lds_ptr lds\) \{).*?\n\}",
             r"\1 dma16s(base, off, lds); }", s, "dma16s_gap", required=False)
    s = _launches(s)
    left = [ln for ln in s.splitlines() if re.search(r"\basm\b", ln) or "<<<" in ln]
    if left:
        raise RuntimeError(f"{name}: left for the emulation to handle: {left[:3]}")
    return s


def write(out: Path, sources: list[str]) -> list[Path]:
    out.mkdir(parents=True, exist_ok=True)
    (out / "common_emu.hpp").write_text(common())
    (out / "emu_rt.hpp").write_text((HERE / "emu_rt.hpp").read_text())
    files = []
    for name in sources:
        f = out / (Path(name).stem + "_emu.cpp")
        f.write_text(kernel(name))
        files.append(f)
    return files
