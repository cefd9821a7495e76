"""The instruction stream of this library's own gfx950 build (hipcc -S of prefill.hip, device side): properties the
source states but the compiler decides.

causal_mfma's head_dim-256 steady loop — one block a key tile, 32 MFMAs and one barrier — must be lowered as
wave-uniform control flow: its trip count in scalar registers, its back-edge an SCC branch, and no instruction in
it writing EXEC. Its bound comes from the wave index (threadIdx.x / 64), which the compiler's divergence analysis
does not know to be uniform within a wave; left to itself it lowered the loop (and the tail after it) with EXEC
masks and the tile cursor in vector registers, a form under which an earlier build faulted a GPU. The bound goes
through readfirstlane for that reason, and this test keeps it so. causal_duo's pair loop is held to the same form
(its tile parity comes from the wave index through readfirstlane); removing that readfirstlane fails the test.
"""
import os
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "silvann_amd" / "csrc" / "prefill.hip"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("no hipcc")
    from silvann_amd.build import FLAGS
    out = tmp_path_factory.mktemp("isa") / "prefill.s"
    flags = [f for f in FLAGS if f not in ("-fPIC",)]
    subprocess.run([HIPCC, *flags, "--cuda-device-only", "-S", str(SRC), "-o", str(out)], check=True,
                   capture_output=True, timeout=600)
    return out.read_text()


def kernels(text):
    """{symbol: its lines}."""
    cur, out = None, {}
    for line in text.split("\n"):
        m = re.match(r"^(_Z\S+):", line)
        if m:
            cur = m.group(1)
            out[cur] = []
            continue
        if line.startswith(".Lfunc_end"):
            cur = None
        if cur:
            out[cur].append(line)
    return out


def outer_loops(lines):
    """{header block: the lines of every block LLVM annotates as in that depth-1 loop}."""
    loops, cur = {}, None
    for line in lines:
        m = re.match(r"^(?:\.LBB(\w+)|; %bb\.\d+):(.*)$", line)
        if m:
            note = m.group(2)
            h = re.search(r"Loop: Header=BB(\w+) Depth=1", note)
            if "Loop Header: Depth=1" in note and m.group(1):
                cur = "BB" + m.group(1)
            elif h:
                cur = "BB" + h.group(1)
            else:
                cur = None
            continue
        if cur:
            loops.setdefault(cur, []).append(line)
    return loops


def writes_exec(line):
    s = line.strip()
    return bool(re.match(r"s_\w+_saveexec_b64\b", s) or re.match(r"s_\w+\s+exec\b", s))


def test_steady_loop_is_wave_uniform(asm):
    ks = {k: v for k, v in kernels(asm).items() if "causal_mfmaILi256E" in k}
    assert len(ks) == 8, sorted(ks)   # PAIRED x PTL x RES
    for name, lines in ks.items():
        steady = []
        for header, body in outer_loops(lines).items():
            mfma = sum("v_mfma" in x for x in body)
            barriers = sum(re.match(r"\s+s_barrier\b", x) is not None for x in body)
            if mfma == 32 and barriers == 1 and any("sched_barrier" in x for x in body):
                steady.append((header, body))
        assert steady, f"{name}: no steady loop (32 MFMAs, one barrier, pinned groups) found"
        for header, body in steady:
            bad = [x.strip() for x in body if writes_exec(x)]
            assert not bad, f"{name} loop {header} writes EXEC: {bad[:4]}"
            assert not any(re.match(r"\s+s_cbranch_exec", x) and ".LBB" + header[2:] in x for x in body), \
                f"{name} loop {header} closes on an EXEC branch"


def test_duo_pair_loop_is_wave_uniform(asm):
    """causal_duo's loop over pairs of key tiles (a barrier, the wave's tile's head_dim / 8 MFMAs) branches only on
    wave-uniform values — the tile parity goes through readfirstlane, the diagonal test and the rescale vote are
    scalar — so it must not write EXEC either."""
    ks = {k: v for k, v in kernels(asm).items() if "causal_duoI" in k}
    assert len(ks) == 16, sorted(ks)   # head_dim 128, 256 x PAIRED x PTL x RES
    for name, lines in ks.items():
        mfmas = 32 if "causal_duoILi256E" in name else 16
        loops = [(h, b) for h, b in outer_loops(lines).items()
                 if sum("v_mfma" in x for x in b) == mfmas and sum(re.match(r"\s+s_barrier\b", x) is not None
                                                              for x in b) == 1]
        assert loops, f"{name}: no pair loop ({mfmas} MFMAs, one barrier) found"
        for header, body in loops:
            bad = [x.strip() for x in body if writes_exec(x)]
            assert not bad, f"{name} loop {header} writes EXEC: {bad[:4]}"
