"""What the compiler decided for each kernel of this library's own build (hipcc's kernel-resource-usage report,
which silvann_amd/build.py keeps beside each object): no kernel spills to scratch memory, none asks for more LDS
than a CU has, and the hot kernels keep the occupancy their designs count on — two waves a SIMD for the split-K
decode up to head_dim 256 and for the TurboQuant split (their streaming relies on the second wave), at least one
for the rest."""
import re
from pathlib import Path

import pytest

BUILD = Path(__file__).resolve().parent.parent / "silvann_amd" / "_build"
LDS_BYTES = 160 * 1024


def kernels():
    """{mangled name: {field: int}} over every object's report."""
    out = {}
    for f in sorted(BUILD.glob("*.resources.txt")):
        cur = None
        for line in f.read_text().splitlines():
            m = re.search(r"remark:\s+Function Name: (\S+)", line)
            if m:
                cur = out.setdefault(m.group(1), {})
                continue
            m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[bytes/(?:lane|block)\])?(?: \[waves/SIMD\])?: (\d+)", line)
            if m and cur is not None:
                cur[m.group(1).strip()] = int(m.group(2))
    return out


@pytest.fixture(scope="module")
def report():
    k = kernels()
    if not k:
        pytest.skip("no resource report: build with silvann_amd/build.py first")
    return k


def test_no_scratch_spills_and_lds_within_a_cu(report):
    for name, r in report.items():
        assert r.get("ScratchSize", 0) == 0 and r.get("VGPRs Spill", 0) == 0, (name, r)
        assert r.get("LDS Size", 0) <= LDS_BYTES, (name, r)


@pytest.mark.parametrize("pattern,waves", [
    (r"decode_splitILi(64|128|256)E", 2),   # the split-K decode up to head_dim 256
    (r"tq_splitILi", 2),                    # the TurboQuant split at every width
    (r"decode_splitILi512E", 1),
    (r"decode_latentI", 1),
    (r"causal_mfmaI", 1),
    (r"causal_pipeI", 1),
    (r"causal_duoI", 2),                    # two waves a SIMD is the design of causal_duo
])
def test_occupancy(report, pattern, waves):
    hits = {n: r for n, r in report.items() if re.search(pattern, n)}
    assert hits, pattern
    for name, r in hits.items():
        assert r.get("Occupancy", 0) >= waves, (name, r)
