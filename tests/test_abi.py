"""The C-ABI library: it loads and exports every entry point the header declares (no compute calls)."""
import ctypes
import re
import subprocess

import pytest

from silvann_amd import _lib


def test_header_declares_what_python_types():
    declared = set(_lib.header_functions())
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def test_library_exports_every_header_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    ours = {s for s in exported if s.startswith("silvann_")}
    declared = set(_lib.header_functions())
    assert declared <= exported, declared - exported
    assert ours == declared, ours - declared   # nothing of ours exported that the header does not declare


def test_library_loads_and_reports_version():
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    L = _lib.lib()
    assert L.silvann_gfx950_version().decode().startswith("gfx950")
    assert L.silvann_gfx950_launch_failed() == 0


def test_row_indices_match_reference_table():
    """SILVANN_GFX950_ROW_* are the rows' places in nn__CONTRACT__DOORS (gpu.cuh:93-230)."""
    from oracle.oracle import ROWS, NN_ROWS
    text = _lib.HEADER.read_text()
    rows = dict(re.findall(r"#define SILVANN_GFX950_ROW_(\w+) (\d+)u", text))
    for name, idx in ROWS.items():
        assert int(rows[name.upper()]) == idx, name
    assert int(re.search(r"#define SILVANN_GFX950_NN_ROWS (\d+)u", text).group(1)) == NN_ROWS


def test_row_indices_against_reference_source():
    """Counted from the reference's own door list where /root/reference is present."""
    from pathlib import Path
    from oracle.oracle import ROWS, NN_ROWS
    src = Path("/root/reference/engine/src/packages/nn/contracts/abi/gpu.cuh")
    if not src.exists():
        pytest.skip("reference sources absent")
    lines = src.read_text().splitlines()
    start = next(i for i, l in enumerate(lines) if l.startswith("#define nn__CONTRACT__DOORS"))
    names = []
    for l in lines[start + 1:]:
        m = re.match(r"\s*X\(PKG,\s*[\w ]+,\s*(\w+),", l)
        if m:
            names.append(m.group(1))
        if not l.rstrip().endswith("\\"):
            break
    assert len(names) == NN_ROWS
    for name, idx in ROWS.items():
        assert names[idx] == name
