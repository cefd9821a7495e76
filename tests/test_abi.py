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


def _fn_addr(L, name):
    return ctypes.cast(getattr(L, name), ctypes.c_void_p).value


def test_install_writes_the_rows_a_table_reaches():
    """silvann_gfx950_attention_install: the reference rows land at their indices in a table of the
    reference's size (the appended rows do not fit it and are not written); a table grown by two rows takes
    the first two of them, one grown by five all five; every other slot is left as it was; NULL answers 0."""
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    from oracle.oracle import ROWS, NN_ROWS
    L = _lib.lib()
    text = _lib.HEADER.read_text()
    rows = {int(i): n for n, i in re.findall(r"#define SILVANN_GFX950_ROW_(\w+) (\d+)u", text)}
    for nslots, expect in ((NN_ROWS, len(ROWS)), (NN_ROWS + 2, len(ROWS) + 2), (NN_ROWS + 5, len(ROWS) + 5)):
        buf = (ctypes.c_uint64 * (1 + nslots))()
        sentinel = 0x5A5A0000
        for i in range(nslots):
            buf[1 + i] = sentinel + i
        buf[0] = 8 + 8 * nslots   # uint32 size in bytes, then padding to the first pointer slot
        assert L.silvann_gfx950_attention_install(ctypes.addressof(buf)) == expect
        for i in range(nslots):
            if i in rows:
                assert buf[1 + i] == _fn_addr(L, "silvann_gfx950_" + rows[i].lower()), rows[i]
            else:
                assert buf[1 + i] == sentinel + i, i
    assert len([i for i in rows if i < NN_ROWS]) == len(ROWS) == 23
    assert L.silvann_gfx950_attention_install(None) == 0


def test_install_into_a_copy_of_the_reference_table(ref):
    """Over a copy of the x86_avx2 family's own nn table (oracle/_ref): our rows replace the family's,
    every other door pointer is the family's own."""
    L = _lib.lib()
    nn = ref.family.package_doors[1]
    size = ctypes.c_uint32.from_address(nn).value
    copy = (ctypes.c_uint8 * size)()
    ctypes.memmove(copy, nn, size)
    from oracle.oracle import ROWS
    assert L.silvann_gfx950_attention_install(ctypes.addressof(copy)) == len(ROWS)
    mine = (ctypes.c_uint64 * ((size - 8) // 8)).from_address(ctypes.addressof(copy) + 8)
    theirs = (ctypes.c_uint64 * ((size - 8) // 8)).from_address(nn + 8)
    text = _lib.HEADER.read_text()
    rows = {int(i): n for n, i in re.findall(r"#define SILVANN_GFX950_ROW_(\w+) (\d+)u", text)}
    for i in range((size - 8) // 8):
        if i in rows:
            assert mine[i] == _fn_addr(L, "silvann_gfx950_" + rows[i].lower())
        else:
            assert mine[i] == theirs[i] != 0
