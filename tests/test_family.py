"""libsilvann_gfx950_family.so, this library as a SiLVANN silicon family of its own, on the CPU (no GPU calls).

- It exports exactly one name, `silvann_silicon_family_get`, and none of the `<family>__<door>` names the reference's
  build check rejects (engine/scripts/build_silicon_families.sh:69-79).
- The entry answers a table for ABI version 9 and nothing for another (silicon_family.cuh:33, entry.cuh:69-81).
- The table passes every check the engine's offer makes (packages/sys/cpu/silicon/silicon_family.cuh:48-59) and has
  the shape the engine reads: seven package tables, sys with its 31 doors, nn with the reference's 137 rows and the
  five appended ones, the model packages size-only.
- The nn rows this library runs point at the attention library's own doors (the same code as
  silvann_gfx950_attention_install puts in a table); every other row points at one refusing function.
- The sys doors that touch no card answer as the contract says on a machine with no gfx950 card.
"""
import ctypes
import re
import subprocess

import pytest

from silvann_amd._lib import LIB_PATH

FAMILY_PATH = LIB_PATH.parent / "libsilvann_gfx950_family.so"
SYS_ROWS, NN_ROWS, PACKAGES = 31, 142, 7
SYS_NAMES = ["memory_allocate", "memory_free", "memory_zerofill", "memory_read", "memory_write", "compute_completed",
             "side_open", "side_close", "side_memory_read", "side_memory_write", "memory_allocate_host_ram_mapped",
             "memory_free_host_ram", "device_count", "bind_device", "bound_device", "memory_register_host",
             "memory_unregister_host", "file_open", "file_close", "file_read", "memory_map_file", "memory_prefetch",
             "peer_access", "mark_open", "mark_close", "mark_record", "mark_wait", "side_memory_write_queued",
             "side_memory_read_queued", "side_mark_record", "mark_reached"]


class FamilyTable(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("size", ctypes.c_uint32), ("id", ctypes.c_uint32),
                ("package_count", ctypes.c_uint32), ("name", ctypes.c_char_p),
                ("package_doors", ctypes.POINTER(ctypes.c_void_p))]


def _doors(addr, rows):
    size = ctypes.c_uint32.from_address(addr).value
    return size, [ctypes.c_void_p.from_address(addr + 8 + 8 * i).value for i in range(rows)]


@pytest.fixture(scope="module")
def family():
    if not FAMILY_PATH.exists():
        pytest.skip("the family library is not built")
    lib = ctypes.CDLL(str(FAMILY_PATH))
    get = lib.silvann_silicon_family_get
    get.restype, get.argtypes = ctypes.c_void_p, [ctypes.c_uint32]
    return get


def test_exports_only_the_entry():
    out = subprocess.run(["nm", "-D", "--defined-only", str(FAMILY_PATH)], capture_output=True, text=True,
                         check=True).stdout
    names = [line.split()[-1] for line in out.splitlines() if line.strip()]
    assert names == ["silvann_silicon_family_get"]
    assert not [n for n in names if re.match(r"^[a-z][a-z0-9_]*__", n)]


def test_answers_version_nine_only(family):
    assert family(9)
    assert family(8) is None and family(10) is None and family(0) is None
    assert family(9) == family(9)   # one table for the process


def test_table_passes_the_engines_offer(family):
    t = FamilyTable.from_address(family(9))
    assert (t.abi_version, t.size, t.id, t.package_count) == (9, ctypes.sizeof(FamilyTable), 275, PACKAGES)
    assert t.size >= 32 and t.id < 1024
    assert t.name == b"amd_gfx950_attention"
    size, rows = _doors(t.package_doors[0], SYS_ROWS)
    assert size == 8 + 8 * SYS_ROWS
    assert all(rows) and len(set(rows)) == SYS_ROWS
    for i in range(2, PACKAGES):
        assert ctypes.c_uint32.from_address(t.package_doors[i]).value == 4


def test_nn_rows_are_this_librarys(family):
    from silvann_amd._lib import lib as attention
    t = FamilyTable.from_address(family(9))
    size, rows = _doors(t.package_doors[1], NN_ROWS)
    assert size == 8 + 8 * NN_ROWS
    assert all(rows)
    # the attention library's own table, filled the same way, has its rows where the family has non-refusing ones
    table = (ctypes.c_uint64 * (1 + NN_ROWS))()
    ctypes.c_uint32.from_buffer(table).value = 8 + 8 * NN_ROWS
    installed = attention().silvann_gfx950_attention_install(ctypes.byref(table))
    mine = {i for i in range(NN_ROWS) if table[1 + i]}
    assert len(mine) == installed == 28
    refusing = {rows[i] for i in range(NN_ROWS) if i not in mine}
    assert len(refusing) == 1
    assert all(rows[i] not in refusing for i in mine)
    assert len({rows[i] for i in mine}) == len(mine)
    assert {137, 138, 139, 140, 141, 46, 107} <= mine


def test_card_free_sys_doors(family, tmp_path):
    t = FamilyTable.from_address(family(9))
    _, rows = _doors(t.package_doors[0], SYS_ROWS)
    door = dict(zip(SYS_NAMES, rows))
    fn = lambda name, res, *args: ctypes.CFUNCTYPE(res, *args)(door[name])  # noqa: E731
    register = fn("memory_register_host", ctypes.c_bool, ctypes.c_void_p, ctypes.c_size_t,
                  ctypes.POINTER(ctypes.c_void_p))
    card = ctypes.c_void_p()
    buf = ctypes.create_string_buffer(64)
    assert register(ctypes.addressof(buf), 64, ctypes.byref(card)) is False
    assert fn("memory_map_file", ctypes.c_bool, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64,
              ctypes.c_uint64)(None, 0, 0, 0) is False
    assert fn("memory_prefetch", ctypes.c_bool, ctypes.c_void_p, ctypes.c_size_t)(None, 0) is True
    opened = fn("file_open", ctypes.c_bool, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64))
    handle = ctypes.c_uint64()
    assert opened(str(tmp_path / "absent").encode(), ctypes.byref(handle)) is False
    (tmp_path / "there").write_bytes(b"x" * 10)
    assert opened(None, ctypes.byref(handle)) is False
    assert opened(str(tmp_path / "there").encode(), ctypes.byref(handle)) is True
    assert handle.value != 0   # 0 is never a file
    fn("file_close", None, ctypes.c_uint64)(handle.value)
    fn("file_close", None, ctypes.c_uint64)(0)   # closes nothing
    read = fn("file_read", ctypes.c_bool, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p)
    assert read(0, 0, 16, ctypes.addressof(buf)) is False   # no file: refused before any copy
    import torch
    if not torch.cuda.is_available():
        assert fn("device_count", ctypes.c_uint32)() == 0
        assert fn("bind_device", ctypes.c_uint32, ctypes.c_uint32)(0) == 0
        assert fn("bound_device", ctypes.c_uint32)() == 0xFFFFFFFF
