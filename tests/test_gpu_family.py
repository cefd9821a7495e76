"""libsilvann_gfx950_family.so on gfx950, driven only through the table `silvann_silicon_family_get(9)` answers, as the
engine drives a family (no torch memory): the sys doors (packages/sys/contracts/abi/gpu.cuh:47-77) — binding, card
memory, mapped host RAM, side channels and marks, file reads — and the reference's decode verb through the nn table
(attention_scores then attention_mix, rows 25-26) against the oracle; a row this family does not run makes the next
compute_completed answer false, once.
"""
import ctypes as C

import numpy as np
import pytest

from oracle.oracle import inputs
from silvann_amd._lib import SIGNATURES
from tests.conftest import parity
from tests.test_family import FAMILY_PATH, NN_ROWS, SYS_NAMES, SYS_ROWS, FamilyTable, _doors

pytestmark = pytest.mark.gpu

_b, _u32, _p, _sz = C.c_bool, C.c_uint32, C.c_void_p, C.c_size_t
SYS_TYPES = {
    "memory_allocate": (_b, C.POINTER(_p), _sz), "memory_free": (None, _p), "memory_zerofill": (_b, _p, _sz),
    "memory_read": (_b, _p, _p, _sz), "memory_write": (_b, _p, _p, _sz), "compute_completed": (_b,),
    "side_open": (_b, C.POINTER(_p)), "side_close": (None, _p), "side_memory_read": (_b, _p, _p, _sz, _p),
    "side_memory_write": (_b, _p, _p, _sz, _p), "memory_allocate_host_ram_mapped": (_b, C.POINTER(_p), C.POINTER(_p), _sz),
    "memory_free_host_ram": (None, _p), "device_count": (_u32,), "bind_device": (_u32, _u32), "bound_device": (_u32,),
    "file_open": (_b, C.c_char_p, C.POINTER(C.c_uint64)), "file_close": (None, C.c_uint64),
    "file_read": (_b, C.c_uint64, C.c_uint64, C.c_uint64, _p), "peer_access": (_b, _u32),
    "mark_open": (_b, C.POINTER(_p)), "mark_close": (None, _p), "mark_record": (_b, _p), "mark_wait": (_b, _p),
    "side_memory_write_queued": (_b, _p, _p, _sz, _p), "side_memory_read_queued": (_b, _p, _p, _sz, _p),
    "side_mark_record": (_b, _p, _p), "mark_reached": (_b, _p),
}


class Family:
    def __init__(self):
        get = C.CDLL(str(FAMILY_PATH)).silvann_silicon_family_get
        get.restype, get.argtypes = _p, [_u32]
        t = FamilyTable.from_address(get(9))
        _, sys_rows = _doors(t.package_doors[0], SYS_ROWS)
        _, self.nn_rows = _doors(t.package_doors[1], NN_ROWS)
        self._keep = []
        for name, addr in zip(SYS_NAMES, sys_rows):
            if name in SYS_TYPES:
                f = C.CFUNCTYPE(*SYS_TYPES[name])(addr)
                self._keep.append(f)
                setattr(self, name, f)

    def nn(self, row, symbol):
        return C.CFUNCTYPE(None, *SIGNATURES[symbol])(self.nn_rows[row])

    def alloc(self, nbytes):
        at = _p()
        assert self.memory_allocate(C.byref(at), nbytes)
        return at.value

    def put(self, a):
        a = np.ascontiguousarray(a)
        at = self.alloc(a.nbytes)
        assert self.memory_write(at, a.ctypes.data, a.nbytes)
        return at

    def get(self, at, n, dtype):
        out = np.empty(n, dtype)
        assert self.memory_read(out.ctypes.data, at, out.nbytes)
        return out


@pytest.fixture(scope="module")
def fam():
    f = Family()
    assert f.device_count() >= 1
    assert f.bind_device(0) == 1 and f.bound_device() == 0
    assert f.bind_device(f.device_count()) == 0
    assert f.compute_completed()
    return f


def test_memory_doors(fam):
    print("case: family memory doors", flush=True)
    a = np.arange(1 << 20, dtype=np.uint32)
    at = fam.put(a)
    assert np.array_equal(fam.get(at, a.size, np.uint32), a)
    assert fam.memory_zerofill(at + 4096, 8192)
    back = fam.get(at, a.size, np.uint32)
    assert not back[1024:3072].any() and np.array_equal(back[:1024], a[:1024]) and np.array_equal(back[3072:], a[3072:])
    host, card = _p(), _p()
    assert fam.memory_allocate_host_ram_mapped(C.byref(host), C.byref(card), 4096)
    C.memset(host.value, 0x5A, 4096)
    assert fam.memory_write(at, host.value, 4096)   # mapped host RAM is ordinary host memory to a copy
    assert np.all(fam.get(at, 1024, np.uint8)[:1024] == 0x5A)
    fam.memory_free_host_ram(host.value)
    fam.memory_free(at)
    assert fam.compute_completed()


def test_side_channel_and_marks(fam):
    print("case: family side channel and marks", flush=True)
    ch, mark = _p(), _p()
    assert fam.side_open(C.byref(ch)) and fam.mark_open(C.byref(mark))
    a = np.random.default_rng(1).integers(0, 1 << 31, 1 << 18, dtype=np.int64)
    at = fam.alloc(a.nbytes)
    assert fam.side_memory_write(at, a.ctypes.data, a.nbytes, ch.value)
    out = np.zeros_like(a)
    assert fam.side_memory_read(out.ctypes.data, at, a.nbytes, ch.value)
    assert np.array_equal(out, a)
    out[:] = 0
    b = a[::-1].copy()
    assert fam.side_memory_write_queued(at, b.ctypes.data, b.nbytes, ch.value)
    assert fam.side_memory_read_queued(out.ctypes.data, at, b.nbytes, ch.value)
    assert fam.side_mark_record(mark.value, ch.value) and fam.mark_reached(mark.value)
    assert np.array_equal(out, b)
    assert fam.mark_record(mark.value) and fam.mark_wait(mark.value) and fam.mark_reached(mark.value)
    fam.mark_close(mark.value)
    fam.side_close(ch.value)
    fam.memory_free(at)
    assert fam.peer_access(0)
    assert fam.compute_completed()


def test_file_read(fam, tmp_path):
    print("case: family file_read", flush=True)
    a = np.random.default_rng(2).integers(0, 255, 3 << 20, dtype=np.uint8)
    path = tmp_path / "blob"
    path.write_bytes(a.tobytes())
    h = C.c_uint64()
    assert fam.file_open(str(path).encode(), C.byref(h))
    at = fam.alloc(1 << 20)
    assert fam.file_read(h.value, 12345, 1 << 20, at)
    assert np.array_equal(fam.get(at, 1 << 20, np.uint8), a[12345:12345 + (1 << 20)])
    assert not fam.file_read(h.value, len(a) - 10, 100, at)   # past the end
    fam.file_close(h.value)
    fam.memory_free(at)


@pytest.mark.parametrize("qh,kvh,hd,L", [(16, 2, 256, 2048), (8, 8, 128, 777)])
def test_decode_verb_through_the_family(fam, oracle, qh, kvh, hd, L):
    print(f"case: family decode verb qh{qh} kvh{kvh} hd{hd} L{L}", flush=True)
    q, k, v = inputs(qh + L, (qh * hd,), (L * kvh * hd,), (L * kvh * hd,))
    qd, kd, vd = fam.put(q), fam.put(k), fam.put(v)
    p, o, over = fam.alloc(4 * qh * L), fam.alloc(2 * qh * hd), fam.alloc(4)
    assert fam.memory_zerofill(over, 4)
    fam.nn(25, "silvann_gfx950_attention_scores")(p, qd, kd, qh, kvh, hd, L)
    fam.nn(26, "silvann_gfx950_attention_mix")(o, p, vd, qh, kvh, hd, L, over)
    assert fam.compute_completed()
    want_p = oracle.scores(q, k, qh, kvh, hd, L)
    want_o, _ = oracle.mix(want_p, v, qh, kvh, hd, L)
    parity(fam.get(o, qh * hd, np.float16), want_o)
    assert fam.get(over, 1, np.int32)[0] == 0
    for at in (qd, kd, vd, p, o, over):
        fam.memory_free(at)


def test_unanswered_row_fails_the_next_completion(fam):
    print("case: family unanswered nn row", flush=True)
    C.CFUNCTYPE(None)(fam.nn_rows[0])()
    assert fam.compute_completed() is False
    assert fam.compute_completed() is True
