"""SiLVANN attention for MI355X (gfx950): the nn attention doors and the fused paged decode / causal prefill.

`silvann_amd.doors` is the C ABI with torch tensors for device memory; `silvann_amd.verbs` is the host side
of the reference's attention verbs (their operand checks and door sequences) over those doors.
"""
from ._lib import LibraryMissing, lib  # noqa: F401
from . import doors  # noqa: F401
from . import verbs  # noqa: F401

FAULT_BOUNDS = 0x4E50424E     # "NPBN" packages/nn/contracts/objects/primitives.cuh:5
FAULT_NO_DEVICE = 0x4E504E44  # "NPND" primitives.cuh:6
FAULT_OVERFLOW = 0x4E504F56   # "NPOV" primitives.cuh:57
