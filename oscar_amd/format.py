"""OSCAR INT2 slot contract constants (oscar_ascend/format.py:19-46).

The packed caches keep the reference's byte layout so that the HIP kernels are a
drop-in: per token and KV head, the K slot holds [0:2] K scale, [2:4] K zero,
[4:6] V scale, [6:8] V zero (fp16 little endian), [8:32] untouched padding and
[32:32+D/4] the K codes; the V slot holds the V codes at [0:D/4].  Byte b of a
code run stores codes 4b+k in bits 2k..2k+1.
"""
from __future__ import annotations

BITS = 2
LEVELS = 4
VALUES_PER_BYTE = 4
D_DEFAULT = 256
META_BYTES = 8
PAD_BYTES = 24
K_IDX_OFF = 32
V_IDX_OFF = 96          # offset of the V codes in the logical 160-byte slot
SLOT_SIZE = 160
K_SLOT_BYTES = V_IDX_OFF
V_SLOT_BYTES = SLOT_SIZE - V_IDX_OFF
SCALE_FLOOR = 2.0 ** -14


def check_d(d: int) -> None:
    """format.py:41-45: D must pack into whole bytes and fit the 96-byte K slot."""
    if d % VALUES_PER_BYTE != 0:
        raise ValueError(f"D={d} must be a multiple of {VALUES_PER_BYTE} (INT2 packing)")
    if d // VALUES_PER_BYTE > K_SLOT_BYTES - META_BYTES - PAD_BYTES:
        raise ValueError(f"D={d} exceeds the slot capacity")
