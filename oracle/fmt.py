"""INT2 slot contract, restated in NumPy (test infrastructure only).

Follows /root/reference/oscar_ascend/format.py.  All arithmetic is float32
with IEEE per-operation rounding, matching torch CPU elementwise kernels.
"""
from __future__ import annotations

import numpy as np

# format.py:19-38
BITS = 2
LEVELS = 4
VALUES_PER_BYTE = 4
META_BYTES = 8
PAD_BYTES = 24
K_IDX_OFF = 32
V_IDX_OFF = 96          # offset inside the logical 160-byte slot (= V slot offset 0)
SLOT_SIZE = 160
SCALE_FLOOR = np.float32(2.0 ** -14)


def check_d(d: int) -> None:
    """format.py:41-45."""
    if d % VALUES_PER_BYTE != 0:
        raise ValueError(f"D={d} must be a multiple of {VALUES_PER_BYTE}")
    if d // VALUES_PER_BYTE > V_IDX_OFF - META_BYTES - PAD_BYTES:
        raise ValueError(f"D={d} exceeds the slot capacity")


# ----------------------------------------------------------------- dtype helpers
def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def bf16_round(x) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest even) -> float32 (torch semantics)."""
    x = f32(x)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = rounded.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out = np.where(nan, np.float32(np.nan), out)
    return out.astype(np.float32)


def f16_round(x) -> np.ndarray:
    """float32 -> float16 (RNE) -> float32."""
    return f32(x).astype(np.float16).astype(np.float32)


def round_to(x, q_dtype: str) -> np.ndarray:
    """Round float32 values to the grid of the query dtype ("bf16", "f16" or "f32")."""
    if q_dtype == "bf16":
        return bf16_round(x)
    if q_dtype == "f16":
        return f16_round(x)
    if q_dtype == "f32":
        return f32(x)
    raise ValueError(f"unknown q_dtype {q_dtype!r}")


def bf16_bits(x) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of float32 values already on the bf16 grid."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------- quant / dequant
def vector_scales(x) -> tuple[np.ndarray, np.ndarray]:
    """format.py:51-64: per-vector (scale, zero), both already fp16-rounded."""
    x = f32(x)
    vmin = x.min(axis=-1, keepdims=True)
    vmax = x.max(axis=-1, keepdims=True)
    scale = (vmax - vmin) / np.float32(LEVELS - 1)
    scale = np.where(scale > SCALE_FLOOR, scale, SCALE_FLOOR).astype(np.float32)
    return f16_round(scale), f16_round(vmin)


def quantize_codes(x) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """format.py:78-83: integer codes clamp(floor((x - zero)/scale + 0.5), 0, 3)."""
    x = f32(x)
    scale, zero = vector_scales(x)
    with np.errstate(invalid="ignore"):
        t = np.floor((x - zero) / scale + np.float32(0.5)).astype(np.float32)
        t = np.clip(t, 0, LEVELS - 1)
        q = np.where(np.isnan(t), 0, t).astype(np.int32)
    return q, scale, zero


def pack(q) -> np.ndarray:
    """format.py:84-87: byte b holds q[4b+k] in bits 2k..2k+1."""
    q = np.asarray(q, dtype=np.int32)
    q4 = q.reshape(*q.shape[:-1], q.shape[-1] // VALUES_PER_BYTE, VALUES_PER_BYTE)
    return ((q4[..., 0] & 3) | (q4[..., 1] & 3) << 2 | (q4[..., 2] & 3) << 4
            | (q4[..., 3] & 3) << 6).astype(np.uint8)


def unpack(packed, d: int) -> np.ndarray:
    """format.py:99-110 (integer div/mod chain)."""
    p = np.asarray(packed, dtype=np.int32)
    parts = [(p // (LEVELS ** k)) % LEVELS for k in range(VALUES_PER_BYTE)]
    return np.stack(parts, axis=-1).reshape(*p.shape[:-1], d)


def quantize(x) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """format.py:67-88: x [..., D] fp32 -> (packed u8 [..., D/4], scale, zero)."""
    q, scale, zero = quantize_codes(x)
    return pack(q), scale, zero


def dequant(packed, scale, zero, d: int) -> np.ndarray:
    """format.py:91-96: q*scale + zero (two float32 ops, no fusion)."""
    q = unpack(packed, d).astype(np.float32)
    return (q * f32(scale)).astype(np.float32) + f32(zero)


def f16_le(x) -> tuple[np.ndarray, np.ndarray]:
    """format.py:113-119: fp16 bits as (lo, hi) bytes."""
    bits = f32(x).astype(np.float16).view(np.uint16)
    return (bits & 0xFF).astype(np.uint8), (bits >> 8).astype(np.uint8)


def f16_from_le(lo, hi) -> np.ndarray:
    """format.py:122-125."""
    bits = np.asarray(lo, np.uint16) | (np.asarray(hi, np.uint16) << 8)
    return bits.view(np.float16).astype(np.float32)


def make_slot_bytes(k_rot, v_rot) -> np.ndarray:
    """format.py:131-154: logical 160-byte slot [N, H, 160]."""
    k_rot, v_rot = f32(k_rot), f32(v_rot)
    n, h, d = k_rot.shape
    check_d(d)
    kp, ks, kz = quantize(k_rot)
    vp, vs, vz = quantize(v_rot)
    slot = np.zeros((n, h, SLOT_SIZE), np.uint8)
    for i, val in enumerate((ks, kz, vs, vz)):
        lo, hi = f16_le(val)
        slot[..., 2 * i] = lo[..., 0]
        slot[..., 2 * i + 1] = hi[..., 0]
    slot[..., K_IDX_OFF:K_IDX_OFF + d // 4] = kp
    slot[..., V_IDX_OFF:V_IDX_OFF + d // 4] = vp
    return slot


def parse_slot_bytes(slot, d: int) -> tuple[np.ndarray, np.ndarray]:
    """format.py:157-167."""
    slot = np.asarray(slot, np.uint8)
    ks = f16_from_le(slot[..., 0:1], slot[..., 1:2])
    kz = f16_from_le(slot[..., 2:3], slot[..., 3:4])
    vs = f16_from_le(slot[..., 4:5], slot[..., 5:6])
    vz = f16_from_le(slot[..., 6:7], slot[..., 7:8])
    k = dequant(slot[..., K_IDX_OFF:K_IDX_OFF + d // 4], ks, kz, d)
    v = dequant(slot[..., V_IDX_OFF:V_IDX_OFF + d // 4], vs, vz, d)
    return k, v
