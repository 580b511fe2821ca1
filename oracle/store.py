"""Write path restated in NumPy: rotate, clip, INT2 scatter, staging window.

Test infrastructure only.  Caches are uint8 arrays ``[num_blocks, block_size,
num_kv_heads, slot_bytes]`` exactly as the reference addresses them through
``cache.view(torch.uint8)`` (slot_bytes = D for int8 caches, 2*D for bf16).

Rotation.  The reference computes ``x.float() @ R`` with torch's CPU sgemm
(backend.py:131, :554), whose last bits depend on the BLAS blocking.  The
oracle pins the mathematically canonical value instead: the dot product
evaluated in float64 (products of two float32 values are exact there) and
rounded once to float32, which equals the correctly rounded result unless
the exact sum lies within ~2^-45 (relative) of a float32 rounding boundary.
``rotate_f32gemm`` reproduces the reference's own op for comparisons.
"""
from __future__ import annotations

import numpy as np

from . import fmt


# ------------------------------------------------------------------ rotation
def rotate(x, r) -> np.ndarray:
    """backend.py:131 ``x.float() @ R`` as the correctly rounded fp32 result."""
    x64 = np.asarray(x, np.float32).astype(np.float64)
    return (x64 @ np.asarray(r, np.float32).astype(np.float64)).astype(np.float32)


def rotate_f32gemm(x, r) -> np.ndarray:
    """The reference's literal op (torch CPU fp32 matmul), for comparison only."""
    import torch

    return (torch.from_numpy(np.ascontiguousarray(x, np.float32))
            @ torch.from_numpy(np.ascontiguousarray(r, np.float32))).numpy()


def clip(x_rot, ratio: float) -> np.ndarray:
    """backend.py:132-145: clamp to the idx-th smallest |x| per vector."""
    x_rot = np.asarray(x_rot, np.float32)
    if ratio <= 0.0:
        return x_rot
    d = x_rot.shape[-1]
    idx = min(int(ratio * d), d - 1)
    thr = np.sort(np.abs(x_rot), axis=-1)[..., idx:idx + 1]
    return np.clip(x_rot, -thr, thr).astype(np.float32)


# ------------------------------------------------------------------ INT2 store
def slot_offsets(slots, bs: int, hk: int, cache) -> np.ndarray:
    """store_kernel.py:35-48: byte offsets [N, H] from the live cache strides."""
    st = np.array(cache.strides, np.int64)
    blk, off = slots // bs, slots % bs
    return (blk * st[0] + off * st[1])[:, None] + np.arange(hk) * st[2]


def store_ref(k_rot, v_rot, k8, v8, slot_mapping) -> None:
    """store_kernel.py:54-102.

    Negative slots are skipped; for repeated slots the last token wins
    (``index_put_`` applies writes in order).
    """
    k_rot, v_rot = np.asarray(k_rot, np.float32), np.asarray(v_rot, np.float32)
    slots = np.asarray(slot_mapping, np.int64)
    valid = slots >= 0
    slots, k_rot, v_rot = slots[valid], k_rot[valid], v_rot[valid]
    if slots.size == 0:
        return
    n, h, d = k_rot.shape
    fmt.check_d(d)
    bs = k8.shape[1]
    kp, ks, kz = fmt.quantize(k_rot)
    vp, vs, vz = fmt.quantize(v_rot)
    k_off = slot_offsets(slots, bs, h, k8)
    v_off = slot_offsets(slots, bs, h, v8)
    flat_k, flat_v = k8.reshape(-1), v8.reshape(-1)
    meta = np.zeros((n, h, fmt.META_BYTES), np.uint8)
    for i, val in enumerate((ks, kz, vs, vz)):
        lo, hi = fmt.f16_le(val)
        meta[..., 2 * i], meta[..., 2 * i + 1] = lo[..., 0], hi[..., 0]
    # Sequential index_put_ leaves the last writer of a repeated slot; keep
    # only that token so the vectorised assignment below has unique targets.
    _, last_rev = np.unique(slots[::-1], return_index=True)
    win = np.sort(n - 1 - last_rev)
    k_off, v_off = k_off[win], v_off[win]
    flat_k[k_off[..., None] + np.arange(fmt.META_BYTES)] = meta[win]
    flat_k[k_off[..., None] + fmt.K_IDX_OFF + np.arange(d // 4)] = kp[win]
    flat_v[v_off[..., None] + np.arange(d // 4)] = vp[win]


def dequant_split_ref(k8, v8, blocks, pos, hk: int, d: int):
    """store_kernel.py:105-133: gather + unpack -> fp32 [T, H, D] (rotated space)."""
    blocks, pos = np.asarray(blocks, np.int64), np.asarray(pos, np.int64)
    sk, sv = np.array(k8.strides, np.int64), np.array(v8.strides, np.int64)
    k_off = (blocks * sk[0] + pos * sk[1])[:, None] + np.arange(hk) * sk[2]
    v_off = (blocks * sv[0] + pos * sv[1])[:, None] + np.arange(hk) * sv[2]
    flat_k, flat_v = k8.reshape(-1), v8.reshape(-1)
    meta = flat_k[k_off[..., None] + np.arange(fmt.META_BYTES)]
    ks = fmt.f16_from_le(meta[..., 0:1], meta[..., 1:2])
    kz = fmt.f16_from_le(meta[..., 2:3], meta[..., 3:4])
    vs = fmt.f16_from_le(meta[..., 4:5], meta[..., 5:6])
    vz = fmt.f16_from_le(meta[..., 6:7], meta[..., 7:8])
    io = np.arange(d // 4)
    kp = flat_k[k_off[..., None] + fmt.K_IDX_OFF + io]
    vp = flat_v[v_off[..., None] + io]
    return fmt.dequant(kp, ks, kz, d), fmt.dequant(vp, vs, vz, d)


# ------------------------------------------------------------------ staging
class Staging:
    """backend.py:492-511: per-layer FP32 window arena and owner tags."""

    def __init__(self, bs: int, hk: int, d: int, sink_tokens: int, recent_tokens: int,
                 staging_tokens: int):
        self.bs = bs
        self.sink_eff = (sink_tokens // bs) * bs
        self.sink_pages = self.sink_eff // bs
        self.tail_pages = (recent_tokens + bs - 1) // bs + 1
        self.recent = recent_tokens
        self.rows = max((staging_tokens + bs - 1) // bs, self.sink_pages + self.tail_pages + 2)
        self.stage_k = np.zeros((self.rows, bs, hk, d), np.float32)
        self.stage_v = np.zeros_like(self.stage_k)
        self.owner = np.full((self.rows, bs), -1, np.int64)

    def seat(self, slots):
        slots = np.asarray(slots, np.int64)
        return (slots // self.bs % self.rows) * self.bs + slots % self.bs

    def invalidate(self, slot_mapping) -> None:
        """backend.py:169-176: a rewritten seat loses its unquantized copy."""
        slots = np.asarray(slot_mapping, np.int64)
        valid = slots[slots >= 0]
        self.owner[valid // self.bs % self.rows, valid % self.bs] = -1

    def keep_mask(self, n: int, qsl, seqs) -> np.ndarray:
        """backend.py:521-530: per-token window membership."""
        lengths = [max(0, min(e, n) - min(s, n)) for s, e in zip(qsl[:-1], qsl[1:])]
        req = np.repeat(np.arange(len(lengths)), lengths)
        if req.size != n:
            raise ValueError("query_start_loc does not cover num_actual_tokens")
        seq = np.asarray(seqs[:len(lengths)], np.int64)
        ends = np.asarray(qsl[1:], np.int64)
        pos = seq[req] - ends[req] + np.arange(n)
        return (pos >= seq[req] - self.recent) | (pos < self.sink_eff)

    def write(self, k_rot, v_rot, slot_mapping, qsl, seqs) -> None:
        """backend.py:513-555 given already rotated (unclipped) fp32 K/V.

        One writer per seat: the highest token index (stable sort, take last).
        """
        slots = np.asarray(slot_mapping, np.int64)
        n = slots.shape[0]
        if n == 0:
            return
        keep = self.keep_mask(n, qsl, seqs)
        valid = np.nonzero(slots >= 0)[0]
        seats = self.seat(slots[valid])
        order = np.argsort(seats, kind="stable")
        sorted_seats = seats[order]
        last = np.ones(sorted_seats.shape, bool)
        last[:-1] = sorted_seats[1:] != sorted_seats[:-1]
        selected = valid[order[last]]
        seats = sorted_seats[last]
        rows, offs = seats // self.bs, seats % self.bs
        self.owner[rows, offs] = np.where(keep[selected], slots[selected] // self.bs, -1)
        ret = keep[selected]
        if ret.any():
            sel = selected[ret]
            self.stage_k[rows[ret], offs[ret]] = np.asarray(k_rot, np.float32)[sel]
            self.stage_v[rows[ret], offs[ret]] = np.asarray(v_rot, np.float32)[sel]

    def arrays(self):
        return self.stage_k, self.stage_v, self.owner


def staging_order(seats, capacity: int) -> np.ndarray:
    """backend.py:88-93: stable argsort of seat ids."""
    seats = np.asarray(seats)
    keys = seats.astype(np.float32) if capacity <= 2 ** 24 else seats
    return np.argsort(keys, kind="stable")
