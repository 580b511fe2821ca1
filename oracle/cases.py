"""Seeded synthetic inputs for the BASELINE configurations (test infrastructure only).

Recipe (common to all configs): K/V ~ N(0, 1) rounded to bf16 with 4 seeded
outlier channels scaled x8; q ~ N(0, 1) bf16; R = diag(s) H / sqrt(D) with a
seeded random sign vector s (gen_rotations.py:93-100 builds the normalised H);
128-token pages in randomly permuted block tables.

``make_case`` restates the fixture of delivery/probe_streaming.py:31-81 (history
written straight into the packed cache in rotated space, optional sink/recent
staging window) with its own NumPy generator.
"""
from __future__ import annotations

import math

import numpy as np

from . import fmt
from .store import store_ref

BASE_SEED = 20261201


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def hadamard(d: int) -> np.ndarray:
    """Normalised Sylvester Hadamard matrix (gen_rotations.py:93-100), float64."""
    if d < 1 or d & (d - 1):
        raise ValueError("Hadamard size must be a power of two")
    h = np.ones((1, 1))
    while h.shape[0] < d:
        h = np.block([[h, h], [h, -h]])
    return h / math.sqrt(d)


def hadamard_rotation(d: int, seed: int) -> np.ndarray:
    s = np.where(rng(seed).random(d) < 0.5, -1.0, 1.0)
    return (s[:, None] * hadamard(d)).astype(np.float32)


def qr_rotation(d: int, seed: int) -> np.ndarray:
    q, r = np.linalg.qr(rng(seed).standard_normal((d, d)))
    return (q * np.sign(np.diag(r))).astype(np.float32)


def kv_outliers(n: int, hk: int, d: int, seed: int, outliers: int = 4, factor: float = 8.0):
    g = rng(seed)
    x = g.standard_normal((n, hk, d)).astype(np.float32)
    ch = g.permutation(d)[:outliers]
    x[..., ch] *= factor
    return fmt.bf16_round(x)


def bf16_normal(shape, seed: int) -> np.ndarray:
    return fmt.bf16_round(rng(seed).standard_normal(shape).astype(np.float32))


def empty_caches(num_blocks: int, bs: int, hk: int, d: int, legacy: bool = False):
    width = 2 * d if legacy else d
    return (np.zeros((num_blocks, bs, hk, width), np.uint8),
            np.zeros((num_blocks, bs, hk, width), np.uint8))


def make_case(prefixes, lengths, *, hk=1, group=6, d=256, bs=128, window=True, fresh=True,
              seed=117, sink=128, recent=256, legacy=False, key_ramp=0.0, v_gain=1.0):
    """probe_streaming.py:31-81: packed history + optional staging + current chunk.

    Returns dict(q, k, v, k8, v8, bt, qsl, seqs, scale, stage).  All floats are
    float32 arrays on the bf16 grid; stage = (stage_k, stage_v, owner) or None.
    key_ramp > 0 scales history key t by 1 + key_ramp * t / 1024 (a rising score
    maximum along the history, for the attention kernels' rescale paths).
    v_gain scales every value vector (history and current chunk), e.g. 1e3 for V
    scales far above the unit range.
    """
    g = rng(seed)
    hq = hk * group
    seqs = [p + n if fresh else p for p, n in zip(prefixes, lengths)]
    width = max(16, math.ceil(max(seqs, default=0) / bs / 16) * 16)
    blocks = len(seqs) * width
    bt = g.permutation(blocks).reshape(len(seqs), width).astype(np.int32)
    k8, v8 = empty_caches(blocks, bs, hk, d, legacy)
    qsl = [0]
    slots = []
    for req, (prefix, n) in enumerate(zip(prefixes, lengths)):
        pos = np.arange(prefix)
        slots.append(bt[req, pos // bs].astype(np.int64) * bs + pos % bs)
        qsl.append(qsl[-1] + n)
    total = sum(prefixes)
    old_k = g.standard_normal((total, hk, d)).astype(np.float32)
    if key_ramp:
        # history keys grow with their position (x (1 + key_ramp * pos / 1024)), so a
        # row's score maximum keeps rising along the history
        pos = np.concatenate([np.arange(p_) for p_ in prefixes]) if total else np.zeros(0)
        old_k *= (1.0 + key_ramp * pos / 1024.0).astype(np.float32)[:, None, None]
    old_k = fmt.bf16_round(old_k)
    old_v = fmt.bf16_round(g.standard_normal((total, hk, d)).astype(np.float32) * np.float32(v_gain))
    store_ref(old_k, old_v, k8, v8, np.concatenate(slots) if slots else np.zeros(0, np.int64))
    q = fmt.bf16_round(g.standard_normal((qsl[-1], hq, d)).astype(np.float32))
    k = v = None
    if fresh:
        k = fmt.bf16_round(g.standard_normal((qsl[-1], hk, d)).astype(np.float32))
        v = fmt.bf16_round(g.standard_normal((qsl[-1], hk, d)).astype(np.float32) * np.float32(v_gain))
    stage = None
    if window:
        rows = max(math.ceil(8192 / bs), 4)
        sk = np.zeros((rows, bs, hk, d), np.float32)
        sv = np.zeros_like(sk)
        owner = np.full((rows, bs), -1, np.int64)
        off = 0
        for req, prefix in enumerate(prefixes):
            retained = list(range(min(sink, prefix))) + list(range(max(sink, prefix - recent), prefix))
            for pos in retained:
                block = int(bt[req, pos // bs])
                row, col = block % rows, pos % bs
                owner[row, col] = block
                sk[row, col], sv[row, col] = old_k[off + pos], old_v[off + pos]
            off += prefix
        stage = (sk, sv, owner)
    return dict(q=q, k=k, v=v, k8=k8, v8=v8, bt=bt, qsl=qsl, seqs=seqs, scale=d ** -0.5,
                stage=stage)
