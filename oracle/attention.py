"""Read path restated in NumPy: streaming attention over INT2 history.

Test infrastructure only.  Semantics follow
/root/reference/oscar_ascend/kernels/streaming_attention.py:103-196
(``_read_tile`` + ``streaming_attention_ref``) and the LSE merge of
/root/reference/oscar_ascend/kernels/slab_attention.py:341-356.

The reference's rounding points (streaming_attention.py:122-124,
prepare_kv.py:77): a history value is ``q_dtype(fp16(x))`` where ``x`` is the
fp32 dequantized code (``code*scale + zero``) or, when the seat's owner tag
equals the physical block, the fp32 staged value.  Current-chunk K/V are
used as given (already ``q_dtype``).  Scores, softmax, P@V and LSE are fp32 in
the reference; this oracle evaluates them in float64 (a stricter evaluation of
the same math) and returns float32.
"""
from __future__ import annotations

import numpy as np

from . import fmt
from .store import dequant_split_ref


def round_history(x, q_dtype: str) -> np.ndarray:
    """streaming_attention.py:124: ``x.half().to(dtype)`` (fp16 first, whatever q_dtype)."""
    return fmt.round_to(fmt.f16_round(x), q_dtype)


def read_history(k8, v8, bt_row, start: int, end: int, hk: int, d: int, stage, q_dtype: str):
    """streaming_attention.py:103-124 for positions [start, end) of one request."""
    bs = k8.shape[1]
    pos = np.arange(start, end, dtype=np.int64)
    blocks = np.asarray(bt_row, np.int64)[pos // bs]
    k, v = dequant_split_ref(k8, v8, blocks, pos % bs, hk, d)
    if stage is not None:
        sk, sv, owner = stage
        row, off = blocks % owner.shape[0], pos % bs
        hit = (owner[row, off] == blocks)[:, None, None]
        k = np.where(hit, sk[row, off], k)
        v = np.where(hit, sv[row, off], v)
    return round_history(k, q_dtype), round_history(v, q_dtype)


def attention_ref(q, k_new, v_new, k8, v8, bt, qsl, seqs, scale, stage=None, *,
                  d=None, q_dtype="bf16", rows=None):
    """streaming_attention.py:134-196 (exact softmax, float64 evaluation).

    q: [n, Hq, D] (values on the q_dtype grid), k_new/v_new: [n, Hk, D] or None.
    Query i of a request with ``n_q`` queries and length ``seq`` sees keys
    ``[0, seq - n_q + i + 1)``; rows that see nothing get out 0 and LSE -inf.
    ``rows`` (optional): the query token indices to evaluate; the others are left
    at out 0 / LSE -inf (a sampled check of long chunks).
    Returns (out_rot [n, Hq, D] f32, lse [n, Hq] f32).
    """
    q = np.asarray(q, np.float32)
    n, hq, dd = q.shape
    d = dd if d is None else d
    hk = k8.shape[2]
    group = hq // hk
    out = np.zeros((n, hq, d), np.float32)
    lse = np.full((n, hq), -np.inf, np.float32)
    wanted = None if rows is None else set(int(t) for t in rows)
    for r, (a, b, seq) in enumerate(zip(qsl[:-1], qsl[1:], seqs)):
        if b <= a:
            continue
        if wanted is not None and not any(a <= t < b for t in wanted):
            continue
        n_q = b - a
        prefix = seq - n_q if k_new is not None else seq
        k_hist, v_hist = read_history(k8, v8, bt[r], 0, max(prefix, 0), hk, d, stage, q_dtype)
        if k_new is not None:
            keys = np.concatenate([k_hist, np.asarray(k_new[a:b], np.float32)])
            vals = np.concatenate([v_hist, np.asarray(v_new[a:b], np.float32)])
        else:
            keys, vals = k_hist, v_hist
        keys64, vals64 = keys.astype(np.float64), vals.astype(np.float64)
        # query i sees the first seq - n_q + i + 1 keys; rows are evaluated in blocks,
        # each head group of a KV head at once: S = Q K^T over the block's longest
        # visible prefix, keys past a row's own prefix masked to -inf
        idx = [i for i in range(n_q) if seq - n_q + i + 1 > 0 and (wanted is None or a + i in wanted)]
        for c0 in range(0, len(idx), 128):
            blk = np.asarray(idx[c0:c0 + 128], np.int64)
            visible = seq - n_q + blk + 1
            vmax = int(visible.max())
            hidden = np.arange(vmax)[None, :] >= visible[:, None]
            for kv in range(hk):
                heads = slice(kv * group, (kv + 1) * group)
                qb = q[a + blk, heads].astype(np.float64)                  # [rows, group, D]
                s = (qb.reshape(-1, qb.shape[-1]) @ keys64[:vmax, kv].T).reshape(len(blk), group, vmax) * scale
                s[np.broadcast_to(hidden[:, None, :], s.shape)] = -np.inf
                m = s.max(-1, keepdims=True)
                with np.errstate(invalid="ignore"):
                    p = np.exp(s - m)
                tot = p.sum(-1, keepdims=True)
                o = (p.reshape(-1, vmax) @ vals64[:vmax, kv]).reshape(len(blk), group, -1) / tot
                lse_b = (m + np.log(tot))[..., 0]
                bad = np.isnan(m[..., 0])
                o[bad] = np.nan
                lse_b[bad] = np.nan
                out[a + blk, heads] = o
                lse[a + blk, heads] = lse_b
    return out, lse


def merge_ref(output, lse, part, part_lse, target) -> None:
    """slab_attention.py:341-356: FP32 LSE merge of one partial into (output, lse).

    Empty parts (LSE -inf) contribute nothing whatever their values; NaN
    propagates.  ``target`` indexes the rows of output/lse receiving ``part``.
    """
    old_lse = lse[target]
    part = np.asarray(part, np.float32)
    part_lse = np.asarray(part_lse, np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        maximum = np.maximum(old_lse, part_lse)
        safe = np.where(maximum == -np.inf, np.float32(0), maximum)
        alpha = np.exp(old_lse - safe).astype(np.float32)
        beta = np.exp(part_lse - safe).astype(np.float32)
        denom = (alpha + beta).astype(np.float32)
        denom = np.where(denom == 0.0, np.float32(1), denom)
        old = np.where((old_lse == -np.inf)[..., None], np.float32(0), output[target])
        new = np.where((part_lse == -np.inf)[..., None], np.float32(0), part)
        output[target] = (old * alpha[..., None] + new * beta[..., None]) / denom[..., None]
        lse[target] = maximum + np.log(denom)


def causal_prefill_ref(q, k, v, scale, *, q_dtype="bf16"):
    """decode_kernel.py:70-117 with no cached prefix: causal GQA attention.

    q [n, Hq, D], k/v [n, Hk, D] in the original (unrotated) domain; query i
    sees keys [0, i].  Returns the output rounded to q_dtype.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    n, hq, _ = q.shape
    group = hq // k.shape[1]
    out = np.zeros(q.shape, np.float64)
    for h in range(hq):
        s = q[:, h] @ k[:, h // group].T * scale
        s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
        m = s.max(-1, keepdims=True)
        p = np.exp(s - m)
        out[:, h] = (p @ v[:, h // group]) / p.sum(-1, keepdims=True)
    return fmt.round_to(out.astype(np.float32), q_dtype)
