"""Forward-level oracle: the reference backend's write + window + read path.

Test infrastructure only.  Restates on NumPy arrays the streaming-mode
control flow of /root/reference/oscar_ascend/backend.py:
``do_kv_cache_update`` (:151-198), ``_staging_write`` (:513-555) and
``_streaming_attention`` (:334-393), including the fresh-only split that runs
history-free requests in the original domain (:345-353, :435-458).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import fmt
from .attention import attention_ref, causal_prefill_ref
from .store import Staging, clip, rotate, store_ref


@dataclass
class OracleLayer:
    """Per-layer state the reference keeps on ``layer`` / the impl."""

    k8: np.ndarray            # uint8 [nb, bs, hk, W]
    v8: np.ndarray
    rk: np.ndarray            # fp32 [D, D]
    rv: np.ndarray
    hq: int
    hk: int
    d: int
    scale: float
    sink_tokens: int = 64
    recent_tokens: int = 256
    staging_tokens: int = 8192
    k_clip: float = 0.0
    v_clip: float = 0.0
    window_enabled: bool = True
    staging: Staging | None = None

    def ensure_staging(self) -> Staging:
        """backend.py:492-511."""
        if self.staging is None:
            self.staging = Staging(self.k8.shape[1], self.hk, self.d, self.sink_tokens,
                                   self.recent_tokens, self.staging_tokens)
        return self.staging


def do_kv_cache_update(layer: OracleLayer, key, value, slot_mapping) -> None:
    """backend.py:151-198 (torch reference store path)."""
    slots = np.asarray(slot_mapping, np.int64)
    n = slots.shape[0]
    if n <= 0 or key is None or value is None:
        return
    k = np.asarray(key, np.float32)[:n].reshape(n, layer.hk, layer.d)
    v = np.asarray(value, np.float32)[:n].reshape(n, layer.hk, layer.d)
    if layer.staging is not None:
        layer.staging.invalidate(slots)
    k_rot = clip(rotate(k, layer.rk), layer.k_clip)
    v_rot = clip(rotate(v, layer.rv), layer.v_clip)
    store_ref(k_rot, v_rot, layer.k8, layer.v8, slots)


def staging_write(layer: OracleLayer, key, value, slot_mapping, qsl, seqs) -> None:
    """backend.py:513-555: unclipped, unquantized fp32 rotated values + owner tags."""
    slots = np.asarray(slot_mapping, np.int64)
    n = slots.shape[0]
    if n == 0:
        return
    st = layer.ensure_staging()
    k = np.asarray(key, np.float32)[:n].reshape(n, layer.hk, layer.d)
    v = np.asarray(value, np.float32)[:n].reshape(n, layer.hk, layer.d)
    st.write(rotate(k, layer.rk), rotate(v, layer.rv), slots, qsl, seqs)


def forward(layer: OracleLayer, query, key, value, slot_mapping, qsl, seqs, block_tables,
            num_actual_tokens=None, q_dtype="bf16", rows=None):
    """backend.py:249-282 + :334-393 in streaming mode.

    query [N, Hq, D], key/value [N, Hk, D] or None; all on the q_dtype grid.
    ``rows`` (optional): token indices whose rotated-domain attention is evaluated
    (a sampled check of long chunks); the other cached rows stay 0.  Writes and
    fresh-only prefills are always evaluated in full.
    Returns the output [N, Hq, D] on the q_dtype grid (float32 array).
    """
    def rnd(x):
        return fmt.round_to(x, q_dtype)

    query = np.asarray(query, np.float32)
    n_tok = query.shape[0]
    actual_md = n_tok if num_actual_tokens is None else num_actual_tokens
    if key is not None and value is not None:
        slots = np.asarray(slot_mapping, np.int64)[:actual_md]
        do_kv_cache_update(layer, key, value, slots)
        if layer.window_enabled:
            staging_write(layer, key, value, slots, qsl, seqs)
    output = np.zeros_like(query)
    actual = min(n_tok, actual_md)
    if actual == 0:
        return output
    starts = [min(s, actual) for s in qsl]
    active = [i for i in range(len(starts) - 1) if starts[i + 1] > starts[i]]
    fresh = [i for i in active
             if key is not None and seqs[i] == starts[i + 1] - starts[i]]
    cached = [i for i in active if i not in fresh]
    for i in fresh:
        a, b = starts[i], starts[i + 1]
        output[a:b] = causal_prefill_ref(query[a:b], np.asarray(key, np.float32)[a:b],
                                         np.asarray(value, np.float32)[a:b], layer.scale,
                                         q_dtype=q_dtype)
    if cached:
        ids = np.concatenate([np.arange(starts[i], starts[i + 1]) for i in cached])
        lengths = [starts[i + 1] - starts[i] for i in cached]
        sub_qsl = np.concatenate([[0], np.cumsum(lengths)]).tolist()
        sub_seqs = [seqs[i] for i in cached]
        table = np.asarray(block_tables)[cached]
        sub_rows = None
        if rows is not None:
            wanted = set(int(t) for t in rows)
            sub_rows = [j for j, t in enumerate(ids) if int(t) in wanted]
        if sub_rows is None:
            q_rot = rnd(rotate(query[ids], layer.rk))
        else:
            q_rot = np.zeros((len(ids),) + query.shape[1:], np.float32)
            q_rot[sub_rows] = rnd(rotate(query[ids[sub_rows]], layer.rk))
        k_rot = None if key is None else rnd(rotate(np.asarray(key, np.float32)[ids], layer.rk))
        v_rot = None if value is None else rnd(rotate(np.asarray(value, np.float32)[ids], layer.rv))
        stage = layer.staging.arrays() if (layer.window_enabled and layer.staging) else None
        rotated, _ = attention_ref(q_rot, k_rot, v_rot, layer.k8, layer.v8, table, sub_qsl,
                                   sub_seqs, layer.scale, stage, d=layer.d, q_dtype=q_dtype,
                                   rows=sub_rows)
        keep = ids if sub_rows is None else ids[sub_rows]
        src = rotated if sub_rows is None else rotated[sub_rows]
        output[keep] = rnd(rotate(src, np.ascontiguousarray(layer.rv.T)))
    return output
