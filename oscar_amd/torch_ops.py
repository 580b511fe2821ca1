"""The C-ABI entry points as torch operators (``torch.ops.oscar_amd.*``).

Each operator calls the same library entry point as :mod:`oscar_amd.ops` and carries a
fake (meta) implementation, so the calls are visible to torch: schema-checked, traced
by ``torch.compile`` / ``torch.fx`` with the right output shapes and mutated inputs,
and dispatched on the CUDA (HIP) key only.  A nonzero status raises, as the direct
wrappers do.

Operators (tensors in the layouts of the C structs; optional staging tensors are the
layer's FP32 window arena):

* ``rotate(x, r, transpose) -> Tensor``: x @ R or x @ R^T in x's dtype
  (``oscar_rotate_v1``; backend.py:371,382).
* ``store(key, value, k_cache!, v_cache!, slot_mapping, stage_k!, stage_v!, owner!,
  head_dim, rk, rv, k_clip, v_clip, stage_mode, query_start_loc, seq_lens,
  recent_tokens, sink_tokens_eff) -> ()``: the write path (``oscar_store_v1``;
  store_kernel.py:54-102, backend.py:130-198,513-555); the arena tensors are passed
  (None without a window) because they are mutated.
* ``attention_decode(q, k_new, v_new, k_cache, v_cache, block_table, query_start_loc,
  seq_lens, scale, head_dim, stage_k, stage_v, owner, sink_tokens_eff, recent_tokens)
  -> (out_rot, lse)``: plan + split-K decode + merge (``oscar_attn_plan_v1`` /
  ``oscar_attn_decode_v1``; slab_attention.py:23-92,376-476); the request lists are
  host integers.
* ``attention_prefill(q, k, v, scale, head_dim, history, k_cache, v_cache,
  block_table_row, stage_k, stage_v, owner) -> (out, lse)``: fresh-only (history 0,
  output in q's dtype, lse empty) or continuation prefill (fp32 rotated output and LSE)
  (``oscar_attn_prefill_v1``; prefill.py:69-72, slab_attention.py:376-476).
"""
from __future__ import annotations

import torch

from . import ops

_LIB = "oscar_amd"


def _stage(stage_k, stage_v, owner):
    if stage_k is None and stage_v is None and owner is None:
        return None
    if stage_k is None or stage_v is None or owner is None:
        raise ValueError("the window arena needs stage_k, stage_v and owner together")
    return (stage_k, stage_v, owner)


# ------------------------------------------------------------------ rotate
@torch.library.custom_op(f"{_LIB}::rotate", mutates_args=(), device_types="cuda")
def rotate(x: torch.Tensor, r: torch.Tensor, transpose: bool = False) -> torch.Tensor:
    return ops.rotate(x, r, transpose=transpose)


@rotate.register_fake
def _(x, r, transpose=False):
    return torch.empty_like(x)


# ------------------------------------------------------------------ store
@torch.library.custom_op(f"{_LIB}::store", mutates_args=("k_cache", "v_cache", "stage_k", "stage_v", "owner"),
                         device_types="cuda")
def store(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
          slot_mapping: torch.Tensor, stage_k: torch.Tensor | None, stage_v: torch.Tensor | None,
          owner: torch.Tensor | None, head_dim: int, rk: torch.Tensor | None = None,
          rv: torch.Tensor | None = None, k_clip: float = 0.0, v_clip: float = 0.0, stage_mode: int = 0,
          query_start_loc: torch.Tensor | None = None, seq_lens: torch.Tensor | None = None,
          recent_tokens: int = 0, sink_tokens_eff: int = 0) -> None:
    num_reqs = 0 if seq_lens is None else int(seq_lens.numel())
    ops.store(key, value, k_cache, v_cache, slot_mapping, head_dim=head_dim, rk=rk, rv=rv,
              k_clip=k_clip, v_clip=v_clip, stage=_stage(stage_k, stage_v, owner), stage_mode=stage_mode,
              qsl_dev=query_start_loc, seqs_dev=seq_lens, num_reqs=num_reqs,
              recent_tokens=recent_tokens, sink_tokens_eff=sink_tokens_eff)


@store.register_fake
def _(key, value, k_cache, v_cache, slot_mapping, stage_k, stage_v, owner, head_dim, rk=None, rv=None,
      k_clip=0.0, v_clip=0.0, stage_mode=0, query_start_loc=None, seq_lens=None, recent_tokens=0,
      sink_tokens_eff=0):
    return None


# ------------------------------------------------------------------ decode
@torch.library.custom_op(f"{_LIB}::attention_decode", mutates_args=(), device_types="cuda")
def attention_decode(q: torch.Tensor, k_new: torch.Tensor | None, v_new: torch.Tensor | None,
                     k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                     query_start_loc: list[int], seq_lens: list[int], scale: float, head_dim: int,
                     stage_k: torch.Tensor | None = None, stage_v: torch.Tensor | None = None,
                     owner: torch.Tensor | None = None, sink_tokens_eff: int = 0,
                     recent_tokens: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    hq, hk = q.shape[1], k_cache.shape[2]
    stage = _stage(stage_k, stage_v, owner)
    window = (sink_tokens_eff, recent_tokens) if stage is not None else (0, 0)
    plan = ops.plan_decode(list(query_start_loc), list(seq_lens), has_new=k_new is not None,
                           num_kv_heads=hk, group=hq // hk, head_dim=head_dim, device=q.device, window=window)
    return ops.attention_decode(q, k_new, v_new, k_cache, v_cache, block_table, plan, scale, stage,
                                head_dim=head_dim)


@attention_decode.register_fake
def _(q, k_new, v_new, k_cache, v_cache, block_table, query_start_loc, seq_lens, scale, head_dim,
      stage_k=None, stage_v=None, owner=None, sink_tokens_eff=0, recent_tokens=0):
    n, hq = q.shape[0], q.shape[1]
    return (q.new_empty((n, hq, head_dim), dtype=torch.float32), q.new_empty((n, hq), dtype=torch.float32))


# ------------------------------------------------------------------ prefill
@torch.library.custom_op(f"{_LIB}::attention_prefill", mutates_args=(), device_types="cuda")
def attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, head_dim: int,
                      history: int = 0, k_cache: torch.Tensor | None = None,
                      v_cache: torch.Tensor | None = None, block_table_row: torch.Tensor | None = None,
                      stage_k: torch.Tensor | None = None, stage_v: torch.Tensor | None = None,
                      owner: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    n, hq = q.shape[0], q.shape[1]
    lse = torch.empty((n, hq) if history > 0 else (0,), dtype=torch.float32, device=q.device)
    out = ops.attention_prefill(q, k, v, scale, head_dim=head_dim, history=history, k_cache=k_cache,
                                v_cache=v_cache, block_table_row=block_table_row,
                                stage=_stage(stage_k, stage_v, owner), lse=lse if history > 0 else None)
    return out, lse


@attention_prefill.register_fake
def _(q, k, v, scale, head_dim, history=0, k_cache=None, v_cache=None, block_table_row=None,
      stage_k=None, stage_v=None, owner=None):
    n, hq = q.shape[0], q.shape[1]
    if history > 0:
        return (q.new_empty((n, hq, head_dim), dtype=torch.float32), q.new_empty((n, hq), dtype=torch.float32))
    return q.new_empty((n, hq, head_dim)), q.new_empty((0,), dtype=torch.float32)
