"""OSCAR INT2 FULL-attention impl for MI355X (drop-in for oscar_ascend/backend.py).

The plugin swaps ``impl.__class__`` of FULL decoder layers to
``OscarAttentionBackendImpl``; only ``forward`` and ``do_kv_cache_update`` (and
their helpers) are replaced, with the reference's signatures and metadata
accessors.  The arithmetic runs in liboscar_amd.so:

* write   ``ops.store``: rotate (fp64-accumulated, correctly rounded), sort-clip,
          INT2 quantize/pack/scatter with last-writer-wins, staging owner tags and
          FP32 window, plus the bf16 rotated q/k/v the read path needs;
* read    ``ops.attention_decode`` (requests with <= 32 rows per KV head) and
          ``ops.attention_prefill`` (long continuation chunks and history-free
          prefill in the original domain), then the inverse rotation
          ``ops.rotate(out_rot, R_v^T)``.

There is no dense-history or CPU fallback: failures raise.
"""
from __future__ import annotations

from importlib import import_module, util
from itertools import pairwise

import torch

from . import ops
from ._lib import STAGE_INVALIDATE, STAGE_NONE, STAGE_WRITE
from .config import OscarConfig
from .format import K_IDX_OFF, VALUES_PER_BYTE, check_d
from .rotation import get_layer_rotation

MAX_DECODE_ROWS = 32


def metadata_batch_lists(attn_metadata) -> tuple[list, list]:
    """backend.py:26-56: host (query_start_loc, seq_lens) lists; never a Tensor as bool."""

    def _as_list(x, name: str) -> list:
        if x is None:
            raise RuntimeError(f"attn_metadata.{name} is missing")
        if hasattr(x, "tolist"):
            return x.tolist()
        return list(x)

    q_sl_cpu = getattr(attn_metadata, "query_start_loc_cpu", None)
    ends = getattr(attn_metadata, "actual_seq_lengths_q", None)
    if q_sl_cpu is not None:
        qsl = _as_list(q_sl_cpu, "query_start_loc_cpu")
    elif ends is not None:
        qsl = [0] + _as_list(ends, "actual_seq_lengths_q")
    else:
        qsl = _as_list(attn_metadata.query_start_loc, "query_start_loc")
    seq_cpu = getattr(attn_metadata, "seq_lens_cpu", None)
    if seq_cpu is None:
        seq_cpu = getattr(attn_metadata, "_seq_lens_cpu", None)
    seq_list = getattr(attn_metadata, "seq_lens_list", None)
    seqs = _as_list(seq_list if seq_list is not None else (
        seq_cpu if seq_cpu is not None else attn_metadata.seq_lens), "seq_lens")
    return qsl, seqs


def _block_tables(md):
    bt = getattr(md, "block_tables", None)
    return bt if bt is not None else md.block_table


def _load_base_impl():
    """Base class: vLLM's ROCm attention impl when vLLM is installed, else object.

    Mirrors backend.py:68-85: an installed but broken vendor stack must fail
    loudly instead of silently degrading to a placeholder.
    """
    if util.find_spec("vllm") is None:
        return object
    try:
        _ = import_module("vllm.platforms").current_platform
        native = import_module("vllm.v1.attention.backends.rocm_attn")
        return native.RocmAttentionImpl
    except Exception as exc:
        raise RuntimeError("OSCAR could not import the installed ROCm attention backend") from exc


BaseAttentionImpl = _load_base_impl()


class OscarAttentionBackendImpl(BaseAttentionImpl):  # type: ignore[misc,valid-type]
    """OSCAR INT2 FULL-layer attention (class surgery target)."""

    # ------------------------------------------------------------------ setup
    def _oscar_setup(self) -> None:
        """backend.py:100-123."""
        if getattr(self, "_oscar_cfg", None) is not None:
            return
        cfg = OscarConfig.from_env(head_dim=self.head_size)
        check_d(cfg.head_dim)
        if self.num_heads % self.num_kv_heads:
            raise ValueError("OSCAR requires Hq divisible by Hk")
        self._oscar_cfg = cfg
        self._oscar_stage_ready = False
        self._oscar_stats = {"writes": 0, "kv_bytes_written": 0, "reads": 0}
        if cfg.verbose:
            print(f"[oscar-amd] OSCAR impl ready: D={self.head_size}, slot=160B (K 96B + V 64B), "
                  f"K rotation={'loaded' if cfg.k_rotation_path else 'identity'}, "
                  f"V rotation={'loaded' if cfg.v_rotation_path else 'identity'}, "
                  f"window(sink={cfg.sink_tokens}, recent={cfg.recent_tokens})")

    @property
    def _oscar(self) -> OscarConfig:
        return self._oscar_cfg

    # ------------------------------------------------------------------ geometry
    def _set_caches(self, kv_cache) -> None:
        """backend.py:200-236: accept a (K, V) pair or a stacked tensor; check slot fit."""
        if isinstance(kv_cache, (tuple, list)) and len(kv_cache) >= 2:
            self.key_cache, self.value_cache = kv_cache[0], kv_cache[1]
        elif isinstance(kv_cache, torch.Tensor) and kv_cache.dim() > 0:
            self.key_cache, self.value_cache = kv_cache[0], kv_cache[1]
        if getattr(self, "key_cache", None) is None or getattr(self, "value_cache", None) is None:
            raise ValueError("OSCAR requires K and V caches")
        if not getattr(self, "_oscar_geo_ok", False):
            k8 = self.key_cache.view(torch.uint8)
            v8 = self.value_cache.view(torch.uint8)
            if k8.ndim != 4 or v8.ndim != 4 or not k8.is_contiguous() or not v8.is_contiguous():
                raise ValueError("OSCAR requires contiguous [blocks, tokens, heads, bytes] caches")
            slot_k, slot_v = int(k8.stride(2)), int(v8.stride(2))
            need_k = K_IDX_OFF + self.head_size // VALUES_PER_BYTE
            need_v = self.head_size // VALUES_PER_BYTE
            if slot_k not in (self.head_size, 2 * self.head_size):
                raise AssertionError(f"[oscar-amd] K slot width {slot_k}B, expected "
                                     f"{self.head_size} (packed) or {2 * self.head_size} (legacy)")
            if need_k > slot_k or need_v > slot_v:
                raise AssertionError(f"[oscar-amd] slot too small: K needs {need_k}B / V {need_v}B")
            self._oscar_geo_ok = True

    def _layer_rots(self, layer, device):
        """backend.py:238-246: strict per-layer R_k, R_v cached on the layer."""
        if not getattr(layer, "_oscar_rots", None):
            cfg = self._oscar
            rk = get_layer_rotation(cfg.k_rotation_path, layer.layer_name, self.head_size, device,
                                    mode="k", strict=True)
            rv = get_layer_rotation(cfg.v_rotation_path, layer.layer_name, self.head_size, device,
                                    mode="v", strict=True)
            layer._oscar_rots = (rk, rv)
        rk, rv = layer._oscar_rots
        if rk.device != device or rk.dtype != torch.float32:
            rk = rk.to(device=device, dtype=torch.float32).contiguous()
            rv = rv.to(device=device, dtype=torch.float32).contiguous()
            layer._oscar_rots = (rk, rv)
        return layer._oscar_rots

    # ------------------------------------------------------------------ staging arena
    def _ensure_staging(self, layer, kv_cache) -> None:
        """backend.py:492-511: per-layer FP32 window arena and owner tags."""
        if getattr(layer, "_oscar_stage_ready", False):
            return
        bs = kv_cache[0].shape[1]
        cfg = self._oscar
        self.stage_block = bs
        self.sink_eff = (cfg.sink_tokens // bs) * bs
        self.sink_pages = self.sink_eff // bs
        self.tail_pages = (cfg.recent_tokens + bs - 1) // bs + 1
        rows = max((cfg.staging_tokens + bs - 1) // bs, self.sink_pages + self.tail_pages + 2)
        dev = kv_cache[0].device
        layer._oscar_stage_k = torch.zeros(rows, bs, self.num_kv_heads, self.head_size,
                                           dtype=torch.float32, device=dev)
        layer._oscar_stage_v = torch.zeros_like(layer._oscar_stage_k)
        layer._oscar_slot_owner = torch.full((rows, bs), -1, dtype=torch.int64, device=dev)
        layer._oscar_stage_rows = rows
        layer._oscar_stage_ready = True
        self._oscar_stage_ready = True

    def _stage(self, layer):
        if self._oscar.window_enabled and getattr(layer, "_oscar_stage_ready", False):
            return (layer._oscar_stage_k, layer._oscar_stage_v, layer._oscar_slot_owner)
        return None

    # ------------------------------------------------------------------ write path
    def _store(self, layer, key, value, slot_mapping, *, mode, qsl=None, seqs=None, query=None,
               outputs=None):
        n = slot_mapping.shape[0]
        D, hk = self.head_size, self.num_kv_heads
        rk, rv = self._layer_rots(layer, key.device)
        stage = None
        if getattr(layer, "_oscar_stage_ready", False):
            stage = (layer._oscar_stage_k, layer._oscar_stage_v, layer._oscar_slot_owner)
        extra = {}
        if mode == STAGE_WRITE:
            n_req = len(seqs)
            qsl_t = torch.tensor(qsl[: n_req + 1], dtype=torch.int32).to(key.device)
            seq_t = torch.tensor(seqs[:n_req] or [0], dtype=torch.int32).to(key.device)
            extra = dict(qsl_dev=qsl_t, seqs_dev=seq_t, num_reqs=n_req,
                         recent_tokens=self._oscar.recent_tokens,
                         sink_tokens_eff=self.sink_eff)
        q_rot = k_rot = v_rot = None
        if outputs:
            k_rot = torch.empty(n, hk, D, dtype=key.dtype, device=key.device)
            v_rot = torch.empty_like(k_rot)
            if query is not None:
                q_rot = torch.empty(n, query.shape[1], D, dtype=query.dtype, device=key.device)
        ops.store(key[:n], value[:n], self.key_cache, self.value_cache, slot_mapping,
                  head_dim=D, rk=rk, rv=rv, k_clip=self._oscar.k_clip_ratio,
                  v_clip=self._oscar.v_clip_ratio, stage=stage,
                  stage_mode=mode if stage is not None else STAGE_NONE,
                  query=None if query is None else query[:n], query_rot=q_rot,
                  key_rot=k_rot, value_rot=v_rot, **extra)
        self._oscar_stats["writes"] += 1
        self._oscar_stats["kv_bytes_written"] += n * hk * 160
        return q_rot, k_rot, v_rot

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping) -> None:
        """backend.py:151-198: standalone INT2 write; rewritten seats lose their window copy."""
        if key is None or value is None:
            return
        slot_mapping = slot_mapping.to(device=key.device, dtype=torch.int64)
        if slot_mapping.shape[0] <= 0:
            return
        self._set_caches(kv_cache)
        self._store(layer, key, value, slot_mapping, mode=STAGE_INVALIDATE)

    def _staging_write(self, layer, key, value, attn_metadata) -> None:
        """backend.py:513-555: window values and owner tags (the INT2 bytes are rewritten
        with identical contents by the same fused call)."""
        n = attn_metadata.num_actual_tokens
        if n == 0:
            return
        qsl, seqs = metadata_batch_lists(attn_metadata)
        slots = attn_metadata.slot_mapping[:n].to(device=key.device, dtype=torch.int64)
        self._store(layer, key, value, slots, mode=STAGE_WRITE, qsl=qsl, seqs=seqs)

    # ------------------------------------------------------------------ forward
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        """backend.py:249-282 (streaming mode)."""
        assert output is not None, "Output tensor must be provided."
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("OSCAR fused output quantization is unsupported")
        if attn_metadata is None:
            return output.fill_(0)
        self._set_caches(kv_cache)
        if (key is None) != (value is None):
            raise ValueError("Both new K and V must be supplied together")
        rotated = None
        if key is not None:
            n = attn_metadata.num_actual_tokens
            slots = attn_metadata.slot_mapping[:n].to(device=key.device, dtype=torch.int64)
            mode = STAGE_NONE
            qsl = seqs = None
            if self._oscar.window_enabled:
                self._ensure_staging(layer, kv_cache)
                mode = STAGE_WRITE
                qsl, seqs = metadata_batch_lists(attn_metadata)
            elif getattr(layer, "_oscar_stage_ready", False):
                mode = STAGE_INVALIDATE
            if n > 0:
                rotated = self._store(layer, key.view(-1, self.num_kv_heads, self.head_size),
                                      value.view(-1, self.num_kv_heads, self.head_size), slots,
                                      mode=mode, qsl=qsl, seqs=seqs,
                                      query=query.view(-1, self.num_heads, self.head_size),
                                      outputs=True)
        return self._streaming_attention(layer, query, key, value, kv_cache, attn_metadata,
                                         output, rotated)

    def _streaming_attention(self, layer, query, key, value, kv_cache, metadata, output,
                             rotated=None):
        """backend.py:334-393: fresh-only requests prefill in the original domain; cached
        requests attend in the rotated domain, then out_rot @ R_v^T."""
        if (key is None) != (value is None):
            raise ValueError("Both new K and V must be supplied together")
        if query.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("OSCAR MI355X attention requires bf16 or fp16 queries; "
                             f"got dtype={query.dtype}")
        D, hq, hk = self.head_size, self.num_heads, self.num_kv_heads
        group = hq // hk
        q3 = query.view(-1, hq, D)
        actual = min(q3.shape[0], metadata.num_actual_tokens)
        output.zero_()
        if actual == 0:
            return output
        out3 = output.view(-1, hq, D)
        starts, seqs = metadata_batch_lists(metadata)
        starts = [min(s, actual) for s in starts]
        active = [i for i, (a, b) in enumerate(pairwise(starts)) if b > a]
        fresh = [i for i in active if key is not None and seqs[i] == starts[i + 1] - starts[i]]
        cached = [i for i in active if i not in fresh]
        k3 = None if key is None else key.view(-1, hk, D)
        v3 = None if value is None else value.view(-1, hk, D)
        for i in fresh:
            a, b = starts[i], starts[i + 1]
            out3[a:b] = ops.attention_prefill(q3[a:b], k3[a:b], v3[a:b], self.scale, head_dim=D)
        if not cached:
            return output
        rk, rv = self._layer_rots(layer, query.device)
        if rotated is not None:
            q_rot, k_rot, v_rot = rotated
        else:
            q_rot = ops.rotate(q3[:actual], rk)
            k_rot = None if k3 is None else ops.rotate(k3[:actual], rk)
            v_rot = None if v3 is None else ops.rotate(v3[:actual], rv)
        stage = self._stage(layer)
        table = _block_tables(metadata)
        out_rot = torch.zeros(actual, hq, D, dtype=torch.float32, device=query.device)
        lse = torch.full((actual, hq), float("-inf"), dtype=torch.float32, device=query.device)
        has_new = key is not None
        short = [i for i in cached if (starts[i + 1] - starts[i]) * group <= MAX_DECODE_ROWS]
        long = [i for i in cached if i not in short]
        # cache-only long chunks: split into sub-requests of at most 32 rows (right-aligned
        # causality is preserved: sub-request j sees the keys up to its own last query)
        sub_qsl, sub_seqs, sub_rows = [0], [], []
        step = max(1, MAX_DECODE_ROWS // group)
        for i in short + ([] if has_new else long):
            a, b, seq = starts[i], starts[i + 1], seqs[i]
            for s in range(a, b, step):
                e = min(b, s + step)
                sub_rows.append((i, s, e))
                sub_qsl.append(sub_qsl[-1] + e - s)
                sub_seqs.append(seq - (b - e))
        if has_new and any(seqs[i] < starts[i + 1] - starts[i] for i in cached):
            raise ValueError("Sequence length must cover its query chunk")
        if sub_rows:
            ids = torch.cat([torch.arange(s, e) for _, s, e in sub_rows]).to(query.device)
            req = torch.tensor([i for i, _, _ in sub_rows], device=table.device)
            kn = None if not has_new else k_rot[ids]
            vn = None if not has_new else v_rot[ids]
            window = (self.sink_eff, self._oscar.recent_tokens) if stage is not None else (0, 0)
            plan = ops.plan_decode(sub_qsl, sub_seqs, has_new=has_new, num_kv_heads=hk,
                                   group=group, head_dim=D, device=query.device, window=window)
            o, l = ops.attention_decode(q_rot[ids], kn, vn, self.key_cache, self.value_cache,
                                        table[req], plan, self.scale, stage, head_dim=D)
            out_rot[ids], lse[ids] = o, l
        if has_new:
            for i in long:
                a, b, seq = starts[i], starts[i + 1], seqs[i]
                lse_i = torch.empty(b - a, hq, dtype=torch.float32, device=query.device)
                out_rot[a:b] = ops.attention_prefill(
                    q_rot[a:b], k_rot[a:b], v_rot[a:b], self.scale, head_dim=D,
                    history=seq - (b - a), k_cache=self.key_cache, v_cache=self.value_cache,
                    block_table_row=table[i], stage=stage, lse=lse_i)
                lse[a:b] = lse_i
        idx = torch.tensor([t for i in cached for t in range(starts[i], starts[i + 1])],
                           device=query.device)
        out3[idx] = ops.rotate(out_rot[idx], rv, transpose=True, out_dtype=query.dtype)
        self._oscar_stats["reads"] += 1
        self._last_lse = lse
        return output
