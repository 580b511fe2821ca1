"""OSCAR INT2 FULL-attention impl for MI355X (drop-in for oscar_ascend/backend.py).

The plugin swaps ``impl.__class__`` of FULL decoder layers to
``OscarAttentionBackendImpl``; ``forward`` and ``do_kv_cache_update`` keep the
reference's signatures (backend.py:151-158, :249-260) and metadata accessors.  The
arithmetic runs in liboscar_amd.so:

* write  ``ops.store``: rotate (correctly rounded), sort-clip, INT2 quantize / pack /
         scatter with last-writer-wins, owner tags and FP32 window, plus the rotated
         q/k/v the read path needs;
* read   ``ops.attention_decode`` (cached requests; chunks of more than 32 rows per KV
         head as 32-row sub-requests of the plan, up to MAX_SPLIT_ROWS),
         ``ops.attention_prefill`` (longer continuation chunks; history-free requests in
         the original domain), then the inverse rotation ``ops.rotate(out_rot, R_v^T)``.

Host work per call is bounded: the batch is classified on the host from the
metadata's host lists, every integer array the kernels need goes to the device in one
non-blocking copy from pinned memory, and a batch of decode-shaped requests (the
serving steady state) runs with no gathers or scatters.  There is no dense-history or
CPU fallback: failures raise.
"""
from __future__ import annotations

from ctypes import pointer as ctypes_pointer
from dataclasses import dataclass, field
from importlib import import_module, util

import numpy as np
import torch

from . import _lib, ops
from ._lib import STAGE_INVALIDATE, STAGE_NONE, STAGE_WRITE
from .config import OscarConfig
from .integration import arena_rows
from .format import K_IDX_OFF, VALUES_PER_BYTE, check_d
from .rotation import get_layer_rotation

MAX_DECODE_ROWS = 32  # rows (query tokens x heads per KV head) of one decode MFMA tile
# A cached chunk of more rows per KV head runs through the split-K decode as
# sub-requests of MAX_DECODE_ROWS rows (each streams the request's history once), up to
# this many rows; longer chunks go to the MFMA prefill, which decodes the history once
# and shares it between query tiles but walks it serially per query tile (at 24576
# history tokens: 24-156 us for chunks of 8-400 tokens against 1.1 ms).
MAX_SPLIT_ROWS = 32 * 512


# ---------------------------------------------------------------- metadata
def _host_list(value) -> list:
    return value.tolist() if hasattr(value, "tolist") else list(value)


# (attribute, how it becomes query_start_loc) in the order the reference consults them
# (backend.py:26-56): a host tensor first, then vLLM-Ascend's cumulative ends, then the
# device tensor.  Presence is tested with `is not None`: a multi-element tensor has no
# truth value.
_QUERY_STARTS = (("query_start_loc_cpu", lambda v: v),
                 ("actual_seq_lengths_q", lambda ends: [0] + ends),
                 ("query_start_loc", lambda v: v))
_SEQ_LENS = ("seq_lens_list", "seq_lens_cpu", "_seq_lens_cpu", "seq_lens")


def metadata_batch_lists(attn_metadata) -> tuple[list, list]:
    """Host (query_start_loc, seq_lens) lists of a batch."""
    for attr, shape in _QUERY_STARTS:
        value = getattr(attn_metadata, attr, None)
        if value is not None:
            qsl = shape(_host_list(value))
            break
    else:
        raise RuntimeError("attn_metadata carries no query start locations")
    for attr in _SEQ_LENS:
        value = getattr(attn_metadata, attr, None)
        if value is not None:
            return qsl, _host_list(value)
    raise RuntimeError("attn_metadata carries no sequence lengths")


def _block_tables(md):
    bt = getattr(md, "block_tables", None)
    return bt if bt is not None else md.block_table


def _host_int32(value):
    """A host int32 array for the native step (zero-copy for a contiguous CPU int32
    tensor); None when the value lives on the device (reading it would synchronise)."""
    if value is None:
        return None
    if isinstance(value, torch.Tensor):
        if value.device.type != "cpu":
            return None
        return value if value.dtype == torch.int32 and value.is_contiguous() else value.to(torch.int32).contiguous()
    return np.asarray(value, np.int32)


def _address(arr) -> int:
    return arr.data_ptr() if isinstance(arr, torch.Tensor) else arr.ctypes.data


def host_metadata_arrays(md):
    """(query_start_loc, seq_lens) as host int32 arrays, consulted in the order of
    metadata_batch_lists; None if only device copies exist."""
    qsl = _host_int32(getattr(md, "query_start_loc_cpu", None))
    if qsl is None:
        ends = getattr(md, "actual_seq_lengths_q", None)
        if ends is None or isinstance(ends, torch.Tensor) and ends.device.type != "cpu":
            return None
        qsl = np.concatenate([[0], np.asarray(_host_list(ends), np.int32)]).astype(np.int32)
    for attr in _SEQ_LENS[:3]:
        value = getattr(md, attr, None)
        if value is not None:
            seqs = _host_int32(value)
            return (qsl, seqs) if seqs is not None else None
    return None


def _native_base():
    """vLLM's ROCm attention impl when vLLM is installed, else ``object``.  An installed
    but unimportable stack raises (the reference's rule, backend.py:68-85): the plugin
    must not silently degrade to a placeholder."""
    if util.find_spec("vllm") is None:
        return object
    try:
        _ = import_module("vllm.platforms").current_platform
        return import_module("vllm.v1.attention.backends.rocm_attn").RocmAttentionImpl
    except Exception as exc:
        raise RuntimeError("OSCAR could not import the installed ROCm attention backend") from exc


BaseAttentionImpl = _native_base()


# ---------------------------------------------------------------- batch classification
@dataclass
class _Batch:
    """Host view of one read: which requests go where (backend.py:334-393 routing)."""
    qsl: list                  # query starts clipped to the actual token count
    seqs: list
    actual: int
    fresh: list = field(default_factory=list)   # no history: original-domain prefill
    short: list = field(default_factory=list)   # cached, split-K decode (sub-requests of
                                                # <= 32 rows per KV head for longer chunks)
    long: list = field(default_factory=list)    # cached chunk of more than MAX_SPLIT_ROWS: prefill

    @classmethod
    def classify(cls, qsl, seqs, actual, has_new, group):
        b = cls([min(s, actual) for s in qsl], list(seqs), actual)
        for i in range(len(b.qsl) - 1):
            n = b.qsl[i + 1] - b.qsl[i]
            if n <= 0:
                continue
            if has_new and b.seqs[i] == n:
                b.fresh.append(i)
            elif group <= MAX_DECODE_ROWS and (not has_new or n * group <= MAX_SPLIT_ROWS):
                b.short.append(i)
            else:
                b.long.append(i)
        if has_new and any(b.seqs[i] < b.qsl[i + 1] - b.qsl[i] for i in b.short + b.long):
            raise ValueError("Sequence length must cover its query chunk")
        return b

    @property
    def decode_only(self) -> bool:
        """Every active request goes to the split-K decode: the plan runs over the batch
        as it is."""
        return not self.fresh and not self.long

    def span(self, members):
        """(i0, i1, a, b) when requests i0 <= i < i1 are the members and empty requests and
        their query rows are [a, b); None when another request's rows lie in between."""
        lo, hi = min(members), max(members)
        inside = set(members)
        if any(j not in inside and self.qsl[j + 1] > self.qsl[j] for j in range(lo, hi + 1)):
            return None
        return lo, hi + 1, self.qsl[lo], self.qsl[hi + 1]

    @property
    def covers_all(self) -> bool:
        """The requests' query ranges tile [0, actual) (no padding rows to zero)."""
        return self.qsl[0] == 0 and self.qsl[-1] == self.actual


class OscarAttentionBackendImpl(BaseAttentionImpl):  # type: ignore[misc,valid-type]
    """OSCAR INT2 FULL-layer attention (class surgery target)."""

    # ------------------------------------------------------------------ setup
    def _oscar_setup(self) -> None:
        """Idempotent per impl: configuration from the environment, shape checks."""
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
        """Take the (K, V) pair or a stacked [2, ...] tensor; check the slot geometry
        once: the slot width must be D (packed int8) or 2D (legacy bf16) bytes, and the
        96-byte K / 64-byte V payload must fit (backend.py:200-236 contract)."""
        pair = None
        if isinstance(kv_cache, (tuple, list)) and len(kv_cache) >= 2:
            pair = (kv_cache[0], kv_cache[1])
        elif isinstance(kv_cache, torch.Tensor) and kv_cache.dim() > 0:
            pair = (kv_cache[0], kv_cache[1])
        if pair is not None:
            self.key_cache, self.value_cache = pair
        if getattr(self, "key_cache", None) is None or getattr(self, "value_cache", None) is None:
            raise ValueError("OSCAR requires K and V caches")
        if getattr(self, "_oscar_geo_ok", False):
            return
        k8, v8 = self.key_cache.view(torch.uint8), self.value_cache.view(torch.uint8)
        if k8.ndim != 4 or v8.ndim != 4 or not k8.is_contiguous() or not v8.is_contiguous():
            raise ValueError("OSCAR requires contiguous [blocks, tokens, heads, bytes] caches")
        d = self.head_size
        k_slot, v_slot = int(k8.stride(2)), int(v8.stride(2))
        if k_slot not in (d, 2 * d):
            raise AssertionError(f"[oscar-amd] K slot width {k_slot}B, expected {d} (packed) "
                                 f"or {2 * d} (legacy)")
        k_need, v_need = K_IDX_OFF + d // VALUES_PER_BYTE, d // VALUES_PER_BYTE
        if k_need > k_slot or v_need > v_slot:
            raise AssertionError(f"[oscar-amd] slot too small: K needs {k_need}B / V {v_need}B")
        self._oscar_geo_ok = True

    def _layer_rots(self, layer, device):
        """(R_k, R_v) of the layer, loaded strictly once and kept on the layer as fp32."""
        rots = getattr(layer, "_oscar_rots", None)
        if not rots:
            cfg = self._oscar
            rots = tuple(get_layer_rotation(path, layer.layer_name, self.head_size, device,
                                            mode=mode, strict=True)
                         for path, mode in ((cfg.k_rotation_path, "k"), (cfg.v_rotation_path, "v")))
        if rots[0].device != device or rots[0].dtype != torch.float32:
            rots = tuple(r.to(device=device, dtype=torch.float32).contiguous() for r in rots)
        layer._oscar_rots = rots
        return rots

    # ------------------------------------------------------------------ staging arena
    def _ensure_staging(self, layer, kv_cache) -> None:
        """Allocate the layer's FP32 window arena once (backend.py:492-511 sizing): seats
        for ceil(staging / bs) pages, and never fewer than the sink pages, the recent
        pages (+1 for a page boundary) and 2 spare rows."""
        if getattr(layer, "_oscar_stage_ready", False):
            return
        cfg = self._oscar
        bs = kv_cache[0].shape[1]
        self.stage_block = bs
        self.sink_eff = cfg.sink_tokens - cfg.sink_tokens % bs   # whole sink pages only
        rows = arena_rows(cfg, bs)
        dev = kv_cache[0].device
        shape = (rows, bs, self.num_kv_heads, self.head_size)
        layer._oscar_stage_k = torch.zeros(shape, dtype=torch.float32, device=dev)
        layer._oscar_stage_v = torch.zeros(shape, dtype=torch.float32, device=dev)
        layer._oscar_slot_owner = torch.full(shape[:2], -1, dtype=torch.int64, device=dev)
        layer._oscar_stage_rows = rows
        layer._oscar_stage_ready = self._oscar_stage_ready = True

    def _stage(self, layer):
        if self._oscar.window_enabled and getattr(layer, "_oscar_stage_ready", False):
            return (layer._oscar_stage_k, layer._oscar_stage_v, layer._oscar_slot_owner)
        return None

    # ------------------------------------------------------------------ write path
    def _store(self, layer, key, value, slot_mapping, *, mode, qsl_dev=None, seqs_dev=None,
               num_reqs=0, query=None, outputs=False):
        """One fused store call; returns the rotated (q, k, v) for the read when asked."""
        n = slot_mapping.shape[0]
        d, hk = self.head_size, self.num_kv_heads
        rk, rv = self._layer_rots(layer, key.device)
        stage = None
        if getattr(layer, "_oscar_stage_ready", False):
            stage = (layer._oscar_stage_k, layer._oscar_stage_v, layer._oscar_slot_owner)
        window = {}
        if mode == STAGE_WRITE:
            window = dict(qsl_dev=qsl_dev, seqs_dev=seqs_dev, num_reqs=num_reqs,
                          recent_tokens=self._oscar.recent_tokens, sink_tokens_eff=self.sink_eff)
        q_rot = k_rot = v_rot = None
        if outputs:
            k_rot = torch.empty(n, hk, d, dtype=key.dtype, device=key.device)
            v_rot = torch.empty_like(k_rot)
            if query is not None:
                q_rot = torch.empty(n, query.shape[1], d, dtype=query.dtype, device=key.device)
        ops.store(key[:n], value[:n], self.key_cache, self.value_cache, slot_mapping,
                  head_dim=d, rk=rk, rv=rv, k_clip=self._oscar.k_clip_ratio,
                  v_clip=self._oscar.v_clip_ratio, stage=stage,
                  stage_mode=mode if stage is not None else STAGE_NONE,
                  query=None if query is None else query[:n], query_rot=q_rot,
                  key_rot=k_rot, value_rot=v_rot, **window)
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

    # ------------------------------------------------------------------ forward
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        """backend.py:249-282 (streaming mode): write + window, then the read."""
        assert output is not None, "Output tensor must be provided."
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("OSCAR fused output quantization is unsupported")
        if attn_metadata is None:
            return output.fill_(0)
        self._set_caches(kv_cache)
        if (key is None) != (value is None):
            raise ValueError("Both new K and V must be supplied together")
        if self._native_step(layer, query, key, value, kv_cache, attn_metadata, output):
            return output
        return self._run(layer, query, key, value, kv_cache, attn_metadata, output, write=True)

    # ------------------------------------------------------------------ native decode step
    def _native_step(self, layer, query, key, value, kv_cache, md, output) -> bool:
        """Decode-shaped batches in one native call (oscar_decode_step_v1): classification,
        plan, metadata upload, write + window, split-K decode and inverse rotation.  False
        (nothing enqueued) sends the batch down the general path."""
        if query.dtype not in (torch.bfloat16, torch.float16) or output.dtype != query.dtype:
            return False
        host = host_metadata_arrays(md)
        if host is None:
            return False
        qsl, seqs = host
        d, hq, hk = self.head_size, self.num_heads, self.num_kv_heads
        n = min(query.shape[0], md.num_actual_tokens)
        if n <= 0 or len(qsl) < 2 or len(seqs) < len(qsl) - 1:
            return False
        if not (query.is_contiguous() and output.is_contiguous()) or query.numel() // (hq * d) < n:
            return False
        has_new = key is not None
        if has_new and self._oscar.window_enabled:
            self._ensure_staging(layer, kv_cache)
        stream = torch.cuda.current_stream(query.device).cuda_stream
        scratch = ops.DeviceScratch.get(query.device, stream)
        a = self._step_args(layer, query.device, query.dtype)
        if a is None:
            return False
        a.query, a.output, a.num_tokens = query.data_ptr(), output.data_ptr(), n
        if has_new:
            if key.stride(-1) != 1 or value.stride(-1) != 1 or key.stride(0) != value.stride(0) \
                    or key.shape[0] < n or value.shape[0] < n:
                return False
            slots = md.slot_mapping
            if slots.dtype != torch.int64 or not slots.is_contiguous() or slots.device != query.device:
                slots = slots.to(device=query.device, dtype=torch.int64).contiguous()
            a.key, a.value, a.kv_stride_token = key.data_ptr(), value.data_ptr(), key.stride(0)
            a.slot_mapping = slots.data_ptr()
            window = self._stage(layer) is not None
            a.stage_mode = STAGE_WRITE if window else (
                STAGE_INVALIDATE if getattr(layer, "_oscar_stage_ready", False) else STAGE_NONE)
            ws = scratch.store_workspace(
                _lib.load().oscar_store_workspace_bytes_v1(n, hk, d))
            a.store_workspace, a.store_workspace_bytes = ws.data_ptr(), ws.numel()
        else:
            a.key = a.value = a.slot_mapping = None
        table = _block_tables(md)
        if table.dtype != torch.int32 or table.stride(-1) != 1 or table.device != query.device:
            table = table.to(device=query.device, dtype=torch.int32).contiguous()
        if table.ndim != 2:
            raise ValueError("Missing request block-table rows")
        a.block_table, a.block_table_stride = table.data_ptr(), table.stride(0)
        a.block_table_rows, a.block_table_cols = table.shape
        a.host_query_start_loc, a.host_seq_lens = _address(qsl), _address(seqs)
        a.num_reqs = len(qsl) - 1
        ctx = ops.DeviceContext.get(query.device)
        ws = scratch.step_workspace(0)  # shared by every layer: the stream's current buffer
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        rc = ops.decode_step(ctx, a, stream, scratch)
        if rc != 0:
            return False
        if n < query.shape[0]:
            output[n:].zero_()
        self._oscar_stats["reads"] += 1
        if has_new:
            self._oscar_stats["writes"] += 1
            self._oscar_stats["kv_bytes_written"] += n * hk * 160
        return True

    def _step_args(self, layer, device, dtype):
        """The layer's step arguments that stay fixed from call to call (caches, window
        arena, rotations, settings, scratch), rebuilt only when one of them changes."""
        d, hk = self.head_size, self.num_kv_heads
        rk, rv = self._layer_rots(layer, device)
        stage = self._stage(layer)
        scratch = ops.DeviceScratch.get(device)
        bs = self.key_cache.shape[1]
        seats = 0 if stage is None else stage[2].shape[0] * bs
        slot_claims, seat_claims = scratch.claims(self.key_cache.shape[0] * bs, seats)
        arrivals = scratch.store_arrivals(hk)
        key = (self.key_cache.data_ptr(), self.value_cache.data_ptr(), rk.data_ptr(), rv.data_ptr(),
               None if stage is None else stage[2].data_ptr(), dtype, slot_claims.data_ptr(),
               seat_claims.data_ptr(), arrivals.data_ptr())
        cached = getattr(layer, "_oscar_step", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        from ._lib import StepArgs

        a = StepArgs()
        a.cache = ops.cache_struct(self.key_cache, self.value_cache, d)
        keep = [rk, rv]
        if stage is not None:
            st = ops.staging_struct(stage, self.key_cache, d)
            keep.append(st)
            a.staging = ctypes_pointer(st)
            a.sink_tokens_eff, a.recent_tokens = self.sink_eff, self._oscar.recent_tokens
        a.num_q_heads = self.num_heads
        a.q_dtype = ops.dtype_code(dtype)
        a.rk, a.rv = rk.data_ptr(), rv.data_ptr()
        a.k_clip_ratio, a.v_clip_ratio = self._oscar.k_clip_ratio, self._oscar.v_clip_ratio
        a.scale = float(self.scale)
        a.slot_claims, a.seat_claims = slot_claims.data_ptr(), seat_claims.data_ptr()
        a.epoch_counter = scratch.epoch_counter.data_ptr()
        a.arrivals = arrivals.data_ptr()
        layer._oscar_step = (key, a, keep)
        return a

    def _streaming_attention(self, layer, query, key, value, kv_cache, metadata, output):
        """backend.py:334-393: the read alone (the history and window are the state)."""
        return self._run(layer, query, key, value, kv_cache, metadata, output, write=False)

    def _run(self, layer, query, key, value, kv_cache, md, output, *, write):
        if (key is None) != (value is None):
            raise ValueError("Both new K and V must be supplied together")
        if query.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("OSCAR MI355X attention requires bf16 or fp16 queries; "
                             f"got dtype={query.dtype}")
        d, hq, hk = self.head_size, self.num_heads, self.num_kv_heads
        group = hq // hk
        dev = query.device
        q3 = query.view(-1, hq, d)
        k3 = None if key is None else key.view(-1, hk, d)
        v3 = None if value is None else value.view(-1, hk, d)
        n_md = md.num_actual_tokens
        actual = min(q3.shape[0], n_md)
        has_new = key is not None
        if write and has_new and (q3.shape[0] < n_md or k3.shape[0] < n_md or v3.shape[0] < n_md):
            raise ValueError("query/key/value hold fewer rows than num_actual_tokens")
        qsl, seqs = metadata_batch_lists(md)
        batch = _Batch.classify(qsl, seqs, actual, has_new, group)
        stage_mode = STAGE_NONE
        if write and has_new:
            if self._oscar.window_enabled:
                self._ensure_staging(layer, kv_cache)
                stage_mode = STAGE_WRITE
            elif getattr(layer, "_oscar_stage_ready", False):
                stage_mode = STAGE_INVALIDATE
        write_now = write and has_new and n_md > 0
        window = (self.sink_eff, self._oscar.recent_tokens) if self._stage(layer) is not None else (0, 0)

        # ---- host planning, then every integer array in one upload
        parts = []
        if write_now and stage_mode == STAGE_WRITE:
            store_qsl = [min(s, n_md) for s in qsl]
            parts += [np.asarray(store_qsl, np.int32), np.asarray(seqs[:len(qsl) - 1] or [0], np.int32)]
        plan, route = None, None
        if batch.short:
            route = self._decode_route(batch)
            plan = ops.plan_decode(route["qsl"], route["seqs"], has_new=has_new, num_kv_heads=hk,
                                   group=group, head_dim=d, device=dev, window=window,
                                   upload_now=False)
            parts += plan.host_parts() + route["index_parts"]
        cached_rows, cached_span = None, None
        if not batch.decode_only and (batch.short or batch.long):
            cached_span = batch.span(batch.short + batch.long)
            if cached_span is None:
                cached_rows = np.concatenate([np.arange(batch.qsl[i], batch.qsl[i + 1])
                                              for i in batch.short + batch.long]).astype(np.int64)
                parts.append(cached_rows)
        dev_parts = ops.upload(parts, dev) if parts else []
        if write_now and stage_mode == STAGE_WRITE:
            store_qsl_dev, store_seqs_dev, dev_parts = dev_parts[0], dev_parts[1], dev_parts[2:]
        if plan is not None:
            plan.adopt(dev_parts[:4])
            route["index_dev"] = dev_parts[4:4 + len(route["index_parts"])]
            dev_parts = dev_parts[4 + len(route["index_parts"]):]
        cached_rows_dev = dev_parts[0] if cached_rows is not None else None

        # ---- write
        rotated = None
        if write_now:
            slots = md.slot_mapping[:n_md].to(device=dev, dtype=torch.int64)
            extra = {}
            if stage_mode == STAGE_WRITE:
                extra = dict(qsl_dev=store_qsl_dev, seqs_dev=store_seqs_dev, num_reqs=len(qsl) - 1)
            rotated = self._store(layer, k3, v3, slots, mode=stage_mode, query=q3, outputs=True, **extra)

        # ---- read
        if actual < q3.shape[0] or actual == 0 or not (batch.decode_only and batch.covers_all):
            output.zero_()
        if actual == 0:
            return output
        out3 = output.view(-1, hq, d)
        for i in batch.fresh:
            a, b = batch.qsl[i], batch.qsl[i + 1]
            ops.attention_prefill(q3[a:b], k3[a:b], v3[a:b], self.scale, head_dim=d, out=out3[a:b])
        if not (batch.short or batch.long):
            return output
        rk, rv = self._layer_rots(layer, dev)
        if rotated is not None and rotated[0] is not None:
            q_rot, k_rot, v_rot = (t[:actual] for t in rotated)
        else:
            q_rot = ops.rotate(q3[:actual], rk)
            k_rot = None if k3 is None else ops.rotate(k3[:actual], rk)
            v_rot = None if v3 is None else ops.rotate(v3[:actual], rv)
        stage = self._stage(layer)
        table = _block_tables(md)
        out_rot = torch.empty(actual, hq, d, dtype=torch.float32, device=dev)
        lse = torch.empty(actual, hq, dtype=torch.float32, device=dev)
        if plan is not None:
            if route["identity"]:
                ops.attention_decode(q_rot, k_rot, v_rot, self.key_cache, self.value_cache, table,
                                     plan, self.scale, stage, head_dim=d, out_rot=out_rot, lse=lse)
            elif route["span"] is not None:
                i0, i1, a, b = route["span"]
                cut = (lambda t: None if t is None else t[a:b])
                ops.attention_decode(cut(q_rot), cut(k_rot), cut(v_rot), self.key_cache,
                                     self.value_cache, table[i0:i1], plan, self.scale, stage,
                                     head_dim=d, out_rot=out_rot[a:b], lse=lse[a:b])
            else:
                ids, req = route["index_dev"]
                pick = (lambda t: None if t is None else torch.index_select(t, 0, ids))
                o, l_ = ops.attention_decode(pick(q_rot), pick(k_rot), pick(v_rot), self.key_cache,
                                             self.value_cache, torch.index_select(table, 0, req),
                                             plan, self.scale, stage, head_dim=d)
                out_rot.index_copy_(0, ids, o)
                lse.index_copy_(0, ids, l_)
        if has_new:
            for i in batch.long:
                a, b = batch.qsl[i], batch.qsl[i + 1]
                ops.attention_prefill(q_rot[a:b], k_rot[a:b], v_rot[a:b], self.scale, head_dim=d,
                                      history=batch.seqs[i] - (b - a), k_cache=self.key_cache,
                                      v_cache=self.value_cache, block_table_row=table[i],
                                      stage=stage, out=out_rot[a:b], lse=lse[a:b])
        if batch.decode_only:
            ops.rotate(out_rot, rv, transpose=True, out_dtype=query.dtype, out=out3[:actual])
        elif cached_span is not None:
            _, _, a, b = cached_span
            ops.rotate(out_rot[a:b], rv, transpose=True, out_dtype=query.dtype, out=out3[a:b])
        else:
            rows = torch.index_select(out_rot, 0, cached_rows_dev)
            out3.index_copy_(0, cached_rows_dev, ops.rotate(rows, rv, transpose=True, out_dtype=query.dtype))
        self._oscar_stats["reads"] += 1
        self._last_lse = lse
        return output

    def _decode_route(self, batch: _Batch) -> dict:
        """Requests for the split-K decode (the planner cuts chunks of more than 32 rows
        per KV head into sub-requests).  A decode-only batch is planned as it is (the
        plan's request r is metadata request r: no gathers); otherwise the decode
        requests form a compact batch: the batch's own rows and block-table rows where the
        decode requests (and empty ones between them) are consecutive, as a decode-first
        batch order leaves them; gathered by row and block-table row otherwise."""
        if batch.decode_only:
            return dict(identity=True, span=None, qsl=batch.qsl, seqs=batch.seqs, index_parts=[])
        span = batch.span(batch.short)
        if span is not None:
            i0, i1, a, _ = span
            return dict(identity=False, span=span, qsl=[batch.qsl[i] - a for i in range(i0, i1 + 1)],
                        seqs=batch.seqs[i0:i1], index_parts=[])
        sub_qsl, sub_seqs, ids, req = [0], [], [], []
        for i in batch.short:
            a, b = batch.qsl[i], batch.qsl[i + 1]
            ids.extend(range(a, b))
            req.append(i)
            sub_qsl.append(sub_qsl[-1] + b - a)
            sub_seqs.append(batch.seqs[i])
        return dict(identity=False, span=None, qsl=sub_qsl, seqs=sub_seqs,
                    index_parts=[np.asarray(ids, np.int64), np.asarray(req, np.int64)])
