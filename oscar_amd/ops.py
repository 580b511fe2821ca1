"""Torch-facing wrappers around the C ABI (include/oscar_amd.h).

PyTorch is used for device memory and streams only; every computation runs in
liboscar_amd.so.  All functions raise when the library is missing or a launch
fails; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import (GROUP_INTS, OSCAR_BF16, OSCAR_F16, OSCAR_F32, STAGE_INVALIDATE, STAGE_NONE,
                   STAGE_WRITE, WORK_INTS)

_DTYPES = {torch.float32: OSCAR_F32, torch.float16: OSCAR_F16, torch.bfloat16: OSCAR_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    return _DTYPES[dtype]


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(*tensors) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("OSCAR HIP ops need device tensors (no CPU fallback)")


def cache_struct(k_cache: torch.Tensor, v_cache: torch.Tensor, head_dim: int) -> _lib.Cache:
    """Byte view of a packed cache pair [num_blocks, block_size, Hk, D] (int8 or bf16)."""
    k8, v8 = k_cache.view(torch.uint8), v_cache.view(torch.uint8)
    if k8.ndim != 4 or v8.ndim != 4 or not k8.is_contiguous() or not v8.is_contiguous():
        raise ValueError("OSCAR requires contiguous [blocks, tokens, heads, bytes] caches")
    c = _lib.Cache()
    c.k, c.v = k8.data_ptr(), v8.data_ptr()
    c.num_blocks, c.block_size, c.num_kv_heads = k8.shape[0], k8.shape[1], k8.shape[2]
    c.head_dim = head_dim
    for i in range(3):
        c.k_stride[i] = k8.stride(i)
        c.v_stride[i] = v8.stride(i)
    return c


def staging_struct(stage, k_cache: torch.Tensor | None = None, head_dim: int | None = None) -> _lib.Staging | None:
    """The FP32 window arena (stage_k, stage_v, owner) as a C struct.  With the cache
    given, its geometry is checked against it (streaming_attention.py:55-65): owner
    [rows, block_size], values [rows, block_size, Hk, D], rows >= 1, all contiguous."""
    if stage is None:
        return None
    sk, sv, owner = stage
    if sk.dtype != torch.float32 or sv.dtype != torch.float32 or owner.dtype != torch.int64:
        raise ValueError("staging arena must be fp32 values and int64 owner tags")
    if not (sk.is_contiguous() and sv.is_contiguous() and owner.is_contiguous()):
        raise ValueError("Streaming staging tensors must be contiguous")
    if k_cache is not None:
        rows = owner.shape[0] if owner.ndim == 2 else 0
        want = (rows, k_cache.shape[1], k_cache.shape[2], head_dim)
        if rows < 1 or tuple(owner.shape) != want[:2] or tuple(sk.shape) != want or tuple(sv.shape) != want:
            raise ValueError("Invalid streaming staging geometry")
    s = _lib.Staging()
    s.stage_k, s.stage_v, s.owner, s.rows = sk.data_ptr(), sv.data_ptr(), owner.data_ptr(), owner.shape[0]
    return s


def upload(parts, device) -> list:
    """Host integer arrays (int32 / int64) to the device in ONE non-blocking copy.

    The arrays are packed at 8-byte aligned offsets into one pinned host buffer (torch's
    caching host allocator keeps the block until the copy has run, so the host never
    waits for the stream); the returned device tensors are views of one device buffer."""
    arrays = [np.ascontiguousarray(p) for p in parts]
    offsets, total = [], 0
    for a in arrays:
        if a.dtype not in (np.int32, np.int64):
            raise TypeError("upload() takes int32 or int64 arrays")
        offsets.append(total)
        total += (a.nbytes + 7) & ~7
    host = torch.empty(max(total, 8), dtype=torch.uint8, pin_memory=True)
    view = host.numpy()
    for a, o in zip(arrays, offsets):
        view[o:o + a.nbytes] = a.view(np.uint8)
    dev = host.to(device, non_blocking=True)
    out = []
    for a, o in zip(arrays, offsets):
        dt = torch.int32 if a.dtype == np.int32 else torch.int64
        out.append(dev[o:o + a.nbytes].view(dt) if a.size else torch.empty(0, dtype=dt, device=device))
    return out


class DeviceScratch:
    """Scratch of one (device, stream): last-writer claim tables, the claim epoch, the
    small store's arrival counters and the growable workspaces of the store, the decode,
    the prefill and the native step.  Work enqueued on different streams gets different
    scratch, so concurrent calls never share these buffers (each is allocated while its
    stream is current, so torch's allocator orders its reuse on that stream)."""

    _by_device: dict = {}

    def __init__(self, device: torch.device):
        self.device = device
        self.step_ws = torch.empty(0, dtype=torch.uint8, device=device)
        # claim epoch lives on the device so that captured graphs replay with fresh epochs
        self.epoch_counter = torch.zeros(2, dtype=torch.int64, device=device)
        self.slot_claims = torch.zeros(0, dtype=torch.int64, device=device)
        self.seat_claims = torch.zeros(0, dtype=torch.int64, device=device)
        self.store_ws = torch.empty(0, dtype=torch.uint8, device=device)
        self.arrivals = torch.zeros(0, dtype=torch.int32, device=device)
        self.attn_ws = torch.empty(0, dtype=torch.uint8, device=device)
        self.prefill_ws = torch.empty(0, dtype=torch.uint8, device=device)

    @classmethod
    def get(cls, device: torch.device, stream: int | None = None) -> "DeviceScratch":
        """The scratch of `device` for `stream` (a raw HIP stream handle; default: the
        device's current stream, the one the caller's work goes to)."""
        index = device.index if device.index is not None else torch.cuda.current_device()
        if stream is None:
            stream = torch.cuda.current_stream(index).cuda_stream
        key = (index, stream)
        if key not in cls._by_device:
            cls._by_device[key] = cls(torch.device("cuda", index))
        return cls._by_device[key]

    def claims(self, slots: int, seats: int):
        """Claim tables; growing one restarts both tables and the epoch from zero."""
        grow = self.slot_claims.numel() < slots or self.seat_claims.numel() < max(seats, 1)
        if grow:
            self.slot_claims = torch.zeros(max(slots, self.slot_claims.numel()), dtype=torch.int64,
                                           device=self.device)
            self.seat_claims = torch.zeros(max(seats, 1, self.seat_claims.numel()), dtype=torch.int64,
                                           device=self.device)
            self.epoch_counter.zero_()
        return self.slot_claims, self.seat_claims

    def store_workspace(self, nbytes: int) -> torch.Tensor:
        if self.store_ws.numel() < nbytes:
            self.store_ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
        return self.store_ws

    def store_arrivals(self, num_kv_heads: int) -> torch.Tensor:
        """Arrival counters of the one-launch store (calls of <= 64 tokens): zeroed
        once, and every call leaves them zero."""
        need = 2 * 64 * num_kv_heads
        if self.arrivals.numel() < need:
            self.arrivals = torch.zeros(need, dtype=torch.int32, device=self.device)
        return self.arrivals

    def prefill_workspace(self, nbytes: int) -> torch.Tensor:
        if self.prefill_ws.numel() < nbytes:
            self.prefill_ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
        return self.prefill_ws

    def attn_workspace(self, nbytes: int) -> torch.Tensor:
        if self.attn_ws.numel() < nbytes:
            self.attn_ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
        return self.attn_ws

    def step_workspace(self, nbytes: int) -> torch.Tensor:
        """The native decode step's workspace (rotated q / k / v, out_rot, LSE, item
        partials)."""
        if self.step_ws.numel() < max(nbytes, 1):  # never hand out an empty buffer
            self.step_ws = torch.empty(max(nbytes, 4 << 20), dtype=torch.uint8, device=self.device)
        return self.step_ws


class DeviceContext:
    """The library's native context for one device (pinned + device metadata ring of the
    decode step, safe to share between streams: a ring slot is reused once the event
    recorded after its last reader has completed), created once per device and
    destroyed with the process."""

    _by_device: dict = {}

    def __init__(self, index: int):
        lib = _lib.load()
        ptr = C.c_void_p()
        _lib.check(lib.oscar_context_create_v1(index, C.byref(ptr)), "oscar_context_create_v1")
        self.ptr = ptr
        self.index = index

    @classmethod
    def get(cls, device: torch.device) -> "DeviceContext":
        index = device.index if device.index is not None else torch.cuda.current_device()
        ctx = cls._by_device.get(index)
        if ctx is None:
            ctx = cls._by_device[index] = cls(index)
        return ctx


def decode_step(ctx: DeviceContext, args: "_lib.StepArgs", stream: int, scratch: DeviceScratch) -> int:
    """oscar_decode_step_v1; grows the stream's step workspace and retries once when it
    is too small.  Returns 0, or STEP_NOT_DECODE when the batch needs the general path."""
    lib = _lib.load()
    rc = lib.oscar_decode_step_v1(ctx.ptr, C.byref(args), C.c_void_p(stream))
    if rc == -28 and args.workspace_needed > args.workspace_bytes:
        ws = scratch.step_workspace(args.workspace_needed)
        args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
        rc = lib.oscar_decode_step_v1(ctx.ptr, C.byref(args), C.c_void_p(stream))
    if rc < 0:
        _lib.check(rc, "oscar_decode_step_v1")
    return rc


# ------------------------------------------------------------------------ store
def store(key, value, k_cache, v_cache, slot_mapping, **kw):
    """Rotate + clip + INT2 quantize + scatter (+ staging window) in one C call.

    key/value [N, Hk, D] (bf16/fp16/fp32), slot_mapping [N] int64 (negative = skip).
    rk/rv fp32 [D, D] or None for identity.  Optional query [N, Hq, D] and
    *_rot outputs receive the unclipped rotated values in the input dtype.  Keyword
    arguments as store_args.
    """
    args = store_args(key, value, k_cache, v_cache, slot_mapping, **kw)
    if args is not None:
        _lib.check(_lib.load().oscar_store_v1(C.byref(args[0]), C.c_void_p(_stream(key.device))), "oscar_store_v1")


def store_args(key, value, k_cache, v_cache, slot_mapping, *, head_dim, rk=None, rv=None,
               k_clip=0.0, v_clip=0.0, stage=None, stage_mode=STAGE_NONE, qsl_dev=None,
               seqs_dev=None, num_reqs=0, recent_tokens=0, sink_tokens_eff=0, query=None,
               query_rot=None, key_rot=None, value_rot=None):
    """The C arguments of a store (None for an empty call) and the tensors they point
    into, for oscar_store_v1 (store) or oscar_decode_write_v1 (attention_decode's
    `store`)."""
    _require_cuda(key, value, k_cache, v_cache, slot_mapping)
    n = slot_mapping.shape[0]
    if n == 0:
        return None
    lib = _lib.load()
    dev = key.device
    hk = k_cache.shape[2]
    if key.dtype not in _DTYPES or value.dtype != key.dtype:
        raise ValueError("key/value must share a float dtype")
    key = key[:n].reshape(n, hk, head_dim)
    value = value[:n].reshape(n, hk, head_dim)
    if key.stride(2) != 1 or key.stride(1) != head_dim or value.stride(2) != 1 or value.stride(1) != head_dim:
        key, value = key.contiguous(), value.contiguous()
    slot_mapping = slot_mapping.to(device=dev, dtype=torch.int64).contiguous()
    scratch = DeviceScratch.get(dev)
    cache = cache_struct(k_cache, v_cache, head_dim)
    st = staging_struct(stage, k_cache, head_dim)
    seats = 0 if st is None else st.rows * cache.block_size
    slot_claims, seat_claims = scratch.claims(cache.num_blocks * cache.block_size, seats)
    a = _lib.StoreArgs()
    a.key, a.value = key.data_ptr(), value.data_ptr()
    a.kv_dtype = _DTYPES[key.dtype]
    a.num_tokens = n
    a.key_stride_token, a.value_stride_token = key.stride(0), value.stride(0)
    if query is not None:
        query = query[:n]
        if query.stride(-1) != 1 or query.stride(-2) != head_dim:
            query = query.contiguous()
        a.query, a.num_q_heads, a.query_stride_token = query.data_ptr(), query.shape[1], query.stride(0)
    for name, r in (("rk", rk), ("rv", rv)):
        if r is not None:
            if r.dtype != torch.float32 or not r.is_contiguous() or r.shape != (head_dim, head_dim):
                raise ValueError(f"{name} must be a contiguous fp32 [{head_dim}, {head_dim}] tensor")
            setattr(a, name, r.data_ptr())
    a.k_clip_ratio, a.v_clip_ratio = float(k_clip), float(v_clip)
    a.slot_mapping = slot_mapping.data_ptr()
    a.cache = cache
    a.stage_mode = stage_mode if st is not None else STAGE_NONE
    if st is not None:
        a.staging = st
    if stage_mode == STAGE_WRITE:
        a.query_start_loc, a.seq_lens = qsl_dev.data_ptr(), seqs_dev.data_ptr()
        a.num_reqs, a.recent_tokens, a.sink_tokens_eff = num_reqs, recent_tokens, sink_tokens_eff
    for name, t in (("query_rot", query_rot), ("key_rot", key_rot), ("value_rot", value_rot)):
        if t is not None:
            if not t.is_contiguous() or t.dtype != key.dtype:
                raise ValueError(f"{name} must be contiguous in the key dtype")
            setattr(a, name, t.data_ptr())
    a.slot_claims, a.seat_claims = slot_claims.data_ptr(), seat_claims.data_ptr()
    a.epoch_counter = scratch.epoch_counter.data_ptr()
    if n >= 1 << 24:
        raise ValueError("oscar store: at most 2^24 tokens per call")
    need = lib.oscar_store_workspace_bytes_v1(n, hk, head_dim)
    ws = scratch.store_workspace(need)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    a.arrivals = scratch.store_arrivals(hk).data_ptr()
    return a, (key, value, slot_mapping, query, st, ws)


# ------------------------------------------------------------------------ rotate
def rotate(x: torch.Tensor, r: torch.Tensor, *, transpose=False, out_dtype=None, out=None):
    """x [..., D] @ R (or @ R^T) with MFMA hi/lo products; returns out_dtype (default x dtype)."""
    _require_cuda(x, r)
    d = x.shape[-1]
    rows = x.numel() // d
    x2 = x.reshape(rows, d)
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    out_dtype = out_dtype or x.dtype
    if out is None:
        out = torch.empty(*x.shape[:-1], d, dtype=out_dtype, device=x.device)
    o2 = out.reshape(rows, d)
    a = _lib.RotateArgs()
    a.x, a.x_dtype, a.rows, a.x_stride_row = x2.data_ptr(), _DTYPES[x2.dtype], rows, x2.stride(0)
    a.r, a.transpose = r.contiguous().data_ptr(), int(bool(transpose))
    a.out, a.out_dtype, a.out_stride_row, a.head_dim = o2.data_ptr(), _DTYPES[out_dtype], o2.stride(0), d
    lib = _lib.load()
    _lib.check(lib.oscar_rotate_v1(C.byref(a), C.c_void_p(_stream(x.device))), "oscar_rotate_v1")
    return out


# ------------------------------------------------------------------------ decode attention
@dataclass
class DecodePlan:
    """A split-K plan: host records (items, groups) and, once uploaded, their device copies."""
    host_items: np.ndarray   # int32 [num_items * WORK_INTS]
    host_groups: np.ndarray  # int32 [num_groups * GROUP_INTS]
    host_qsl: list
    host_seqs: list
    has_new: bool
    num_items: int
    num_groups: int
    partial_bytes: int
    max_group_items: int
    items: torch.Tensor | None = None   # device int32 copies
    groups: torch.Tensor | None = None
    qsl: torch.Tensor | None = None
    seqs: torch.Tensor | None = None

    def host_parts(self) -> list:
        """The arrays the kernels read, in upload() order (items, groups, qsl, seqs)."""
        return [self.host_items, self.host_groups, np.asarray(self.host_qsl, np.int32),
                np.asarray(self.host_seqs or [0], np.int32)]

    def adopt(self, device_parts: list) -> "DecodePlan":
        self.items, self.groups, self.qsl, self.seqs = device_parts
        return self


def plan_decode(qsl: list, seqs: list, *, has_new: bool, num_kv_heads: int, group: int,
                head_dim: int, device, target_items: int | None = None,
                chunk_tokens: int = 8192, window: tuple = (0, 0), upload_now: bool = True) -> DecodePlan:
    """Split-K plan (host): items of whole 32-token tiles, balanced over the CUs.

    window = (sink_tokens, recent_tokens) of the FP32 staging window, a balance hint
    (the expected window tiles go to items of their own); (0, 0) = no window.
    upload_now=False leaves the device copies to the caller (one combined upload()).
    """
    lib = _lib.load()
    nreq = len(seqs)
    qa = (C.c_int32 * (nreq + 1))(*qsl)
    sa = (C.c_int32 * max(nreq, 1))(*seqs)
    if target_items is None:
        target_items = cu_count(device)
    plan = _lib.Plan()
    sink, recent = (int(x) for x in window)
    # one call with room for any plan the target allows (at most 3 ranges per group,
    # at most 256 tiles per item); a second, exact call only if that was too small
    sub = max(1, 32 // group)  # query tokens per sub-request (32 rows per kv head)
    ngroups = num_kv_heads * sum(-(-(b - a) // sub) for a, b in zip(qsl, qsl[1:]) if b > a)
    guess = max(target_items, 1) + 3 * ngroups + sum(-(-s // 8192) for s in seqs) * num_kv_heads
    items = np.zeros(max(guess, 1) * WORK_INTS, np.int32)
    groups = np.zeros(max(ngroups, 1) * GROUP_INTS, np.int32)
    i_ptr = items.ctypes.data_as(C.POINTER(C.c_int32))
    g_ptr = groups.ctypes.data_as(C.POINTER(C.c_int32))
    n = lib.oscar_attn_plan_v1(qa, sa, nreq, int(has_new), num_kv_heads, group, head_dim,
                               chunk_tokens, target_items, sink, recent, i_ptr, guess,
                               g_ptr, max(ngroups, 1), C.byref(plan))
    if n == -28:
        items = np.zeros(max(plan.num_items, 1) * WORK_INTS, np.int32)
        i_ptr = items.ctypes.data_as(C.POINTER(C.c_int32))
        n = lib.oscar_attn_plan_v1(qa, sa, nreq, int(has_new), num_kv_heads, group, head_dim,
                                   chunk_tokens, target_items, sink, recent, i_ptr, plan.num_items,
                                   g_ptr, max(ngroups, 1), C.byref(plan))
    if n < 0:
        _lib.check(n, "oscar_attn_plan_v1")
    p = DecodePlan(items[: plan.num_items * WORK_INTS], groups[: plan.num_groups * GROUP_INTS],
                   list(qsl), list(seqs), bool(has_new), plan.num_items, plan.num_groups,
                   plan.partial_bytes, plan.max_group_items)
    if upload_now:
        p.adopt(upload(p.host_parts(), device))
    return p


_CU_COUNT: dict = {}


def cu_count(device) -> int:
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    if key not in _CU_COUNT:
        _CU_COUNT[key] = torch.cuda.get_device_properties(key).multi_processor_count
    return _CU_COUNT[key]


def _check_table(table: torch.Tensor, plan: DecodePlan, block_size: int) -> None:
    """streaming_attention.py:48-53: the block table must cover every history."""
    if table.ndim != 2 or table.shape[0] < len(plan.host_seqs):
        raise ValueError("Missing request block-table rows")
    for a, b, seq in zip(plan.host_qsl, plan.host_qsl[1:], plan.host_seqs):
        hist = seq - (b - a) if plan.has_new else seq
        if b > a and math.ceil(hist / block_size) > table.shape[1]:
            raise ValueError("Block table cannot cover the history")


def attention_decode(q, k_new, v_new, k_cache, v_cache, block_table, plan: DecodePlan, scale,
                     stage=None, *, head_dim, out_rot=None, lse=None, phases=0, static_scratch=False,
                     store=None):
    """Rotated-domain attention over INT2 history (+ current chunk): (out_rot fp32, lse fp32).

    q (and k_new / v_new) are bf16 or fp16; history values are rounded q_dtype(fp16(x)).
    static_scratch: call oscar_attn_decode_static_v1 (item partials in the library's
    static device array, no workspace).  store: store_args(...) of the step's write, whose
    rotated outputs are q / k_new / v_new: one oscar_decode_write_v1 call runs the store
    and the decode (a small store's quantization then rides in the merge launch)."""
    _require_cuda(q, k_cache, v_cache, block_table)
    if store is not None and static_scratch:
        raise ValueError("store= goes with the workspace decode only")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("OSCAR HIP attention requires bf16 or fp16 queries")
    n, hq, _ = q.shape
    dev = q.device
    if out_rot is None:
        out_rot = torch.zeros(n, hq, head_dim, dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.full((n, hq), -math.inf, dtype=torch.float32, device=dev)
    if plan.num_items == 0 or n == 0:
        if store is not None:
            _lib.check(_lib.load().oscar_store_v1(C.byref(store[0]), C.c_void_p(_stream(dev))), "oscar_store_v1")
        return out_rot, lse
    if q.stride(2) != 1 or q.stride(1) != head_dim:
        q = q.contiguous()
    if (k_new is None) != (v_new is None):
        raise ValueError("Both new K and V must be supplied together")
    if k_new is not None:
        if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
            raise ValueError("Current K/V must match the query dtype")
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    table = block_table.to(device=dev, dtype=torch.int32)
    if table.stride(1) != 1:
        table = table.contiguous()
    if plan.has_new != (k_new is not None):
        raise ValueError("plan and call disagree on the presence of current K/V")
    if plan.items is None:
        raise ValueError("the decode plan has not been uploaded")
    _check_table(table, plan, k_cache.shape[1])
    st = staging_struct(stage, k_cache, head_dim)
    a = _lib.AttnArgs()
    a.q, a.num_tokens, a.num_q_heads, a.q_stride_token = q.data_ptr(), n, hq, q.stride(0)
    if k_new is not None:
        a.k_new, a.v_new, a.kv_new_stride_token = k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0)
    a.cache = cache_struct(k_cache, v_cache, head_dim)
    a.block_table, a.block_table_stride = table.data_ptr(), table.stride(0)
    a.block_table_rows, a.block_table_cols = table.shape
    a.query_start_loc, a.seq_lens, a.num_reqs = plan.qsl.data_ptr(), plan.seqs.data_ptr(), plan.seqs.numel()
    if st is not None:
        a.staging = C.pointer(st)
    a.scale = float(scale)
    a.items, a.num_items = plan.items.data_ptr(), plan.num_items
    a.groups, a.num_groups = plan.groups.data_ptr(), plan.num_groups
    if not static_scratch:
        ws = DeviceScratch.get(dev).attn_workspace(plan.partial_bytes)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    a.max_group_items = plan.max_group_items
    a.out_rot, a.lse = out_rot.data_ptr(), lse.data_ptr()
    a.phases = int(phases)
    a.q_dtype = _DTYPES[q.dtype]
    lib = _lib.load()
    if store is not None:
        _lib.check(lib.oscar_decode_write_v1(C.byref(store[0]), C.byref(a), C.c_void_p(_stream(dev))),
                   "oscar_decode_write_v1")
        return out_rot, lse
    entry = "oscar_attn_decode_static_v1" if static_scratch else "oscar_attn_decode_v1"
    _lib.check(getattr(lib, entry)(C.byref(a), C.c_void_p(_stream(dev))), entry)
    return out_rot, lse


# ------------------------------------------------------------------------ prefill
def attention_prefill(q, k, v, scale, *, head_dim, history=0, k_cache=None, v_cache=None,
                      block_table_row=None, stage=None, out=None, lse=None, split=True):
    """Causal GQA prefill of one request.

    q/k/v are bf16 or fp16 (history values rounded q_dtype(fp16(x))).
    history == 0: original-domain fresh-only prefill, returns [n, Hq, D] in q's dtype.
    history > 0: rotated continuation over the packed history, returns fp32 out_rot
    (and fills lse [n, Hq] when given).
    split: cut the query tiles' key ranges into balanced chunks (a larger workspace for
    their partials and one merge launch); False runs one workgroup per query tile.
    """
    _require_cuda(q, k, v)
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("OSCAR HIP prefill requires bf16 or fp16 q/k/v of one dtype")
    n, hq, _ = q.shape
    hk = k.shape[1]
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if out is None:
        out = torch.empty(n, hq, head_dim, dtype=q.dtype if history == 0 else torch.float32,
                          device=q.device)
    a = _lib.PrefillArgs()
    a.q, a.q_stride_token, a.k, a.v, a.kv_stride_token = q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), k.stride(0)
    a.num_tokens, a.num_q_heads, a.num_kv_heads, a.head_dim = n, hq, hk, head_dim
    a.history = history
    keep = []
    if history > 0:
        a.cache = cache_struct(k_cache, v_cache, head_dim)
        row = block_table_row.to(device=q.device, dtype=torch.int32).contiguous()
        if math.ceil(history / k_cache.shape[1]) > row.numel():
            raise ValueError("Block table cannot cover the history")
        keep.append(row)
        a.block_table_row, a.block_table_cols = row.data_ptr(), row.numel()
        st = staging_struct(stage, k_cache, head_dim)
        if st is not None:
            keep.append(st)
            a.staging = C.pointer(st)
    a.scale = float(scale)
    a.out, a.out_stride_token = out.data_ptr(), out.stride(0)
    a.q_dtype = _DTYPES[q.dtype]
    if lse is not None:
        a.lse = lse.data_ptr()
    lib = _lib.load()
    # the history values plus the partials of the balanced split (0 for calls too small
    # to split and without history)
    need = lib.oscar_prefill_workspace_bytes_v2(history, n, hq, hk, head_dim)
    if need < 0:
        raise ValueError("OSCAR HIP prefill: unsupported sizes")
    if not split:
        need = lib.oscar_prefill_workspace_bytes_v1(history, hk, head_dim)
    if need > 0:
        # the size asked for, not the shared buffer's (which an earlier call may have
        # grown past v1's size: the call would then split)
        ws = DeviceScratch.get(q.device).prefill_workspace(need)
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
    _lib.check(lib.oscar_attn_prefill_v1(C.byref(a), C.c_void_p(_stream(q.device))), "oscar_attn_prefill_v1")
    return out
