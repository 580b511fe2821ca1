"""Serving seams around the OSCAR layers of one worker.

The reference hooks its worker twice (oscar_ascend/integration.py:77-245): when vLLM
sizes the KV cache, OSCAR's own device buffers are set aside first; when the cache is
allocated, every OSCAR layer gets its caches, rotations and FP32 window arena at once
(not lazily on a first request), the allocation is checked against the plan, the
layer coverage is verified, and one ``READY`` JSON line per rank records what was set
up.  This module provides the same seams for the ROCm worker, in three layers:

* accounting (pure functions): :func:`memory_budget`, :func:`layer_fixed_bytes`,
  :func:`per_block_overhead`, :func:`transient_reserve`, :func:`verify_layers`;
* the manifest: :func:`source_fingerprint`, :func:`ready_manifest`,
  :func:`ready_line`, :func:`validate_ready` (the delivery checker's rules,
  delivery/check_ready.py:8-29);
* :func:`install_runner_hooks`, which wraps a worker's ``determine_available_memory``
  and its model runner's ``initialize_kv_cache_tensors`` (vLLM's GPU worker classes
  unless others are passed).

The byte counts are this backend's own buffers: per layer the fp32 R_k and R_v and the
window arena (two fp32 planes plus an int64 owner tag per seat); per cache slot the
8-byte last-writer claim of calls of more than 64 tokens; per worker (layers run one
after another) the largest transient workspace of one forward.
"""
from __future__ import annotations

import hashlib
import json
from copy import deepcopy
from pathlib import Path

MARK = "[oscar-amd]"
READY_MARK = f"{MARK} READY "
_PACKAGE = Path(__file__).resolve().parent
_ROOT = _PACKAGE.parent


# ------------------------------------------------------------------ accounting
def memory_budget(available: int, native_per_block: int, shadow_per_block: int, fixed_bytes: int) -> int:
    """KV-cache bytes left to vLLM: whole blocks of (native + shadow) bytes out of what
    remains after the fixed buffers, counted at the native size (the contract of
    integration.py:17-23: errors when no block fits)."""
    if native_per_block <= 0 or available <= fixed_bytes:
        raise ValueError("Insufficient memory for OSCAR persistent buffers")
    blocks = (available - fixed_bytes) // (native_per_block + shadow_per_block)
    if blocks < 1:
        raise ValueError("OSCAR memory budget cannot hold one cache block")
    return blocks * native_per_block


def arena_rows(cfg, block_size: int) -> int:
    """Seat rows of a layer's FP32 window arena: ceil(staging / bs) pages, and never
    fewer than the whole sink pages, the recent pages plus a page boundary, and two
    spare rows (backend.py:492-511)."""
    sink_pages = cfg.sink_tokens // block_size
    tail_pages = -(-cfg.recent_tokens // block_size) + 1
    return max(-(-cfg.staging_tokens // block_size), sink_pages + tail_pages + 2)


def layer_fixed_bytes(cfg, num_kv_heads: int, head_dim: int, block_size: int) -> int:
    """Persistent bytes of one OSCAR layer: R_k and R_v (fp32), and with the window on
    the arena's K and V planes (fp32) and owner tags (int64), plus the seat claims (one
    table serves every layer of a device: counted per layer, an upper bound)."""
    total = 2 * head_dim * head_dim * 4
    if cfg.window_enabled:
        seats = arena_rows(cfg, block_size) * block_size
        total += seats * (2 * num_kv_heads * head_dim * 4 + 8 + 8)
    return total


def per_block_overhead(block_size: int) -> int:
    """Bytes per cache block outside the pool: the slot claims (int64 per slot)."""
    return 8 * block_size


def _lib_sizes():
    from . import _lib

    return _lib.load()


def transient_reserve(impls, max_tokens: int, max_model_len: int = 0) -> int:
    """Largest transient workspace of one forward over the worker's OSCAR layers
    (layers run one after another, so the worker needs one layer's worth): the store
    workspace, the step's rotated q/k/v/output, LSE and the item partials of the
    planner's upper bound of items, and the continuation prefill's bf16 history of up
    to ``max_model_len`` tokens with the partials of its split over ``max_tokens`` query
    tokens (the reference's streaming_reserve role,
    integration.py:36-62; its slab workspace knob bounds no buffer here)."""
    active = [impl for impl in impls if getattr(impl._oscar, "attention_mode", "streaming") == "streaming"]
    if not active:
        return 0
    if max_tokens <= 0:
        raise ValueError("The transient reserve requires max_num_batched_tokens")
    lib = _lib_sizes()
    best = 0
    for impl in active:
        hq, hk, d = impl.num_heads, impl.num_kv_heads, impl.head_size
        # items: one per 8192-key slab of every request's history, plus one per request
        # and head for the current chunk (upper bound for max_tokens single-token requests)
        items = (max(max_model_len, max_tokens) // 8192 + 1) * hk + max_tokens * hk
        step = lib.oscar_step_workspace_bytes_v1(max_tokens, hq, hk, d, items)
        store = lib.oscar_store_workspace_bytes_v1(max_tokens, hk, d)
        # history values plus the split prefill's partials (largest at the most tokens)
        prefill = max(0, lib.oscar_prefill_workspace_bytes_v2(max(max_model_len, 0), max_tokens, hq, hk, d))
        best = max(best, step + store + prefill)
    return best


def verify_layers(layer_types, actual_ids) -> None:
    """Every FULL attention layer of the model (kinds "full_attention" / "attention" in
    ``layer_types``) is an OSCAR layer, once, and no other layer is (integration.py:65-74)."""
    expected = {i for i, kind in enumerate(layer_types) if kind in ("full_attention", "attention")}
    ids = list(actual_ids)
    if not expected or set(ids) != expected or len(ids) != len(expected):
        raise RuntimeError(f"Incomplete OSCAR layers: expected={sorted(expected)}, actual={sorted(ids)}")


# ------------------------------------------------------------------ manifest
def _fingerprint_files():
    files = sorted(_PACKAGE.glob("*.py")) + sorted((_PACKAGE / "csrc").glob("*"))
    files += sorted((_ROOT / "include").glob("*.h"))
    return [f for f in files if f.is_file()]


def source_fingerprint() -> str:
    """sha256 over the package's Python sources, the HIP / C++ sources and the C-ABI
    header (names and bytes): a worker's manifest names the checkout it runs."""
    digest = hashlib.sha256()
    for path in _fingerprint_files():
        digest.update(str(path.relative_to(_ROOT)).encode())
        digest.update(path.read_bytes())
    return digest.hexdigest()


def ready_manifest(*, rank: int, world_size: int, layers, layer_ids, shadow_layers, native_bytes: int,
                   persistent_bytes: int, transient_bytes: int) -> dict:
    return {
        "rank": rank,
        "world_size": world_size,
        "layers": sorted(layers),
        "layer_ids": sorted(layer_ids),
        "shadow_layers": sorted(shadow_layers),
        "native_bytes": native_bytes,
        "persistent_bytes": persistent_bytes,
        "streaming_transient_bytes": transient_bytes,
        "source": str(_PACKAGE),
        "sha256": source_fingerprint(),
        "verified": True,
    }


def ready_line(manifest: dict) -> str:
    return READY_MARK + json.dumps(manifest, sort_keys=True)


def validate_ready(log: str, expected_sha: str | None = None) -> dict:
    """The verified per-rank manifests of a server log, keyed by rank; raises
    ValueError unless every tensor-parallel rank reported the same verified,
    non-empty layer set from the expected source and the log holds no failure."""
    records = {}
    for line in log.splitlines():
        if READY_MARK in line:
            record = json.loads(line.split(READY_MARK, 1)[1])
            if not record.get("verified") or not record.get("layers"):
                raise ValueError("Unverified or empty layer manifest")
            records[record["rank"]] = record
    if not records:
        raise ValueError("No verified cache initialization manifests")
    first = next(iter(records.values()))
    if set(records) != set(range(first["world_size"])):
        raise ValueError("Missing tensor-parallel rank manifests")
    for record in records.values():
        if record["world_size"] != first["world_size"] or record["layers"] != first["layers"]:
            raise ValueError("Ranks disagree about model coverage")
        if record["sha256"] != (expected_sha or first["sha256"]):
            raise ValueError("Worker source does not match this checkout")
    if f"{MARK} injection failed" in log or "Traceback (most recent call last)" in log:
        raise ValueError("Server log contains an initialization or runtime failure")
    return records


# ------------------------------------------------------------------ worker hooks
def _oscar_impl(module):
    impl = getattr(module, "impl", None)
    return impl if getattr(impl, "_oscar_cfg", None) is not None else None


def _is_shadow(module) -> bool:
    from .mtp_shadow import is_shadow_impl

    return is_shadow_impl(getattr(module, "impl", None))


def plan_memory(runner, available: int, kv_cache_utils=None) -> dict:
    """The memory plan of a runner's forward context: native bytes per block from a
    provisional cache config, the shadow pool and claim bytes per block, the fixed
    per-layer buffers and the transient reserve; returns the plan with the budget."""
    ctx = runner.compilation_config.static_forward_context
    targets = [m for m in ctx.values() if _oscar_impl(m) is not None]
    cfg = runner.vllm_config
    if getattr(cfg.cache_config, "num_gpu_blocks_override", None) is not None:
        raise ValueError("num_gpu_blocks_override bypasses OSCAR memory budgeting")
    if getattr(cfg.parallel_config, "data_parallel_size", 1) != 1:
        raise ValueError("OSCAR manifest validation supports DP=1")
    if getattr(cfg.parallel_config, "pipeline_parallel_size", 1) != 1:
        raise ValueError("OSCAR memory accounting supports PP=1")
    if kv_cache_utils is None:
        from vllm.v1.core import kv_cache_utils
    specs = deepcopy(runner.get_kv_cache_spec())
    groups = kv_cache_utils.get_kv_cache_groups(cfg, deepcopy(specs))
    provisional = kv_cache_utils.get_kv_cache_config_from_groups(cfg, groups, available)
    if provisional.num_blocks < 1:
        raise ValueError("No native cache blocks fit")
    native = sum(t.size for t in provisional.kv_cache_tensors) // provisional.num_blocks
    shadow = fixed = 0
    block_size = 0
    for name, module in ctx.items():
        spec = specs[name]
        if _is_shadow(module):
            # bf16 K and V of the draft layer for every block of the pool
            shadow += spec.block_size * spec.num_kv_heads * (spec.head_size + (spec.head_size_v or spec.head_size)) * 2
        elif (impl := _oscar_impl(module)) is not None:
            fixed += layer_fixed_bytes(impl._oscar, impl.num_kv_heads, impl.head_size, spec.block_size)
            block_size = max(block_size, spec.block_size)
    claims = per_block_overhead(block_size) if targets else 0
    sched = getattr(cfg, "scheduler_config", None)
    model = getattr(cfg, "model_config", None)
    transient = transient_reserve([_oscar_impl(m) for m in targets], getattr(sched, "max_num_batched_tokens", 0),
                                  getattr(model, "max_model_len", 0) or 0)
    fixed += transient
    budget = memory_budget(available, native, shadow + claims, fixed)
    return {"available": available, "native": native, "shadow": shadow, "claims_per_block": claims,
            "fixed": fixed, "budget": budget, "streaming_transient_bytes": transient}


def initialize_layers(runner, config, caches) -> dict | None:
    """Bind every OSCAR layer to its caches, rotations and window arena, the draft
    layers to their shadow pools; check the allocation against the plan and the layer
    coverage; returns the READY manifest (None without OSCAR layers)."""
    from .rotation import layer_index_from_name

    ctx = runner.compilation_config.static_forward_context
    names, ids, shadows = [], [], []
    persistent = 0
    for name, module in ctx.items():
        impl = getattr(module, "impl", None)
        if _oscar_impl(module) is not None:
            cache = caches[name]
            impl._set_caches(cache)
            rk, rv = impl._layer_rots(module, cache[0].device)
            persistent += rk.numel() * rk.element_size() + rv.numel() * rv.element_size()
            if impl._oscar.window_enabled:
                impl._ensure_staging(module, cache)
                persistent += sum(t.numel() * t.element_size()
                                  for t in (module._oscar_stage_k, module._oscar_stage_v, module._oscar_slot_owner))
            names.append(name)
            ids.append(layer_index_from_name(name))
        elif _is_shadow(module):
            shadow_kv = impl._shadow_kv(caches[name])
            impl.key_cache, impl.value_cache = shadow_kv
            persistent += sum(t.numel() * t.element_size() for t in shadow_kv)
            shadows.append(name)
    if not names:
        return None
    plan = getattr(runner, "_oscar_memory_plan", None) or {}
    native_bytes = sum(t.size for t in config.kv_cache_tensors)
    transient = plan.get("streaming_transient_bytes", 0)
    if plan and native_bytes + persistent + transient > plan["available"]:
        raise RuntimeError("Actual OSCAR persistent allocation exceeds the profiled budget")
    hf = getattr(runner.model_config, "hf_text_config", None)
    verify_layers(getattr(hf, "layer_types", None) or [], ids)
    try:
        import torch.distributed as dist

        rank = dist.get_rank() if dist.is_initialized() else 0
    except Exception:  # pragma: no cover - torch without distributed
        rank = 0
    return ready_manifest(rank=rank, world_size=runner.vllm_config.parallel_config.tensor_parallel_size,
                          layers=names, layer_ids=ids, shadow_layers=shadows, native_bytes=native_bytes,
                          persistent_bytes=persistent, transient_bytes=transient)


def install_runner_hooks(worker_cls=None, runner_cls=None, kv_cache_utils=None) -> None:
    """Wrap ``worker_cls.determine_available_memory`` (budget after OSCAR's buffers) and
    ``runner_cls.initialize_kv_cache_tensors`` (layer binding, checks, READY line).
    Idempotent per worker class; defaults to vLLM's GPU worker and model runner."""
    if worker_cls is None or runner_cls is None:
        from vllm.v1.worker.gpu_model_runner import GPUModelRunner
        from vllm.v1.worker.gpu_worker import Worker

        worker_cls, runner_cls = worker_cls or Worker, runner_cls or GPUModelRunner
    if getattr(worker_cls, "_oscar_memory_hook", False):
        return
    original_memory = worker_cls.determine_available_memory
    original_caches = runner_cls.initialize_kv_cache_tensors

    def determine_available_memory(worker):
        available = original_memory(worker)
        runner = worker.model_runner
        ctx = runner.compilation_config.static_forward_context
        if not any(_oscar_impl(m) is not None for m in ctx.values()):
            return available
        plan = plan_memory(runner, available, kv_cache_utils)
        runner._oscar_memory_plan = plan
        worker.available_kv_cache_memory_bytes = plan["budget"]
        print(f"{MARK} MEMORY " + json.dumps(plan, sort_keys=True), flush=True)
        return plan["budget"]

    def initialize_kv_cache_tensors(runner, config, *args, **kwargs):
        caches = original_caches(runner, config, *args, **kwargs)
        manifest = initialize_layers(runner, config, caches)
        if manifest is not None:
            print(ready_line(manifest), flush=True)
        return caches

    worker_cls.determine_available_memory = determine_available_memory
    runner_cls.initialize_kv_cache_tensors = initialize_kv_cache_tensors
    worker_cls._oscar_memory_hook = True
