"""Serving seams around the OSCAR layers of one worker.

The reference hooks its worker twice (oscar_ascend/integration.py:77-245): when vLLM
sizes the KV pool, OSCAR's own device buffers are set aside first; when the pool is
allocated, every OSCAR layer is bound at once (not lazily on a first request) and one
``READY`` JSON line per rank records what was set up.  This module provides the same
two seams for the ROCm worker, built around one object:

* a :class:`Ledger` of every device buffer this backend keeps beside vLLM's pool, each
  entry tagged with how it scales -- per layer (the fp32 rotations and the FP32 window
  arena), per pool block (the last-writer slot claims and the MTP drafts' bf16 shadow
  pools), once per device (seat claims, the claim epoch, arrival counters, the static
  decode scratch, the native step's metadata ring) or transient (the largest one-layer
  workspace of a forward; layers run one after another).  :func:`plan_memory` builds it
  from the model's layers when vLLM sizes the pool and hands vLLM what it leaves;
* :func:`initialize_layers` binds the layers, allocates the per-device scratch and the
  transient workspaces up front (so the first large batch allocates nothing), measures
  what the device allocator actually gave out, checks it against the plan, and returns
  the manifest (its field names are the interface the delivery checker reads);
* :func:`validate_ready` checks a server log's manifests as the delivery checker does
  (delivery/check_ready.py:8-29): every rank present, all verified, one layer set, one
  source checkout, no failure in the log.

:func:`install_runner_hooks` wraps a worker's ``determine_available_memory`` and its
model runner's ``initialize_kv_cache_tensors`` (vLLM's GPU worker classes unless others
are passed).
"""
from __future__ import annotations

import hashlib
import json
from collections import defaultdict
from copy import deepcopy
from dataclasses import dataclass, field
from pathlib import Path

MARK = "[oscar-amd]"
READY_MARK = f"{MARK} READY "
_PACKAGE = Path(__file__).resolve().parent
_ROOT = _PACKAGE.parent

# decode partials of oscar_attn_decode_static_v1 (include/oscar_amd.h): a file-scope
# device array held on every device the library runs on
STATIC_DECODE_ITEMS = 512
# the native step's metadata ring (step.cpp): 32 slots of 64 KiB on the device
STEP_RING_BYTES = 32 * (64 << 10)
SCOPES = ("layer", "block", "device", "transient")


# ------------------------------------------------------------------ the ledger
@dataclass
class Ledger:
    """Device buffers by scope: ``layer`` and ``device`` entries are bytes held for the
    process' life, ``block`` entries are bytes per pool block, ``transient`` entries are
    alternatives of which the largest is held (one layer's forward at a time)."""

    entries: list = field(default_factory=list)  # (scope, owner, role, bytes)

    def add(self, scope: str, owner: str, role: str, nbytes: int) -> None:
        if scope not in SCOPES or nbytes < 0:
            raise ValueError(f"bad ledger entry {scope!r} {role!r} {nbytes}")
        self.entries.append((scope, owner, role, int(nbytes)))

    def total(self, scope: str) -> int:
        sizes = [b for s, _, _, b in self.entries if s == scope]
        if scope == "transient":
            # one entry per layer: layers take turns with the same workspaces
            return max(sizes, default=0)
        return sum(sizes)

    def fixed(self) -> int:
        """Bytes that do not scale with the pool: held buffers plus the transient peak."""
        return self.total("layer") + self.total("device") + self.total("transient")

    def by_role(self) -> dict:
        out = defaultdict(int)
        for scope, _, role, nbytes in self.entries:
            key = f"{scope}:{role}"
            out[key] = max(out[key], nbytes) if scope == "transient" else out[key] + nbytes
        return dict(out)


def memory_budget(available: int, native_per_block: int, shadow_per_block: int, fixed_bytes: int) -> int:
    """Pool bytes vLLM may allocate (the contract of integration.py:17-23).

    What is left after ``fixed_bytes`` holds whole blocks of ``native_per_block`` pool
    bytes, each dragging ``shadow_per_block`` bytes of this backend's per-block buffers
    along; the budget is the pool part of those blocks.  Raises when not one block fits."""
    room = available - fixed_bytes
    if native_per_block <= 0 or room <= 0:
        raise ValueError(f"OSCAR buffers ({fixed_bytes} B) leave no room for the KV pool in {available} B")
    blocks = room // (native_per_block + shadow_per_block)
    if blocks == 0:
        raise ValueError(f"OSCAR memory budget: {room} B hold no block of "
                         f"{native_per_block} + {shadow_per_block} B")
    return native_per_block * blocks


def arena_rows(cfg, block_size: int) -> int:
    """Seat rows of a layer's FP32 window arena: ceil(staging / bs) pages, and never
    fewer than the whole sink pages, the recent pages plus a page boundary, and two
    spare rows (backend.py:492-511)."""
    sink_pages = cfg.sink_tokens // block_size
    tail_pages = -(-cfg.recent_tokens // block_size) + 1
    return max(-(-cfg.staging_tokens // block_size), sink_pages + tail_pages + 2)


def layer_fixed_bytes(cfg, num_kv_heads: int, head_dim: int, block_size: int) -> int:
    """Bytes one OSCAR layer holds: R_k and R_v in fp32, and with the window on its
    arena (fp32 K and V values and an int64 owner tag per seat)."""
    rotations = 2 * head_dim * head_dim * 4
    if not cfg.window_enabled:
        return rotations
    seats = arena_rows(cfg, block_size) * block_size
    return rotations + seats * (2 * num_kv_heads * head_dim * 4 + 8)


def per_block_overhead(block_size: int) -> int:
    """Bytes per pool block outside the pool: the int64 last-writer claim of each slot
    (one table per device, shared by the layers)."""
    return 8 * block_size


def _lib_sizes():
    from . import _lib

    return _lib.load()


def decode_items_bound(max_tokens: int, max_model_len: int, num_kv_heads: int, group: int,
                       max_seqs: int = 0, target_items: int = 256) -> int:
    """Upper bound on the split-K plan's items for one batch (oscar_attn_plan_v1): at
    least the target, else per (sub-)request group at most three ranges plus one item per
    8192 keys.  Groups: a sub-request of 32 rows per KV head, at most one per request
    plus one per 32 rows of query (requests are at most max_seqs, else max_tokens)."""
    requests = max_seqs if max_seqs > 0 else max_tokens
    groups = num_kv_heads * (min(requests, max_tokens) + -(-max_tokens * group // 32))
    return max(target_items, groups * (3 + -(-max(max_model_len, max_tokens) // 8192)))


def transient_parts(impl, max_tokens: int, max_model_len: int = 0, max_seqs: int = 0) -> dict:
    """The workspaces one forward of this layer may need at once, by name: the store's
    (calls of up to max_tokens), the native step's (rotated q/k/v, out_rot, LSE and the
    item partials), the general decode's item partials, and the continuation prefill's
    (the bf16 history of up to max_model_len tokens and the partials of its split over
    max_tokens query tokens)."""
    lib = _lib_sizes()
    hq, hk, d = impl.num_heads, impl.num_kv_heads, impl.head_size
    items = decode_items_bound(max_tokens, max_model_len, hk, hq // hk, max_seqs)
    return {
        "store": lib.oscar_store_workspace_bytes_v1(max_tokens, hk, d),
        "step": lib.oscar_step_workspace_bytes_v1(max_tokens, hq, hk, d, items),
        "decode": items * 32 * (d + 1) * 4,
        "prefill": max(0, lib.oscar_prefill_workspace_bytes_v2(max(max_model_len, 0), max_tokens, hq, hk, d)),
    }


def _streaming(impls):
    return [impl for impl in impls if getattr(impl._oscar, "attention_mode", "streaming") == "streaming"]


def transient_reserve(impls, max_tokens: int, max_model_len: int = 0, max_seqs: int = 0) -> int:
    """The largest transient workspace one forward over the worker's OSCAR layers needs
    (the role of the reference's streaming_reserve, integration.py:36-62).  Layers run
    one after another and share the per-device workspaces, so this is one layer's
    worth."""
    active = _streaming(impls)
    if not active:
        return 0
    if max_tokens <= 0:
        raise ValueError("The transient reserve requires max_num_batched_tokens")
    return max(sum(transient_parts(impl, max_tokens, max_model_len, max_seqs).values()) for impl in active)


def verify_layers(layer_types, actual_ids) -> None:
    """Every FULL attention layer of the model (kinds "full_attention" / "attention" in
    ``layer_types``) is an OSCAR layer, once, and no other layer is (integration.py:65-74)."""
    full = sorted(i for i, kind in enumerate(layer_types) if kind in ("full_attention", "attention"))
    got = sorted(actual_ids)
    if not full or got != full:
        raise RuntimeError(f"Incomplete OSCAR layers: expected={full}, actual={got}")


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
                   persistent_bytes: int, transient_bytes: int, measured_bytes=None) -> dict:
    """The per-rank READY record.  The keys through ``verified`` are the delivery
    checker's interface; ``measured_bytes`` (this backend's addition) is what the device
    allocator handed out while the layers were bound, None off the GPU."""
    return {
        "rank": rank,
        "world_size": world_size,
        "layers": sorted(layers),
        "layer_ids": sorted(layer_ids),
        "shadow_layers": sorted(shadow_layers),
        "native_bytes": native_bytes,
        "persistent_bytes": persistent_bytes,
        "streaming_transient_bytes": transient_bytes,
        "measured_bytes": measured_bytes,
        "source": str(_PACKAGE),
        "sha256": source_fingerprint(),
        "verified": True,
    }


def ready_line(manifest: dict) -> str:
    return READY_MARK + json.dumps(manifest, sort_keys=True)


def _read_manifests(log: str) -> dict:
    records = {}
    for line in log.splitlines():
        _, mark, payload = line.partition(READY_MARK)
        if mark:
            record = json.loads(payload)
            records[record.get("rank")] = record
    return records


def validate_ready(log: str, expected_sha: str | None = None) -> dict:
    """The per-rank manifests of a server log, keyed by rank (the delivery checker's
    rules, delivery/check_ready.py:8-29); raises ValueError naming the first rule a log
    breaks."""
    records = _read_manifests(log)
    if not records:
        raise ValueError("No verified READY manifest in the log")
    for rank, record in sorted(records.items(), key=lambda kv: str(kv[0])):
        if record.get("verified") is not True or not record.get("layers"):
            raise ValueError(f"Unverified or empty manifest from rank {rank}")
    world = {record["world_size"] for record in records.values()}
    if len(world) != 1:
        raise ValueError(f"Ranks report different world sizes {sorted(world)}")
    ranks = set(range(world.pop()))
    if set(records) != ranks:
        raise ValueError(f"Tensor-parallel rank(s) {sorted(ranks - set(records))} sent no manifest; "
                         f"unexpected rank(s) {sorted(set(records) - ranks, key=str)}")
    layer_sets = {tuple(record["layers"]) for record in records.values()}
    if len(layer_sets) != 1:
        raise ValueError("Ranks report different layer coverage")
    want = expected_sha or records[min(records)]["sha256"]
    stale = sorted(rank for rank, record in records.items() if record["sha256"] != want)
    if stale:
        raise ValueError(f"Rank(s) {stale} run a source other than this checkout")
    if f"{MARK} injection failed" in log or "Traceback (most recent call last)" in log:
        raise ValueError("The log records an injection failure or a Python traceback")
    return records


# ------------------------------------------------------------------ worker hooks
def _oscar_impl(module):
    impl = getattr(module, "impl", None)
    return impl if getattr(impl, "_oscar_cfg", None) is not None else None


def _is_shadow(module) -> bool:
    from .mtp_shadow import is_shadow_impl

    return is_shadow_impl(getattr(module, "impl", None))


_ENGINE_RULES = (
    (lambda c: getattr(c.cache_config, "num_gpu_blocks_override", None) is not None,
     "num_gpu_blocks_override sizes the pool without OSCAR's buffers"),
    (lambda c: getattr(c.parallel_config, "data_parallel_size", 1) != 1,
     "OSCAR manifests cover data-parallel size 1 only"),
    (lambda c: getattr(c.parallel_config, "pipeline_parallel_size", 1) != 1,
     "OSCAR memory accounting covers pipeline-parallel size 1 only"),
)


def _limits(cfg) -> tuple[int, int, int]:
    sched = getattr(cfg, "scheduler_config", None)
    model = getattr(cfg, "model_config", None)
    return (getattr(sched, "max_num_batched_tokens", 0) or 0, getattr(model, "max_model_len", 0) or 0,
            getattr(sched, "max_num_seqs", 0) or 0)


def build_ledger(ctx: dict, specs: dict, cfg) -> Ledger:
    """The ledger of a runner's forward context (layer name -> module) and KV specs."""
    ledger = Ledger()
    max_tokens, max_len, max_seqs = _limits(cfg)
    oscar = []
    block_size = seat_bytes = arrivals = 0
    for name, module in ctx.items():
        spec = specs[name]
        if _is_shadow(module):
            width = spec.head_size + (getattr(spec, "head_size_v", None) or spec.head_size)
            ledger.add("block", name, "mtp shadow pool", spec.block_size * spec.num_kv_heads * width * 2)
            continue
        impl = _oscar_impl(module)
        if impl is None:
            continue
        oscar.append(impl)
        c, bs = impl._oscar, spec.block_size
        ledger.add("layer", name, "rotations", 2 * impl.head_size ** 2 * 4)
        if c.window_enabled:
            seats = arena_rows(c, bs) * bs
            ledger.add("layer", name, "window arena", seats * (2 * impl.num_kv_heads * impl.head_size * 4 + 8))
            seat_bytes = max(seat_bytes, 8 * seats)
        block_size = max(block_size, bs)
        arrivals = max(arrivals, 2 * 64 * impl.num_kv_heads * 4)
        ledger.add("transient", name, "workspaces", sum(transient_parts(impl, max_tokens, max_len, max_seqs).values())
                   if getattr(c, "attention_mode", "streaming") == "streaming" else 0)
    if oscar:
        if max_tokens <= 0:
            raise ValueError("The transient reserve requires max_num_batched_tokens")
        ledger.add("block", "device", "slot claims", per_block_overhead(block_size))
        ledger.add("device", "device", "seat claims", seat_bytes)
        ledger.add("device", "device", "claim epoch and arrival counters", 16 + arrivals)
        ledger.add("device", "device", "static decode scratch", STATIC_DECODE_ITEMS * 32 * 257 * 4)
        ledger.add("device", "device", "step metadata ring", STEP_RING_BYTES)
    return ledger


def plan_memory(runner, available: int, kv_cache_utils=None) -> dict:
    """The memory plan of a runner: native pool bytes per block (from a provisional
    cache config of vLLM's), the ledger of this backend's buffers, and the budget."""
    cfg = runner.vllm_config
    for broken, why in _ENGINE_RULES:
        if broken(cfg):
            raise ValueError(why)
    ctx = runner.compilation_config.static_forward_context
    if kv_cache_utils is None:
        from vllm.v1.core import kv_cache_utils
    specs = deepcopy(runner.get_kv_cache_spec())
    groups = kv_cache_utils.get_kv_cache_groups(cfg, deepcopy(specs))
    provisional = kv_cache_utils.get_kv_cache_config_from_groups(cfg, groups, available)
    if provisional.num_blocks < 1:
        raise ValueError("Not one native cache block fits the available memory")
    native = sum(t.size for t in provisional.kv_cache_tensors) // provisional.num_blocks
    ledger = build_ledger(ctx, specs, cfg)
    shadow = sum(b for s, _, role, b in ledger.entries if s == "block" and role == "mtp shadow pool")
    claims = ledger.total("block") - shadow
    budget = memory_budget(available, native, ledger.total("block"), ledger.fixed())
    return {"available": available, "native": native, "shadow": shadow, "claims_per_block": claims,
            "fixed": ledger.fixed(), "budget": budget, "streaming_transient_bytes": ledger.total("transient"),
            "ledger": ledger.by_role()}


def _nbytes(*tensors) -> int:
    return sum(t.numel() * t.element_size() for t in tensors)


def _allocated(device) -> int | None:
    import torch

    if device.type != "cuda":
        return None
    torch.cuda.synchronize(device)
    return torch.cuda.memory_allocated(device)


def _warm_gathers(dev) -> None:
    """torch loads a kernel's code object at the kernel's first launch (about 0.1 s for its
    indexing kernels): launch the row gathers and scatters of the mixed-batch route (a
    batch whose decode requests are not consecutive) once at initialization instead."""
    import torch

    idx = torch.zeros(1, dtype=torch.int64, device=dev)
    for dt in (torch.float32, torch.bfloat16, torch.float16, torch.int32):
        t = torch.zeros(1, 1, dtype=dt, device=dev)
        t.index_copy_(0, idx, torch.index_select(t, 0, idx))


def reserve_device_scratch(impls, caches_of, max_tokens: int, max_len: int, max_seqs: int = 0) -> int:
    """Allocate the scratch of the current stream on each layer's device (claim tables,
    epoch, arrival counters) and its workspaces at their planned sizes, so that no
    forward allocates; returns the bytes of the scratch that stays (the workspaces are
    the plan's transient reserve, counted apart)."""
    from . import ops

    touched = {}
    for impl, cache in zip(impls, caches_of):
        dev = cache[0].device
        if dev.type != "cuda":
            continue
        scratch = ops.DeviceScratch.get(dev)
        touched[id(scratch)] = scratch
        bs = cache[0].shape[1]
        seats = arena_rows(impl._oscar, bs) * bs if impl._oscar.window_enabled else 0
        scratch.claims(cache[0].shape[0] * bs, seats)
        scratch.store_arrivals(impl.num_kv_heads)
        if getattr(impl._oscar, "attention_mode", "streaming") == "streaming" and max_tokens > 0:
            parts = transient_parts(impl, max_tokens, max_len, max_seqs)
            scratch.store_workspace(parts["store"])
            scratch.attn_workspace(parts["decode"])
            scratch.prefill_workspace(parts["prefill"])
            scratch.step_workspace(parts["step"])
            ops.DeviceContext.get(dev)
            _warm_gathers(dev)
    return sum(_nbytes(s.epoch_counter, s.slot_claims, s.seat_claims, s.arrivals) for s in touched.values())


def initialize_layers(runner, config, caches) -> dict | None:
    """Bind every OSCAR layer to its caches, rotations and window arena and every MTP
    draft layer to its shadow pool, allocate the per-device scratch and workspaces,
    check what was allocated against the plan and the layer coverage against the model;
    returns the READY manifest (None without OSCAR layers)."""
    from .mtp_shadow import shadow_halves
    from .rotation import layer_index_from_name

    ctx = runner.compilation_config.static_forward_context
    bound = [(name, m) for name, m in ctx.items() if _oscar_impl(m) is not None]
    if not bound:
        return None
    device = caches[bound[0][0]][0].device
    before = _allocated(device)
    persistent = 0
    for name, module in bound:
        impl, cache = module.impl, caches[name]
        impl._set_caches(cache)
        persistent += _nbytes(*impl._layer_rots(module, cache[0].device))
        if impl._oscar.window_enabled:
            impl._ensure_staging(module, cache)
            persistent += _nbytes(module._oscar_stage_k, module._oscar_stage_v, module._oscar_slot_owner)
    shadows = [name for name, m in ctx.items() if _is_shadow(m)]
    for name in shadows:
        impl = ctx[name].impl
        twin = impl._shadow_kv(caches[name])
        impl.key_cache, impl.value_cache = shadow_halves(twin)
        if twin is not caches[name]:
            persistent += _nbytes(*shadow_halves(twin))
    max_tokens, max_len, max_seqs = _limits(runner.vllm_config)
    persistent += reserve_device_scratch([m.impl for _, m in bound], [caches[n] for n, _ in bound],
                                         max_tokens, max_len, max_seqs)
    after = _allocated(device)
    plan = getattr(runner, "_oscar_memory_plan", None) or {}
    native_bytes = sum(t.size for t in config.kv_cache_tensors)
    transient = plan.get("streaming_transient_bytes", 0)
    if plan and native_bytes + persistent + transient > plan["available"]:
        raise RuntimeError(f"OSCAR buffers as allocated ({persistent} B + {transient} B transient) and the "
                           f"pool ({native_bytes} B) exceed the {plan['available']} B the plan was made for")
    hf = getattr(runner.model_config, "hf_text_config", None)
    ids = [layer_index_from_name(name) for name, _ in bound]
    verify_layers(getattr(hf, "layer_types", None) or [], ids)
    try:
        import torch.distributed as dist

        rank = dist.get_rank() if dist.is_initialized() else 0
    except Exception:  # pragma: no cover - torch without distributed
        rank = 0
    return ready_manifest(rank=rank, world_size=runner.vllm_config.parallel_config.tensor_parallel_size,
                          layers=[name for name, _ in bound], layer_ids=ids, shadow_layers=shadows,
                          native_bytes=native_bytes, persistent_bytes=persistent, transient_bytes=transient,
                          measured_bytes=None if before is None else after - before)


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
    sizing, binding = worker_cls.determine_available_memory, runner_cls.initialize_kv_cache_tensors

    def determine_available_memory(worker):
        available = sizing(worker)
        runner = worker.model_runner
        if not any(_oscar_impl(m) is not None for m in runner.compilation_config.static_forward_context.values()):
            return available
        runner._oscar_memory_plan = plan = plan_memory(runner, available, kv_cache_utils)
        worker.available_kv_cache_memory_bytes = plan["budget"]
        print(f"{MARK} MEMORY " + json.dumps(plan, sort_keys=True), flush=True)
        return plan["budget"]

    def initialize_kv_cache_tensors(runner, config, *args, **kwargs):
        caches = binding(runner, config, *args, **kwargs)
        manifest = initialize_layers(runner, config, caches)
        if manifest is not None:
            print(ready_line(manifest), flush=True)
        return caches

    worker_cls.determine_available_memory = determine_available_memory
    runner_cls.initialize_kv_cache_tensors = initialize_kv_cache_tensors
    worker_cls._oscar_memory_hook = True
