"""Serving seams (oscar_amd.integration, oscar_amd.mtp_shadow) on the CPU.

Closed forms for the budget (oscar_ascend/integration.py:17-23 contract, the
reference test's figures), layer coverage, the READY-manifest rules of
delivery/check_ready.py:8-29, the transient reserve, the worker hooks driven with
stand-in worker / runner classes, and the bf16 shadow pool of MTP draft layers.
"""
import json
from types import SimpleNamespace as NS

import pytest
import torch

from oscar_amd import integration as integ
from oscar_amd.config import OscarConfig
from oscar_amd.mtp_shadow import install_shadow, is_shadow_impl, shadow_impl_class
from test_host import make_impl


def test_budget_sets_aside_fixed_buffers_and_shadow_blocks():
    # (10000 - 1000) // (100 + 25) = 72 blocks of 100 native bytes
    budget = integ.memory_budget(10000, 100, 25, 1000)
    assert budget == 7200 and budget + (budget // 100) * 25 + 1000 <= 10000
    assert integ.memory_budget(10000, 100, 0, 0) == 10000
    for args in [(100, 100, 25, 100), (1000, 0, 0, 0), (1000, 600, 500, 0)]:
        with pytest.raises(ValueError):
            integ.memory_budget(*args)


def test_layer_coverage_must_be_exact():
    integ.verify_layers(["linear_attention", "full_attention"], [1])
    integ.verify_layers(["attention", "linear_attention", "full_attention"], [2, 0])
    for types, ids in [(["full_attention"] * 2, [0]), (["full_attention"], [0, 0]),
                       (["full_attention", "linear_attention"], [1]), (["linear_attention"], [])]:
        with pytest.raises(RuntimeError):
            integ.verify_layers(types, ids)


def test_ready_manifests_are_validated_per_rank():
    record = {"rank": 0, "world_size": 2, "layers": ["layer.1"], "verified": True, "sha256": "a"}
    line = lambda r: integ.READY_MARK + json.dumps(r)
    with pytest.raises(ValueError, match="rank"):
        integ.validate_ready(line(record))  # rank 1 missing
    logs = line(record) + "\n" + line(dict(record, rank=1))
    assert len(integ.validate_ready(logs, "a")) == 2
    with pytest.raises(ValueError, match="source"):
        integ.validate_ready(logs, "stale")
    with pytest.raises(ValueError, match="coverage"):
        integ.validate_ready(line(record) + "\n" + line(dict(record, rank=1, layers=["layer.2"])))
    with pytest.raises(ValueError, match="Unverified"):
        integ.validate_ready(line(dict(record, verified=False)))
    with pytest.raises(ValueError, match="failure"):
        integ.validate_ready(logs + "\nTraceback (most recent call last):")
    with pytest.raises(ValueError, match="No verified"):
        integ.validate_ready("nothing here")


def test_fingerprint_covers_the_native_sources():
    names = {p.name for p in integ._fingerprint_files()}
    assert {"store.hip", "attn_decode.hip", "oscar_amd.h", "integration.py"} <= names
    assert len(integ.source_fingerprint()) == 64


def test_arena_rows_and_layer_bytes():
    cfg = OscarConfig()  # sink 64, recent 256, staging 8192
    assert integ.arena_rows(cfg, 128) == 64                  # ceil(8192 / 128)
    cfg.staging_tokens = 0
    assert integ.arena_rows(cfg, 128) == 0 + (2 + 1) + 2     # sink pages 0, recent 2 + 1, 2 spare
    assert integ.arena_rows(cfg, 32) == 2 + (8 + 1) + 2
    cfg = OscarConfig()
    per_seat = 2 * 1 * 256 * 4 + 8  # fp32 K and V values, int64 owner tag
    assert integ.layer_fixed_bytes(cfg, 1, 256, 128) == 2 * 256 * 256 * 4 + 64 * 128 * per_seat
    cfg.sink_tokens = cfg.recent_tokens = 0  # window off
    assert integ.layer_fixed_bytes(cfg, 1, 256, 128) == 2 * 256 * 256 * 4


def test_transient_reserve_is_one_layer_per_worker():
    impl = make_impl()
    r = integ.transient_reserve([impl], 15360, 32768)
    assert r == integ.transient_reserve([impl] * 16, 15360, 32768)
    assert r > integ.transient_reserve([impl], 1024, 32768) > 0
    # at least the prefill's bf16 history and the store workspace of the batch
    assert r >= 2 * 32768 * 1 * 256 * 2
    with pytest.raises(ValueError, match="max_num_batched_tokens"):
        integ.transient_reserve([impl], 0)


def _fixture():
    impl = make_impl(d=64, hq=2, hk=1)
    impl._oscar.staging_tokens = 64
    layer = NS(layer_name="model.layers.0.self_attn.attn", impl=impl)
    cache = [torch.zeros(8, 4, 1, 64, dtype=torch.int8) for _ in range(2)]
    return impl, layer, cache


def test_worker_hooks_budget_then_bind_layers_and_report(capsys):
    impl, layer, cache = _fixture()

    class Native:
        def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs):
            return kv_cache

    draft_impl = Native()
    install_shadow(draft_impl)
    draft_name = "model.mtp.layers.0.self_attn.attn"
    ctx = {layer.layer_name: layer, draft_name: NS(impl=draft_impl)}
    specs = {name: NS(block_size=4, num_kv_heads=1, head_size=64, head_size_v=64) for name in ctx}
    config = NS(kv_cache_tensors=[NS(size=8192)], num_blocks=8)
    kv_utils = NS(get_kv_cache_groups=lambda *a: [], get_kv_cache_config_from_groups=lambda *a: config)

    class Runner:
        compilation_config = NS(static_forward_context=ctx)
        vllm_config = NS(cache_config=NS(num_gpu_blocks_override=None),
                         parallel_config=NS(pipeline_parallel_size=1, tensor_parallel_size=1),
                         scheduler_config=NS(max_num_batched_tokens=64), model_config=NS(max_model_len=256))
        model_config = NS(hf_text_config=NS(layer_types=["full_attention"]))

        def get_kv_cache_spec(self):
            return specs

        def initialize_kv_cache_tensors(self, config):
            return {layer.layer_name: cache, draft_name: [torch.zeros(8, 4, 1, 64, dtype=torch.int8)] * 2}

    class Worker:
        model_runner = Runner()

        def determine_available_memory(self):
            return 1 << 30

    integ.install_runner_hooks(Worker, Runner, kv_utils)
    integ.install_runner_hooks(Worker, Runner, kv_utils)  # idempotent
    worker = Worker()
    budget = worker.determine_available_memory()
    plan = worker.model_runner._oscar_memory_plan
    # native 8192 / 8 = 1024 bytes per block; per block also the draft's bf16 K and V
    # (4 tokens x 64 x 2 x 2 bytes) and 8-byte claims for its 4 slots
    assert plan["native"] == 1024 and plan["shadow"] == 4 * 64 * 2 * 2 and plan["claims_per_block"] == 32
    assert budget == integ.memory_budget(1 << 30, 1024, 1024 + 32, plan["fixed"]) < 1 << 30
    assert worker.available_kv_cache_memory_bytes == budget
    caches = worker.model_runner.initialize_kv_cache_tensors(config)
    assert layer._oscar_stage_ready and impl.key_cache is cache[0]
    assert draft_impl.key_cache.dtype == torch.bfloat16
    assert draft_impl.key_cache.shape == caches[draft_name][0].shape
    out = capsys.readouterr().out
    assert "[oscar-amd] MEMORY " in out
    records = integ.validate_ready(out, integ.source_fingerprint())
    assert records[0]["layer_ids"] == [0] and records[0]["shadow_layers"] == [draft_name]
    assert records[0]["persistent_bytes"] > 0


def test_hooks_reject_budget_overrides_and_pipeline_parallelism():
    impl, layer, cache = _fixture()
    ctx = {layer.layer_name: layer}
    for cache_cfg, par in [(NS(num_gpu_blocks_override=4), NS(pipeline_parallel_size=1)),
                           (NS(num_gpu_blocks_override=None), NS(pipeline_parallel_size=2))]:
        runner = NS(compilation_config=NS(static_forward_context=ctx),
                    vllm_config=NS(cache_config=cache_cfg, parallel_config=par))
        with pytest.raises(ValueError):
            integ.plan_memory(runner, 1 << 30, NS())


def test_mtp_shadow_pool_replaces_an_int8_pool_once():
    seen = []

    class Native:
        def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs):
            seen.append(kv_cache)
            return "native"

    impl = Native()
    install_shadow(impl)
    assert is_shadow_impl(impl) and isinstance(impl, Native)
    assert shadow_impl_class(Native) is type(impl) and shadow_impl_class(type(impl)) is type(impl)
    pool = [torch.ones(3, 4, 1, 8, dtype=torch.int8)] * 2
    assert impl.forward(None, None, None, None, pool, None) == "native"
    k, v = seen[-1]
    assert k.dtype == v.dtype == torch.bfloat16 and k.shape == pool[0].shape and not k.any()
    impl.forward(None, None, None, None, pool, None)
    assert seen[-1][0] is k  # allocated once
    bf16 = [torch.ones(3, 4, 1, 8, dtype=torch.bfloat16)] * 2
    other = Native()
    install_shadow(other)
    other.forward(None, None, None, None, bf16, None)
    assert seen[-1] is bf16  # a bf16 pool goes through unchanged
    assert not is_shadow_impl(Native())
    assert not hasattr(impl, "do_kv_cache_update")  # only where the native class has it


def test_mtp_shadow_pool_keeps_a_stacked_pool_stacked_and_covers_kv_updates():
    """A stacked [2, ...] int8 pool gets a stacked bf16 twin (a native impl may unbind
    it), and do_kv_cache_update writes the draft's K/V into the twin, never the pool."""
    class Native:
        def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs):
            return kv_cache

        def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
            k_cache, v_cache = kv_cache.unbind(0)
            k_cache.view(-1, *key.shape[1:])[slot_mapping] = key
            v_cache.view(-1, *value.shape[1:])[slot_mapping] = value

    impl = Native()
    install_shadow(impl)
    pool = torch.zeros(2, 3, 4, 1, 8, dtype=torch.int8)
    twin = impl.forward(None, None, None, None, pool, None)
    assert isinstance(twin, torch.Tensor) and twin.shape == pool.shape and twin.dtype == torch.bfloat16
    key = torch.full((2, 1, 8), 1.5, dtype=torch.bfloat16)
    impl.do_kv_cache_update(None, key, -key, pool, torch.tensor([1, 6]))
    assert not pool.any()  # the int8 pool is untouched
    flat = twin.view(2, -1, 1, 8)
    assert (flat[0, [1, 6]] == 1.5).all() and (flat[1, [1, 6]] == -1.5).all() and flat[0, 0].eq(0).all()
    assert impl.forward(None, None, None, None, pool, None) is twin  # allocated once
    with pytest.raises(ValueError):
        impl.forward(None, None, None, None, torch.zeros(3, 4, 1, 8, dtype=torch.int8), None)


def test_plugin_surgery_routes_full_layers_to_oscar_and_drafts_to_the_shadow(monkeypatch):
    """The Attention.__init__ after-hook (plugin.py:73-181 role) with a stand-in
    Attention class and model config: the FULL layer's impl becomes the OSCAR impl,
    the MTP draft's impl keeps its class behind the shadow pool."""
    from oscar_amd import plugin
    from oscar_amd.backend import OscarAttentionBackendImpl

    hybrid = NS(is_hybrid=True)
    monkeypatch.setattr(plugin, "_should_oscar",
                        lambda layer, impl, model_config=None: not plugin.skip_reasons(layer, impl, hybrid))
    monkeypatch.setattr(plugin, "_wants_shadow",
                        lambda layer, model_config=None: plugin._is_mtp_draft(layer.layer_name))

    class NativeImpl:
        def __init__(self):
            self.head_size, self.num_heads, self.num_kv_heads, self.scale = 64, 2, 1, 0.125
            self.attn_type, self.sliding_window, self.sinks = "decoder", None, None
            self.key_cache = self.value_cache = None

        def forward(self, *args, **kwargs):
            return "native"

    class Attention:
        def __init__(self, layer_name):
            self.layer_name, self.impl = layer_name, NativeImpl()

    plugin._patch_attention_class(Attention)
    full = Attention("model.layers.3.self_attn.attn")
    draft = Attention("model.mtp.layers.0.self_attn.attn")
    assert isinstance(full.impl, OscarAttentionBackendImpl) and full.impl._oscar_cfg is not None
    assert is_shadow_impl(draft.impl) and isinstance(draft.impl, NativeImpl)
    assert not isinstance(draft.impl, OscarAttentionBackendImpl)
