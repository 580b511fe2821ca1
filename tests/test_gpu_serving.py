"""The serving seams on the GPU: rotations from a calibration checkpoint, and layers bound
by the cache-initialization hook, each driven through impl.forward against the oracle.

* A ``format_version`` 2 checkpoint in the writer's layout (tools/gen_rotations.py:228-239:
  ``layers[str(id)] = {rotation, rotation_v, eigenvalues, eigenvalues_v}``), named by
  ``OSCAR_ASCEND_K_ROTATION_PATH`` / ``OSCAR_ASCEND_V_ROTATION_PATH``, is read by the
  impl itself (rotation.py:93-129): no test injects ``_oscar_rots``.
* ``integration.plan_memory`` and ``integration.initialize_layers`` run on a stand-in
  runner with real device caches (the role of integration.py:77-245); the bound layer
  then serves a prefill and an MTP step, the MTP draft layer writes bf16 K/V through its
  shadow pool, and the manifest's byte counts are checked against what the device
  allocator handed out while the layers were bound.
"""
from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from oracle import backend as ob
from oracle import cases
from window_check import assert_window_close

pytestmark = pytest.mark.gpu

D, HQ, HK, BS = 256, 6, 1, 128


def _write_checkpoint(path, layers):
    """The calibration writer's format-2 layout: {layer id (str): {rotation, rotation_v,
    eigenvalues, eigenvalues_v}} with the recipe fields."""
    torch.save({
        "format_version": 2,
        "objective": "qqt_r_h_pbr_k / sst_r_h_pbr_v",
        "source_grouping": "layer",
        "layers": {str(i): {"rotation": torch.from_numpy(rk), "rotation_v": torch.from_numpy(rv),
                            "eigenvalues": torch.ones(D), "eigenvalues_v": torch.ones(D)}
                   for i, (rk, rv) in layers.items()},
    }, path)


def _impl():
    from oscar_amd.backend import OscarAttentionBackendImpl

    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_heads, impl.num_kv_heads, impl.scale = D, HQ, HK, D ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()  # reads OSCAR_ASCEND_* from the environment
    return impl


def _metadata(dev, slots, qsl, seqs, table):
    md = NS(num_actual_tokens=qsl[-1], slot_mapping=torch.tensor(np.asarray(slots, np.int64), device=dev),
            query_start_loc_cpu=torch.tensor(qsl), seq_lens_list=list(seqs))
    md.block_tables = torch.from_numpy(np.ascontiguousarray(table)).to(dev)
    return md


def _run_steps(impl, layer, caches, oracle_layer, table, steps, seed, dev):
    """Forward steps of two requests (new tokens per request per step) through the impl
    and the oracle; outputs within 2e-2 + one bf16 ulp, then bytes and tags equal."""
    lens = [0] * table.shape[0]
    written = ([], [])
    for step, news in enumerate(steps):
        slots, qsl, seqs = [], [0], []
        for r, n in enumerate(news):
            pos = np.arange(lens[r], lens[r] + n)
            slots += (table[r, pos // BS].astype(np.int64) * BS + pos % BS).tolist()
            qsl.append(qsl[-1] + n)
            seqs.append(lens[r] + n)
        n = qsl[-1]
        q = cases.bf16_normal((n, HQ, D), seed + step)
        k = cases.kv_outliers(n, HK, D, seed + 100 + step)
        v = cases.kv_outliers(n, HK, D, seed + 200 + step)
        written[0].append(k)
        written[1].append(v)
        out = torch.empty(n, HQ * D, dtype=torch.bfloat16, device=dev)
        tq, tk, tv = (torch.from_numpy(x).to(dev).bfloat16() for x in (q, k, v))
        impl.forward(layer, tq.view(n, -1), tk.view(n, -1), tv.view(n, -1), caches,
                     _metadata(dev, slots, qsl, seqs, table), output=out)
        torch.cuda.synchronize()
        ref = ob.forward(oracle_layer, q, k, v, slots, qsl, seqs, table)
        got = out.float().view(n, HQ, D).cpu().numpy()
        err = np.abs(got - ref)
        print(f"step {step} {news}: max|out - oracle| = {err.max():.3e}", flush=True)
        assert (err <= 2e-2 + 2.0 ** -7 * np.abs(ref)).all(), f"step {step}: output differs from the oracle"
        lens = seqs
    assert np.array_equal(caches[0].view(torch.uint8).cpu().numpy(), oracle_layer.k8)
    assert np.array_equal(caches[1].view(torch.uint8).cpu().numpy(), oracle_layer.v8)
    assert np.array_equal(layer._oscar_slot_owner.cpu().numpy(), oracle_layer.staging.owner)
    assert_window_close(layer._oscar_stage_k.cpu().numpy(), oracle_layer.staging.stage_k, written[0],
                        oracle_layer.rk, "K window")
    assert_window_close(layer._oscar_stage_v.cpu().numpy(), oracle_layer.staging.stage_v, written[1],
                        oracle_layer.rv, "V window")


def test_checkpoint_rotations_drive_the_store_and_decode(cuda, tmp_path, monkeypatch):
    """Row f2: R_k / R_v of the layer's own entry (not another layer's, not the identity)
    reach the HIP store and decode when the impl loads them from the checkpoint."""
    dev = cuda
    mats = {3: (cases.qr_rotation(D, 31), cases.qr_rotation(D, 32)),
            11: (cases.qr_rotation(D, 41), cases.hadamard_rotation(D, 42))}
    path = tmp_path / "rotations.pt"
    _write_checkpoint(path, mats)
    monkeypatch.setenv("OSCAR_ASCEND_K_ROTATION_PATH", str(path))
    monkeypatch.setenv("OSCAR_ASCEND_V_ROTATION_PATH", str(path))
    impl = _impl()
    layer = NS(layer_name="model.layers.11.self_attn.attn")
    nb = 24
    caches = [torch.zeros(nb, BS, HK, D, dtype=torch.int8, device=dev) for _ in range(2)]
    table = np.random.default_rng(43).permutation(nb).reshape(2, nb // 2).astype(np.int32)
    rk, rv = mats[11]
    oracle_layer = ob.OracleLayer(k8=np.zeros((nb, BS, HK, D), np.uint8), v8=np.zeros((nb, BS, HK, D), np.uint8),
                                  rk=rk, rv=rv, hq=HQ, hk=HK, d=D, scale=D ** -0.5)
    _run_steps(impl, layer, caches, oracle_layer, table, [(600, 300), (4, 1), (4, 4)], 500, dev)
    # the matrices the impl holds are the checkpoint's, bit for bit
    assert torch.equal(layer._oscar_rots[0].cpu(), torch.from_numpy(rk))
    assert torch.equal(layer._oscar_rots[1].cpu(), torch.from_numpy(rv))


def test_cache_initialization_binds_device_layers_and_counts_their_bytes(cuda, tmp_path, monkeypatch):
    """Row f4 on the device: plan_memory, then initialize_layers on real caches; the bound
    FULL layer serves steps that match the oracle, the MTP draft writes bf16 K/V into its
    shadow (the int8 pool stays untouched), and the manifest's persistent bytes plus the
    workspaces reserved at initialization equal the allocator's growth."""
    from oscar_amd import integration as integ
    from oscar_amd import ops
    from oscar_amd.mtp_shadow import install_shadow

    dev = cuda
    mats = {0: (cases.hadamard_rotation(D, 51), cases.qr_rotation(D, 52)),
            2: (cases.qr_rotation(D, 53), cases.qr_rotation(D, 54))}
    path = tmp_path / "rotations.pt"
    _write_checkpoint(path, mats)
    monkeypatch.setenv("OSCAR_ASCEND_K_ROTATION_PATH", str(path))
    monkeypatch.setenv("OSCAR_ASCEND_V_ROTATION_PATH", str(path))

    class Native:
        """A native bf16 attention impl: its KV update scatters bf16 rows into the pool."""

        def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs):
            return kv_cache

        def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
            kc, vc = kv_cache
            kc.view(-1, HK, D)[slot_mapping] = key
            vc.view(-1, HK, D)[slot_mapping] = value

    names = ["model.layers.0.self_attn.attn", "model.layers.2.self_attn.attn"]
    draft_name = "model.mtp.layers.0.self_attn.attn"
    ctx = {name: NS(layer_name=name, impl=_impl()) for name in names}
    draft = Native()
    install_shadow(draft)
    ctx[draft_name] = NS(layer_name=draft_name, impl=draft)
    nb = 32
    specs = {name: NS(block_size=BS, num_kv_heads=HK, head_size=D, head_size_v=D) for name in ctx}
    config = NS(kv_cache_tensors=[NS(size=2 * nb * BS * HK * D)] * len(ctx), num_blocks=nb)
    kv_utils = NS(get_kv_cache_groups=lambda *a: [], get_kv_cache_config_from_groups=lambda *a: config)
    runner = NS(compilation_config=NS(static_forward_context=ctx),
                vllm_config=NS(cache_config=NS(num_gpu_blocks_override=None),
                               parallel_config=NS(pipeline_parallel_size=1, tensor_parallel_size=1),
                               scheduler_config=NS(max_num_batched_tokens=1024, max_num_seqs=8),
                               model_config=NS(max_model_len=2048)),
                model_config=NS(hf_text_config=NS(layer_types=["full_attention", "linear_attention",
                                                               "full_attention"])),
                get_kv_cache_spec=lambda: specs)
    runner._oscar_memory_plan = plan = integ.plan_memory(runner, 8 << 30, kv_utils)
    assert plan["budget"] < 8 << 30 and plan["ledger"]["device:static decode scratch"] == 512 * 32 * 257 * 4
    caches = {name: [torch.zeros(nb, BS, HK, D, dtype=torch.int8, device=dev) for _ in range(2)] for name in ctx}
    stream = torch.cuda.Stream(dev)  # a stream of its own: scratch is per (device, stream)
    with torch.cuda.stream(stream):
        manifest = integ.initialize_layers(runner, config, caches)
        scratch = ops.DeviceScratch.get(dev)
        workspaces = sum(t.numel() for t in (scratch.store_ws, scratch.attn_ws, scratch.prefill_ws, scratch.step_ws))
        print(f"manifest: persistent {manifest['persistent_bytes']} B, measured {manifest['measured_bytes']} B, "
              f"workspaces {workspaces} B", flush=True)
        assert manifest["layer_ids"] == [0, 2] and manifest["shadow_layers"] == [draft_name]
        # torch's caching allocator rounds a small block up to 512 bytes, and a large one
        # (over 1 MiB) keeps any remainder of its segment of up to 1 MiB: the growth is the
        # exact bytes plus at most that per tensor (a missed 256 KiB rotation or 16 MiB
        # arena would not fit the slack of the small ones, nor the arena that of all)
        held_tensors = [t for name in names for t in (*ctx[name]._oscar_rots, ctx[name]._oscar_stage_k,
                                                       ctx[name]._oscar_stage_v, ctx[name]._oscar_slot_owner)]
        held_tensors += [*draft._oscar_shadow_kv, scratch.epoch_counter, scratch.slot_claims, scratch.seat_claims,
                         scratch.arrivals, scratch.store_ws, scratch.attn_ws, scratch.prefill_ws, scratch.step_ws]
        slack = sum((1 << 20) if t.numel() * t.element_size() > (1 << 20) else 511 for t in held_tensors)
        extra = manifest["measured_bytes"] - (manifest["persistent_bytes"] + workspaces)
        assert 0 <= extra <= slack, (extra, slack)
        # layer-owned bytes: rotations and window arenas of both layers, the draft's shadow
        rows = integ.arena_rows(ctx[names[0]].impl._oscar, BS)
        layer_bytes = 2 * (2 * D * D * 4 + rows * BS * (2 * HK * D * 4 + 8)) + 2 * nb * BS * HK * D * 2
        held = sum(t.numel() * t.element_size() for t in (scratch.epoch_counter, scratch.slot_claims,
                                                          scratch.seat_claims, scratch.arrivals))
        assert manifest["persistent_bytes"] == layer_bytes + held
        assert workspaces >= manifest["streaming_transient_bytes"] >= 0
        integ.validate_ready(integ.ready_line(manifest), integ.source_fingerprint())

        # the bound FULL layer 2 serves a prefill and MTP / decode steps against the oracle
        layer = ctx[names[1]]
        rk, rv = mats[2]
        assert torch.equal(layer._oscar_rots[0].cpu(), torch.from_numpy(rk))
        oracle_layer = ob.OracleLayer(k8=np.zeros((nb, BS, HK, D), np.uint8), v8=np.zeros((nb, BS, HK, D), np.uint8),
                                      rk=rk, rv=rv, hq=HQ, hk=HK, d=D, scale=D ** -0.5)
        table = np.random.default_rng(61).permutation(nb).reshape(2, nb // 2).astype(np.int32)
        _run_steps(layer.impl, layer, caches[names[1]], oracle_layer, table, [(700, 200), (4, 4), (1, 4)], 700, dev)

        # the draft writes bf16 K/V through the shadow; the int8 pool stays zero
        key = torch.full((3, HK, D), 0.5, dtype=torch.bfloat16, device=dev)
        draft.do_kv_cache_update(None, key, -key, caches[draft_name], torch.tensor([5, 77, 300], device=dev))
        torch.cuda.synchronize()
        assert not caches[draft_name][0].any() and not caches[draft_name][1].any()
        assert draft.key_cache.dtype == torch.bfloat16
        assert (draft.key_cache.view(-1, HK, D)[[5, 77, 300]] == 0.5).all()
    # nothing the steps needed outgrew the scratch reserved at initialization
    assert scratch.store_ws.numel() + scratch.attn_ws.numel() + scratch.prefill_ws.numel() + \
        scratch.step_ws.numel() == workspaces
