"""Host-side mirror of the reference plugin/impl on the CPU (no kernel launches).

Restates the reference's host tests for this path: metadata accessors
(tests/test_backend.py:112-120), class-surgery rollback (:141-157), rotation
loading (:243-251, tests/test_numeric.py:160-183 and :274-296), MTP/hybrid
routing (tests/test_numeric.py:218-246 and :369-379), configuration defaults
(tests/test_streaming_backend.py:188-197) and cache geometry checks.
"""
from types import SimpleNamespace as NS

import pytest
import torch

from oscar_amd import plugin, rotation
from oscar_amd.backend import OscarAttentionBackendImpl, metadata_batch_lists
from oscar_amd.config import OscarConfig


def meta(slots, ends, seqs):
    return NS(num_actual_tokens=len(slots), slot_mapping=torch.tensor(slots),
              query_start_loc=torch.tensor([0] + ends), actual_seq_lengths_q=ends,
              seq_lens=torch.tensor(seqs), seq_lens_cpu=torch.tensor(seqs), seq_lens_list=seqs)


def test_host_metadata_does_not_read_device_query_starts():
    class NoRead:
        def tolist(self):
            raise AssertionError("unexpected device sync")

    md = meta([0, 1], [1, 2], [9, 12])
    md.query_start_loc = NoRead()
    assert metadata_batch_lists(md) == ([0, 1, 2], [9, 12])
    md2 = NS(query_start_loc_cpu=torch.tensor([0, 3]), seq_lens=NoRead(), seq_lens_list=[7])
    assert metadata_batch_lists(md2) == ([0, 3], [7])


def test_failed_surgery_restores_class_and_state():
    class Original:
        pass

    class Broken(Original):
        def _oscar_setup(self):
            self.partial = True
            raise ValueError("unsupported")

    impl = Original()
    impl.keep = 123
    with pytest.raises(ValueError):
        plugin.install_impl(impl, Broken)
    assert type(impl) is Original and vars(impl) == {"keep": 123}


def test_config_defaults_and_validation(monkeypatch):
    for name in ("OSCAR_ASCEND_ATTENTION_MODE", "OSCAR_ASCEND_SINK_TOKENS", "OSCAR_ASCEND_GROUP_SIZE",
                 "OSCAR_ASCEND_K_CLIP_RATIO", "OSCAR_ASCEND_STAGING_TOKENS"):
        monkeypatch.delenv(name, raising=False)
    cfg = OscarConfig.from_env(head_dim=256)
    assert cfg.attention_mode == "streaming" and cfg.window_enabled
    assert (cfg.sink_tokens, cfg.recent_tokens, cfg.staging_tokens) == (64, 256, 8192)
    assert cfg.slot_bytes == 160 and cfg.data_bytes == 64
    monkeypatch.setenv("OSCAR_ASCEND_STAGING_TOKENS", "0")
    assert not OscarConfig.from_env(head_dim=256).window_enabled
    monkeypatch.setenv("OSCAR_ASCEND_K_CLIP_RATIO", "1.5")
    with pytest.raises(ValueError, match="clip"):
        OscarConfig.from_env(head_dim=256)
    monkeypatch.setenv("OSCAR_ASCEND_K_CLIP_RATIO", "0")
    monkeypatch.setenv("OSCAR_ASCEND_GROUP_SIZE", "32")
    with pytest.raises(ValueError, match="per-vector"):
        OscarConfig.from_env(head_dim=256)
    monkeypatch.setenv("OSCAR_ASCEND_GROUP_SIZE", "0")
    monkeypatch.setenv("OSCAR_ASCEND_ATTENTION_MODE", "bogus")
    with pytest.raises(ValueError):
        OscarConfig.from_env(head_dim=256)


def test_missing_rotation_layer_rejected_when_strict(tmp_path):
    path = tmp_path / "rotation.pt"
    torch.save({"layers": {"1": {"rotation": torch.eye(64)}}}, path)
    with pytest.raises(ValueError, match="missing layer"):
        rotation.get_layer_rotation(str(path), "model.layers.0.self_attn.attn", 64, "cpu", strict=True)
    r = rotation.get_layer_rotation(str(path), "model.layers.0.self_attn.attn", 64, "cpu")
    assert torch.equal(r, torch.eye(64))


def test_rotation_checkpoint_layouts(tmp_path):
    q = torch.linalg.qr(torch.randn(64, 64, dtype=torch.float64))[0].float()
    qv = torch.linalg.qr(torch.randn(64, 64, dtype=torch.float64))[0].float()
    layouts = {
        "nested": {"layers": {"model.layers.3.self_attn": {"rotation": q, "rotation_v": qv}}},
        "flat": {3: q},
        "names": {"model.layers.3.attn": q},
        "stacked": torch.stack([torch.eye(64)] * 3 + [q]),
    }
    for name, obj in layouts.items():
        path = tmp_path / f"{name}.pt"
        torch.save(obj, path)
        rk = rotation.get_layer_rotation(str(path), "model.layers.3.self_attn.attn", 64, "cpu",
                                         mode="k", strict=True)
        assert torch.equal(rk, q), name
        rv = rotation.get_layer_rotation(str(path), "model.layers.3.self_attn.attn", 64, "cpu",
                                         mode="v", strict=True)
        assert torch.equal(rv, qv if name == "nested" else q), name
    bad = tmp_path / "bad.pt"
    torch.save({3: torch.ones(64, 64)}, bad)
    with pytest.raises(ValueError, match="orthogonal"):
        rotation.get_layer_rotation(str(bad), "model.layers.3.attn", 64, "cpu", strict=True)
    torch.save({3: torch.eye(32)}, bad)
    rotation.load_rotation_table.cache_clear()
    with pytest.raises(ValueError, match="shape"):
        rotation.get_layer_rotation(str(bad), "model.layers.3.attn", 64, "cpu")


def test_layer_index_parsing():
    assert rotation.layer_index_from_name("model.layers.11.self_attn.attn") == 11
    assert rotation.layer_index_from_name("blocks_7") == 7
    assert rotation.layer_index_from_name("attn") is None


def test_should_oscar_routes_only_full_decoder_layers_of_hybrid_models():
    hybrid = NS(is_hybrid=False, hf_text_config=NS(layer_types=["linear_attention", "full_attention"]))
    dense = NS(is_hybrid=False, hf_text_config=NS(layer_types=["attention", "attention"]))
    assert plugin.hybrid_model(hybrid) and not plugin.hybrid_model(dense)
    assert plugin.hybrid_model(NS(is_hybrid=True))
    impl = NS(attn_type="decoder", sliding_window=None, sinks=None)
    full = NS(layer_name="model.layers.3.self_attn.attn")
    assert plugin._should_oscar(full, impl, hybrid)
    assert not plugin._should_oscar(NS(layer_name="model.mtp.layers.0.self_attn.attn"), impl, hybrid)
    assert not plugin._should_oscar(full, impl, dense)
    assert not plugin._should_oscar(full, NS(attn_type=NS(value="encoder"), sliding_window=None,
                                             sinks=None), hybrid)
    assert not plugin._should_oscar(full, NS(attn_type="decoder", sliding_window=128, sinks=None), hybrid)


def make_impl(d=256, hq=6, hk=1):
    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_heads, impl.num_kv_heads, impl.scale = d, hq, hk, d ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    return impl


def test_cache_geometry_checks():
    impl = make_impl()
    impl._set_caches([torch.zeros(4, 128, 1, 256, dtype=torch.int8)] * 2)    # packed
    impl = make_impl()
    impl._set_caches([torch.zeros(4, 128, 1, 256, dtype=torch.bfloat16)] * 2)  # legacy width
    impl = make_impl()
    with pytest.raises(AssertionError, match="slot width"):
        impl._set_caches([torch.zeros(4, 128, 1, 200, dtype=torch.int8)] * 2)
    impl = make_impl()
    with pytest.raises(ValueError):
        impl._set_caches(None)
    with pytest.raises(ValueError, match="divisible"):
        make_impl(hq=6, hk=4)


def test_staging_arena_geometry_matches_reference_sizing():
    impl = make_impl()
    impl._oscar.sink_tokens, impl._oscar.recent_tokens, impl._oscar.staging_tokens = 64, 256, 8192
    layer = NS()
    cache = [torch.zeros(8, 128, 1, 256, dtype=torch.int8)] * 2
    impl._ensure_staging(layer, cache)
    assert layer._oscar_stage_rows == 64 and impl.sink_eff == 0
    assert layer._oscar_stage_k.shape == (64, 128, 1, 256)
    assert (layer._oscar_slot_owner == -1).all()
    addr = layer._oscar_stage_k.data_ptr()
    impl._ensure_staging(layer, cache)
    assert layer._oscar_stage_k.data_ptr() == addr  # allocated once per layer


def test_forward_requires_output_and_paired_kv():
    impl = make_impl()
    cache = [torch.zeros(4, 128, 1, 256, dtype=torch.int8)] * 2
    q = torch.zeros(1, 6 * 256, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        impl.forward(NS(), q, None, None, cache, meta([0], [1], [1]), output=None)
    out = torch.ones(1, 6 * 256, dtype=torch.bfloat16)
    assert (impl.forward(NS(), q, None, None, cache, None, output=out) == 0).all()
    with pytest.raises(ValueError, match="together"):
        impl.forward(NS(), q, torch.zeros(1, 256, dtype=torch.bfloat16), None, cache,
                     meta([0], [1], [1]), output=out)


def test_native_step_reads_host_metadata_in_the_accessor_order():
    from oscar_amd.backend import host_metadata_arrays

    md = NS(query_start_loc_cpu=torch.tensor([0, 4, 5], dtype=torch.int32),
            seq_lens_list=[100, 7], seq_lens_cpu=torch.tensor([1, 1], dtype=torch.int32))
    qsl, seqs = host_metadata_arrays(md)
    assert qsl.data_ptr() == md.query_start_loc_cpu.data_ptr()   # zero-copy int32 tensor
    assert list(seqs) == [100, 7]                                 # seq_lens_list first
    md2 = NS(actual_seq_lengths_q=[4, 5], seq_lens_cpu=torch.tensor([9, 8]))
    qsl, seqs = host_metadata_arrays(md2)
    assert list(qsl) == [0, 4, 5] and seqs.dtype == torch.int32 and seqs.tolist() == [9, 8]
    # device-only metadata: the native step is skipped (reading it would synchronise)
    assert host_metadata_arrays(NS(query_start_loc=torch.tensor([0, 1]), seq_lens=torch.tensor([3]))) is None


def _plan(qsl, seqs, has_new):
    import numpy as np

    from oscar_amd.ops import DecodePlan

    return DecodePlan(np.zeros(0, np.int32), np.zeros(0, np.int32), list(qsl), list(seqs), has_new,
                      0, 0, 0, 0)


def test_general_path_table_check_raises_like_the_reference():
    """ops._check_table restates streaming_attention.py:48-53: a row per request, and
    ceil(history / block_size) columns where the history is seq minus the chunk when
    new K/V come with the queries (seq alone otherwise); requests without queries in
    the batch read nothing."""
    from oscar_amd.ops import _check_table

    table = torch.zeros(2, 16, dtype=torch.int32)
    _check_table(table, _plan([0, 4, 8], [2052, 2052], True), 128)      # 2048 = 16 pages
    _check_table(table, _plan([0, 4, 4], [2052, 99999], True), 128)     # second request idle
    _check_table(table, _plan([0, 1, 2], [2048, 1], False), 128)
    with pytest.raises(ValueError, match="Block table cannot cover the history"):
        _check_table(table, _plan([0, 4, 8], [2052, 2053], True), 128)
    with pytest.raises(ValueError, match="Block table cannot cover the history"):
        _check_table(table, _plan([0, 1, 2], [2049, 1], False), 128)
    with pytest.raises(ValueError, match="Missing request block-table rows"):
        _check_table(table[:1], _plan([0, 4, 8], [100, 100], True), 128)
    with pytest.raises(ValueError, match="Missing request block-table rows"):
        _check_table(table[0], _plan([0, 4], [100], True), 128)


def test_staging_struct_checks_the_arena_against_the_cache():
    """ops.staging_struct restates streaming_attention.py:55-65: owner [rows, bs], values
    [rows, bs, Hk, D] fp32, rows >= 1, all contiguous."""
    from oscar_amd.ops import staging_struct

    kc = torch.zeros(8, 32, 2, 64, dtype=torch.int8)
    good = (torch.zeros(4, 32, 2, 64), torch.zeros(4, 32, 2, 64), torch.full((4, 32), -1, dtype=torch.int64))
    assert staging_struct(good, kc, 64).rows == 4
    assert staging_struct(None, kc, 64) is None
    bad = {
        "rows": (torch.zeros(0, 32, 2, 64), torch.zeros(0, 32, 2, 64), torch.zeros(0, 32, dtype=torch.int64)),
        "block size": (torch.zeros(4, 16, 2, 64), torch.zeros(4, 16, 2, 64), torch.zeros(4, 16, dtype=torch.int64)),
        "heads": (torch.zeros(4, 32, 1, 64), torch.zeros(4, 32, 1, 64), good[2]),
        "head_dim": (torch.zeros(4, 32, 2, 32), good[1], good[2]),
        "owner rows": (good[0], good[1], torch.zeros(3, 32, dtype=torch.int64)),
        "v shape": (good[0], torch.zeros(4, 32, 2, 65), good[2]),
    }
    for what, stage in bad.items():
        with pytest.raises(ValueError, match="Invalid streaming staging geometry"):
            staging_struct(stage, kc, 64)
    with pytest.raises(ValueError, match="contiguous"):
        staging_struct((good[0].transpose(0, 1), good[1], good[2]), kc, 64)
    with pytest.raises(ValueError, match="fp32"):
        staging_struct((good[0].half(), good[1], good[2]), kc, 64)


def test_mixed_batch_routes_slice_consecutive_decodes_and_gather_otherwise():
    """A batch with a continuation chunk or a fresh prefill sends its short requests to the
    split-K decode: as a slice of the batch's rows and block-table rows when they (and empty
    requests between them) are consecutive, by gathers otherwise (backend.py:334-393 routing)."""
    from oscar_amd.backend import _Batch

    impl = make_impl()
    # continuation of 9256 rows, 16 one-token decodes, a fresh 2048-token prefill
    qsl = [0, 9256] + [9256 + i for i in range(1, 17)] + [9272 + 2048]
    seqs = [15360 + 9256] + [8193] * 16 + [2048]
    b = _Batch.classify(qsl, seqs, qsl[-1], True, 6)
    assert b.long == [0] and b.short == list(range(1, 17)) and b.fresh == [17]
    route = impl._decode_route(b)
    assert route["span"] == (1, 17, 9256, 9272) and route["index_parts"] == []
    assert route["qsl"] == list(range(17)) and route["seqs"] == [8193] * 16
    assert b.span(b.short + b.long) == (0, 17, 0, 9272)
    # an empty request between decodes keeps the slice; a fresh one between them does not
    qsl2 = [0, 4, 4, 5, 305, 306]
    seqs2 = [3004, 10, 130, 300, 701]
    b2 = _Batch.classify(qsl2, seqs2, qsl2[-1], True, 6)
    assert b2.short == [0, 2, 4] and b2.fresh == [3]
    route2 = impl._decode_route(b2)
    assert route2["span"] is None
    assert route2["qsl"] == [0, 4, 5, 6] and route2["seqs"] == [3004, 130, 701]
    assert [p.tolist() for p in route2["index_parts"]] == [[0, 1, 2, 3, 4, 305], [0, 2, 4]]
    b3 = _Batch.classify(qsl2[:5], seqs2[:4], 305, True, 6)
    assert b3.short == [0, 2] and b3.fresh == [3]
    assert impl._decode_route(b3)["span"] == (0, 3, 0, 5)
    assert impl._decode_route(b3)["qsl"] == [0, 4, 4, 5]
