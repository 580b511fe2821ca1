"""The plugin impl's forward on the GPU against the oracle's restatement of the
reference backend (backend.py:249-393): writes, window tags, and attention routed to
fresh-only prefill, split-K decode / MTP and continuation prefill, in bf16 and fp16."""
import numpy as np
import pytest
import torch

from oracle import backend as ob
from oracle import cases

pytestmark = pytest.mark.gpu


class _Layer:
    layer_name = "model.layers.3.self_attn.attn"


class _MD:
    pass


@pytest.mark.parametrize("qdt,ulp", [(torch.bfloat16, 2.0 ** -7), (torch.float16, 2.0 ** -10)],
                         ids=["bf16", "fp16"])
def test_forward_steps_match_oracle(cuda, qdt, ulp):
    from oscar_amd.backend import OscarAttentionBackendImpl

    dev = torch.device("cuda", 0)
    d, hq, hk, bs = 256, 6, 1, 128
    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_heads, impl.num_kv_heads, impl.scale = d, hq, hk, d ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    layer = _Layer()
    rk, rv = cases.hadamard_rotation(d, 5), cases.qr_rotation(d, 6)
    layer._oscar_rots = (torch.from_numpy(rk).to(dev), torch.from_numpy(rv).to(dev))
    nb, per = 24, 12
    caches = [torch.zeros(nb, bs, hk, d, dtype=torch.int8, device=dev) for _ in range(2)]
    table = np.random.default_rng(7).permutation(nb).reshape(2, per).astype(np.int32)
    oracle_layer = ob.OracleLayer(k8=np.zeros((nb, bs, hk, d), np.uint8), v8=np.zeros((nb, bs, hk, d), np.uint8),
                                  rk=rk, rv=rv, hq=hq, hk=hk, d=d, scale=d ** -0.5)
    q_dtype = "bf16" if qdt == torch.bfloat16 else "f16"
    lens = [0, 0]
    # (new tokens of request 0, of request 1): fresh prefills, MTP + single-token
    # decode, continuation chunks of 1200 and 2400 rows (the split-K decode, as 32-row
    # sub-requests) beside a decode and an MTP step (the continuation prefill through
    # the forward: test_config5_batched_forward)
    for step, (n0, n1) in enumerate([(300, 700), (4, 1), (200, 1), (400, 3)]):
        news = [n0, n1]
        slots, qsl, seqs = [], [0], []
        for r, n in enumerate(news):
            pos = np.arange(lens[r], lens[r] + n)
            slots += (table[r, pos // bs].astype(np.int64) * bs + pos % bs).tolist()
            qsl.append(qsl[-1] + n)
            seqs.append(lens[r] + n)
        N = qsl[-1]
        q = cases.bf16_normal((N, hq, d), 100 + step)
        k = cases.kv_outliers(N, hk, d, 200 + step)
        v = cases.kv_outliers(N, hk, d, 300 + step)
        md = _MD()
        md.num_actual_tokens = N
        md.slot_mapping = torch.tensor(slots, device=dev)
        md.query_start_loc_cpu = torch.tensor(qsl)
        md.seq_lens_list = seqs
        md.block_tables = torch.from_numpy(table).to(dev)
        out = torch.empty(N, hq * d, dtype=qdt, device=dev)
        tq, tk, tv = (torch.from_numpy(x).to(dev).to(qdt) for x in (q, k, v))
        impl.forward(layer, tq.view(N, -1), tk.view(N, -1), tv.view(N, -1), caches, md, output=out)
        torch.cuda.synchronize()
        ref = ob.forward(oracle_layer, q, k, v, slots, qsl, seqs, table, q_dtype=q_dtype)
        got = out.float().view(N, hq, d).cpu().numpy()
        # 2e-2 absolute plus one output ulp of the value (outlier channels make early
        # causal rows large, where one ulp exceeds 2e-2)
        excess = float((np.abs(got - ref) - (2e-2 + ulp * np.abs(ref))).max())
        print(f"{q_dtype} step {step}: max|out - oracle| = {np.abs(got - ref).max():.3e}", flush=True)
        assert excess <= 0, f"step {step}: output differs from the oracle"
        lens = seqs
    assert np.array_equal(layer._oscar_slot_owner.cpu().numpy(), oracle_layer.staging.owner)
    assert np.array_equal(caches[0].view(torch.uint8).cpu().numpy(), oracle_layer.k8)
    assert np.array_equal(caches[1].view(torch.uint8).cpu().numpy(), oracle_layer.v8)


@pytest.mark.parametrize("mode", ["mtp_window", "cache_only", "fp16_mtp", "long_chunks", "long_chunks_fresh",
                                  "fresh_last"])
def test_native_decode_step_matches_general_path_and_oracle(cuda, mode):
    """forward() on decode-shaped batches takes oscar_decode_step_v1 (one native call);
    the same batch through the general Python path (_run) and the oracle agree.
    long_chunks: chunks of 240 and 72 rows per KV head (sub-requests of the plan);
    long_chunks_fresh: the same beside a history-free request, which the native step
    declines and the general path routes as a compact decode batch (gathered rows and
    block-table rows, the fresh request lying between decodes) plus a prefill;
    fresh_last: the fresh request after the decodes (their rows and table rows are a
    slice of the batch's)."""
    from oscar_amd import backend as B
    from oracle.attention import attention_ref

    dev = torch.device("cuda", 0)
    qdt = torch.float16 if mode == "fp16_mtp" else torch.bfloat16
    fresh = mode != "cache_only"
    prefixes, lengths = [3000, 129, 700, 24579], [4, 1, 3, 4]
    if mode == "long_chunks":
        lengths = [40, 1, 12, 4]
    if mode == "long_chunks_fresh":
        prefixes, lengths = [3000, 0, 700, 24579], [40, 300, 12, 4]
    if mode == "fresh_last":
        prefixes, lengths = [3000, 700, 24579, 0], [40, 12, 4, 300]
    c = cases.make_case(prefixes, lengths, fresh=fresh, seed=77)
    d, hq, hk = 256, 6, 1
    impl = OscarAttentionBackendImplFactory()
    layer = _Layer()
    eye = torch.eye(d, dtype=torch.float32, device=dev)
    layer._oscar_rots = (eye, eye)
    caches = [torch.from_numpy(c[x]).view(torch.int8).to(dev) for x in ("k8", "v8")]
    impl._set_caches(caches)
    impl._ensure_staging(layer, caches)
    sk, sv, own = c["stage"]
    layer._oscar_stage_k.copy_(torch.from_numpy(sk))
    layer._oscar_stage_v.copy_(torch.from_numpy(sv))
    layer._oscar_slot_owner.copy_(torch.from_numpy(own))
    N = c["qsl"][-1]
    md = _MD()
    md.num_actual_tokens = N
    # the current chunk is not written (slots -1): the history and window stay the state
    md.slot_mapping = torch.full((N,), -1, dtype=torch.int64, device=dev)
    md.query_start_loc_cpu = torch.tensor(c["qsl"], dtype=torch.int32)
    md.seq_lens_cpu = torch.tensor(c["seqs"], dtype=torch.int32)
    md.block_tables = torch.from_numpy(c["bt"]).to(dev)
    tq = torch.from_numpy(c["q"]).to(dev).to(qdt).view(N, -1)
    tk = None if c["k"] is None else torch.from_numpy(c["k"]).to(dev).to(qdt).view(N, -1)
    tv = None if c["v"] is None else torch.from_numpy(c["v"]).to(dev).to(qdt).view(N, -1)
    calls = {"reads": impl._oscar_stats["reads"]}
    out_native = torch.empty(N, hq * d, dtype=qdt, device=dev)
    native = impl._native_step(layer, tq, tk, tv, caches, md, out_native)
    assert native == (mode not in ("long_chunks_fresh", "fresh_last"))
    out_general = torch.empty_like(out_native)
    impl._run(layer, tq, tk, tv, caches, md, out_general, write=True)
    torch.cuda.synchronize()
    assert impl._oscar_stats["reads"] == calls["reads"] + 1 + native
    if not native:
        out_native = out_general
    q_dtype = "f16" if qdt == torch.float16 else "bf16"
    ref_o, _ = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"], c["seqs"],
                             c["scale"], c["stage"], q_dtype=q_dtype)
    ulp = 2.0 ** -7 if qdt == torch.bfloat16 else 2.0 ** -10
    for label, out in (("native", out_native), ("general", out_general)):
        got = out.float().view(N, hq, d).cpu().numpy()
        excess = float((np.abs(got - ref_o) - (2e-2 + ulp * np.abs(ref_o))).max())
        print(f"{mode} {label}: max|out - oracle| = {np.abs(got - ref_o).max():.3e}", flush=True)
        assert excess <= 0, f"{mode} {label} differs from the oracle"
    diff = (out_native.float() - out_general.float()).abs().max().item()
    print(f"{mode}: native vs general max diff {diff:.3e}", flush=True)
    assert diff <= 2e-2


def OscarAttentionBackendImplFactory():
    from oscar_amd.backend import OscarAttentionBackendImpl

    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_heads, impl.num_kv_heads, impl.scale = 256, 6, 1, 256 ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    return impl
