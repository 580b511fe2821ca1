"""GPU parity at the BASELINE configurations, at their full sizes.

Config 1  one request: a 1024-token store (fresh prefill through the impl), then a
          single-token decode, against the oracle backend (backend.py:249-393).
Config 2  the store alone: 15360 tokens, 5 % skipped slots, 2 % rewrites, window
          write / standalone invalidation, with and without the serve-default clip;
          bytes and owner tags bit-exact, window values within the rotation bound (store_kernel.py:54-102,
          backend.py:151-198,513-555).
Config 3  one request, 24576-token history + 4-token MTP: the benchmarked layer step.
Config 4a 8 x (24576 + 4 MTP): the headline step exactly as bench.py builds and times it
          (history written by the store kernel, window live, bench's plan and window
          hint), checked at the attention level (out_rot, LSE) and at the forward level
          (bf16 output, cache bytes, tags, window).
Config 4b 64 cache-only single-token decodes, histories U[1024, 32768] (seed 20261204).
Config 5  the 15360 + 9256 continuation (sampled rows: first, last, both sides of the
          8192-key boundaries, a stride through the chunk) and the batched forward:
          continuation + 16 x (8192 history, 1 token) decodes + one 2048-token fresh
          prefill in one impl.forward call.

Tolerances (stated by the task): output max-abs 2e-2 (bf16 outputs: plus one bf16
ulp of the value), LSE 1e-3; writes bit-exact.
"""
import math

import numpy as np
import pytest
import torch

import bench
from oracle import backend as ob
from oracle import cases, fmt
from oracle.attention import attention_ref
from oracle.store import Staging, clip, rotate, store_ref
from window_check import assert_window_close

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-2
LSE_TOL = 1e-3
BF16_ULP = 2.0 ** -7


def np_u8(t):
    return t.view(torch.uint8).cpu().numpy()


def check_attention(out, lse, ref_out, ref_lse, label, rows=None):
    if rows is not None:
        out, lse, ref_out, ref_lse = out[rows], lse[rows], ref_out[rows], ref_lse[rows]
    fin = np.isfinite(ref_lse)
    assert np.array_equal(fin, np.isfinite(lse)), f"{label}: empty-row pattern differs"
    err_o = float(np.abs(out - ref_out).max())
    err_l = float(np.abs(lse[fin] - ref_lse[fin]).max()) if fin.any() else 0.0
    print(f"{label}: max|dO|={err_o:.3e} max|dLSE|={err_l:.3e}", flush=True)
    assert err_o <= OUT_TOL, f"{label}: output error {err_o}"
    assert err_l <= LSE_TOL, f"{label}: lse error {err_l}"


def check_output(got, ref, label, ulp=BF16_ULP, rows=None):
    if rows is not None:
        got, ref = got[rows], ref[rows]
    excess = float((np.abs(got - ref) - (OUT_TOL + ulp * np.abs(ref))).max())
    print(f"{label}: max|out - oracle| = {np.abs(got - ref).max():.3e}", flush=True)
    assert excess <= 0, f"{label}: output differs from the oracle"


def oracle_layer_from(setup, layer_idx=0):
    """The oracle's view of one of bench.Setup's layers (caches, window, rotations)."""
    c = bench.CONFIG
    kc, vc, (sk, sv, own) = setup.layers[layer_idx]
    layer = ob.OracleLayer(k8=np_u8(kc), v8=np_u8(vc), rk=setup.rk.cpu().numpy(),
                           rv=setup.rv.cpu().numpy(), hq=c["hq"], hk=c["hk"], d=c["d"],
                           scale=setup.scale, sink_tokens=c["sink_tokens"],
                           recent_tokens=c["recent_tokens"], staging_tokens=c["staging_tokens"])
    st = Staging(c["block_size"], c["hk"], c["d"], c["sink_tokens"], c["recent_tokens"],
                 c["staging_tokens"])
    st.stage_k, st.stage_v, st.owner = sk.cpu().numpy(), sv.cpu().numpy(), own.cpu().numpy()
    layer.staging = st
    return layer


# ---------------------------------------------------------------- configs 3 and 4a
@pytest.mark.parametrize("requests", [8, 1], ids=["config4a_8x24k_mtp", "config3_1x24k_mtp"])
def test_decode_step_at_full_size(cuda, requests):
    """The benchmarked layer step (store + window + split-K attention + merge + inverse
    rotation) with bench.py's inputs, plan and window hint, against the oracle."""
    label = f"{requests} x (24576 + 4 MTP)"
    print(f"building {label}", flush=True)
    setup = bench.Setup(cuda, [24576] * requests, 4, True, layers=1)
    layer = oracle_layer_from(setup)
    setup.step(0)
    torch.cuda.synchronize()
    kc, vc, (sk, sv, own) = setup.layers[0]
    bt = setup.bt.cpu().numpy()
    # attention level: the kernel's inputs are the store's rotated q/k/v (bit-exact to
    # the oracle's rotation, checked by the store tests) over the post-store state
    q_rot = setup.q_rot.float().cpu().numpy()
    k_rot = setup.k_rot.float().cpu().numpy()
    v_rot = setup.v_rot.float().cpu().numpy()
    stage_post = (sk.cpu().numpy(), sv.cpu().numpy(), own.cpu().numpy())
    ref_o, ref_l = attention_ref(q_rot, k_rot, v_rot, np_u8(kc), np_u8(vc), bt, setup.qsl,
                                 setup.seqs, setup.scale, stage_post)
    check_attention(setup.out_rot.cpu().numpy(), setup.lse.cpu().numpy(), ref_o, ref_l,
                    f"{label} attention")
    # forward level: write + window + read + inverse rotation from the pre-step state
    ref = ob.forward(layer, setup.q.float().cpu().numpy(), setup.k_new.float().cpu().numpy(),
                     setup.v_new.float().cpu().numpy(), setup.slots.cpu().numpy(), setup.qsl,
                     setup.seqs, bt)
    check_output(setup.out.float().cpu().numpy(), ref, f"{label} forward")
    assert np.array_equal(np_u8(kc), layer.k8), "K cache bytes differ"
    assert np.array_equal(np_u8(vc), layer.v8), "V cache bytes differ"
    assert np.array_equal(stage_post[2], layer.staging.owner), "owner tags differ"
    assert np.array_equal(stage_post[0], layer.staging.stage_k), "K window differs"
    assert np.array_equal(stage_post[1], layer.staging.stage_v), "V window differs"


# ---------------------------------------------------------------- config 4b
def test_config4b_cache_only_batch_at_full_size(cuda):
    hist = np.random.default_rng(20261204).integers(1024, 32769, 64).tolist()
    print(f"building 64 cache-only decodes, {sum(hist)} history tokens", flush=True)
    setup = bench.Setup(cuda, hist, 1, False, layers=1)
    layer = oracle_layer_from(setup)
    setup.step(0)
    torch.cuda.synchronize()
    kc, vc, (sk, sv, own) = setup.layers[0]
    bt = setup.bt.cpu().numpy()
    stage = (sk.cpu().numpy(), sv.cpu().numpy(), own.cpu().numpy())
    ref_o, ref_l = attention_ref(setup.q_rot.float().cpu().numpy(), None, None, np_u8(kc),
                                 np_u8(vc), bt, setup.qsl, setup.seqs, setup.scale, stage)
    check_attention(setup.out_rot.cpu().numpy(), setup.lse.cpu().numpy(), ref_o, ref_l,
                    "config 4b attention")
    ref = ob.forward(layer, setup.q.float().cpu().numpy(), None, None, None, setup.qsl,
                     setup.seqs, bt)
    check_output(setup.out.float().cpu().numpy(), ref, "config 4b forward")


# ---------------------------------------------------------------- config 2
def config2_slots(n, capacity, seed=20261202):
    g = np.random.default_rng(seed)
    slots = g.permutation(capacity)[:n].astype(np.int64)
    slots[g.random(n) < 0.05] = -1
    for i in np.nonzero(g.random(n) < 0.02)[0]:
        if i > 0:
            slots[i] = slots[g.integers(0, i)]
    return slots


@pytest.mark.parametrize("mode,kclip,vclip", [("write", 0.0, 0.0), ("write", 0.96, 0.92),
                                              ("invalidate", 0.0, 0.0)],
                         ids=["window_write", "window_write_clip", "standalone_update"])
def test_config2_store_at_full_size(cuda, mode, kclip, vclip):
    from oscar_amd import ops
    from oscar_amd._lib import STAGE_INVALIDATE, STAGE_WRITE

    n, hk, d, bs = 15360, 1, 256, 128
    nb = 2 * math.ceil(n / bs)
    slots = config2_slots(n, nb * bs)
    k = cases.kv_outliers(n, hk, d, cases.BASE_SEED + 2)
    v = cases.kv_outliers(n, hk, d, cases.BASE_SEED + 3)
    rk, rv = cases.hadamard_rotation(d, 5), cases.qr_rotation(d, 6)
    g = cases.rng(7)
    k8, v8 = (g.integers(0, 256, (nb, bs, hk, d), dtype=np.uint8) for _ in range(2))
    st = Staging(bs, hk, d, 64, 256, 8192)
    # earlier window contents: every seat tagged with some block, values 7
    st.owner[:] = g.integers(0, nb, st.owner.shape)
    st.stage_k[:] = 7.0
    st.stage_v[:] = -7.0
    kc, vc = (torch.from_numpy(a.copy()).view(torch.int8).cuda() for a in (k8, v8))
    sk, sv, own = (torch.from_numpy(a.copy()).cuda() for a in st.arrays())
    kw = {}
    if mode == "write":
        kw = dict(stage_mode=STAGE_WRITE, qsl_dev=torch.tensor([0, n], dtype=torch.int32).cuda(),
                  seqs_dev=torch.tensor([n], dtype=torch.int32).cuda(), num_reqs=1,
                  recent_tokens=256, sink_tokens_eff=st.sink_eff)
    else:
        kw = dict(stage_mode=STAGE_INVALIDATE)
    ops.store(torch.from_numpy(k).bfloat16().cuda(), torch.from_numpy(v).bfloat16().cuda(), kc, vc,
              torch.from_numpy(slots).cuda(), head_dim=d, rk=torch.from_numpy(rk).cuda(),
              rv=torch.from_numpy(rv).cuda(), k_clip=kclip, v_clip=vclip, stage=(sk, sv, own), **kw)
    torch.cuda.synchronize()
    kr, vr = rotate(k, rk), rotate(v, rv)
    if mode == "write":
        store_ref(clip(kr, kclip), clip(vr, vclip), k8, v8, slots)
        st.write(kr, vr, slots, [0, n], [n])
    else:
        st.invalidate(slots)
        store_ref(clip(kr, kclip), clip(vr, vclip), k8, v8, slots)
    got_k, got_v = np_u8(kc), np_u8(vc)
    bad = np.argwhere(got_k != k8)
    print(f"config 2 {mode} clip=({kclip},{vclip}): {len(np.unique(slots[slots >= 0]))} slots, "
          f"{(st.owner >= 0).sum()} tagged seats, K byte mismatches {len(bad)}", flush=True)
    assert np.array_equal(got_k, k8), f"K bytes differ at {bad[:5]}"
    assert np.array_equal(got_v, v8), "V bytes differ"
    assert np.array_equal(own.cpu().numpy(), st.owner), "owner tags differ"
    assert_window_close(sk.cpu().numpy(), st.stage_k, [k], rk, "K window")
    assert_window_close(sv.cpu().numpy(), st.stage_v, [v], rv, "V window")


# ---------------------------------------------------------------- impl harness
class _Layer:
    layer_name = "model.layers.7.self_attn.attn"


class _MD:
    pass


def make_impl(dev, d=256, hq=6, hk=1):
    from oscar_amd.backend import OscarAttentionBackendImpl

    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_heads, impl.num_kv_heads, impl.scale = d, hq, hk, d ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    return impl


def metadata(dev, slots, qsl, seqs, table):
    md = _MD()
    md.num_actual_tokens = qsl[-1]
    md.slot_mapping = torch.tensor(np.asarray(slots, np.int64), device=dev)
    md.query_start_loc_cpu = torch.tensor(qsl)
    md.seq_lens_list = list(seqs)
    md.block_tables = torch.from_numpy(np.ascontiguousarray(table)).to(dev)
    return md


def adopt_case_state(impl, layer, caches, c, dev):
    """Give the impl's layer the case's packed history and FP32 window."""
    impl._ensure_staging(layer, caches)
    sk, sv, own = c["stage"]
    layer._oscar_stage_k.copy_(torch.from_numpy(sk))
    layer._oscar_stage_v.copy_(torch.from_numpy(sv))
    layer._oscar_slot_owner.copy_(torch.from_numpy(own))


def oracle_layer_for_case(c, rk, rv, hq=6, hk=1, d=256):
    layer = ob.OracleLayer(k8=c["k8"].copy(), v8=c["v8"].copy(), rk=rk, rv=rv, hq=hq, hk=hk, d=d,
                           scale=d ** -0.5)
    st = layer.ensure_staging()
    st.stage_k[:], st.stage_v[:], st.owner[:] = c["stage"]
    return layer


# ---------------------------------------------------------------- config 1
def test_config1_store_then_decode_through_forward(cuda):
    """One request: a 1024-token store (a fresh prefill through impl.forward: INT2 write,
    window write, original-domain causal prefill), then a single-token decode."""
    dev = cuda
    d, hq, hk, bs = 256, 6, 1, 128
    impl = make_impl(dev)
    layer = _Layer()
    rk, rv = cases.hadamard_rotation(d, 11), cases.qr_rotation(d, 12)
    layer._oscar_rots = (torch.from_numpy(rk).to(dev), torch.from_numpy(rv).to(dev))
    nb = 16
    caches = [torch.zeros(nb, bs, hk, d, dtype=torch.int8, device=dev) for _ in range(2)]
    table = np.random.default_rng(13).permutation(nb).reshape(1, nb).astype(np.int32)
    oracle_layer = ob.OracleLayer(k8=np.zeros((nb, bs, hk, d), np.uint8),
                                  v8=np.zeros((nb, bs, hk, d), np.uint8), rk=rk, rv=rv, hq=hq,
                                  hk=hk, d=d, scale=d ** -0.5)
    written_k = []
    for p0, p1 in ((0, 1024), (1024, 1025)):
        n = p1 - p0
        pos = np.arange(p0, p1)
        slots = table[0, pos // bs].astype(np.int64) * bs + pos % bs
        q = cases.bf16_normal((n, hq, d), cases.BASE_SEED + p0)
        k = cases.kv_outliers(n, hk, d, cases.BASE_SEED + 1 + p0)
        v = cases.kv_outliers(n, hk, d, cases.BASE_SEED + 2 + p0)
        written_k.append(k)
        md = metadata(dev, slots, [0, n], [p1], table)
        out = torch.empty(n, hq * d, dtype=torch.bfloat16, device=dev)
        tq, tk, tv = (torch.from_numpy(x).to(dev).bfloat16() for x in (q, k, v))
        impl.forward(layer, tq.view(n, -1), tk.view(n, -1), tv.view(n, -1), caches, md, output=out)
        torch.cuda.synchronize()
        ref = ob.forward(oracle_layer, q, k, v, slots, [0, n], [p1], table)
        check_output(out.float().view(n, hq, d).cpu().numpy(), ref, f"config 1 tokens [{p0}, {p1})")
    assert np.array_equal(np_u8(caches[0]), oracle_layer.k8)
    assert np.array_equal(np_u8(caches[1]), oracle_layer.v8)
    assert np.array_equal(layer._oscar_slot_owner.cpu().numpy(), oracle_layer.staging.owner)
    assert_window_close(layer._oscar_stage_k.cpu().numpy(), oracle_layer.staging.stage_k, written_k, rk, "K window")


# ---------------------------------------------------------------- config 5
def continuation_rows(history, n, extra=48, seed=20261205, group=6):
    """First and last rows, both sides of every 8192-key boundary the chunk crosses,
    one query token in every 128-row GQA query tile of the prefill (128 // group tokens
    each; the token's place in its tile moves from tile to tile), so every tile and
    every chunk of the balanced split, with its merge slot, is compared; and a seeded
    sample through the chunk."""
    rows = {0, 1, n - 2, n - 1}
    for key in range(8192, history + n + 1, 8192):
        i = key - history - 1  # query i sees keys [0, history + i + 1)
        rows.update(r for r in (i - 1, i, i + 1) if 0 <= r < n)
    per_tile = 128 // group
    rows.update(min(n - 1, t * per_tile + (t * 8) % per_tile) for t in range(-(-n // per_tile)))
    rows.update(np.random.default_rng(seed).choice(n, extra, replace=False).tolist())
    return sorted(rows)


def test_config5_continuation_at_full_size(cuda):
    """15360-token INT2 history + a 9256-token causal chunk (the MFMA prefill path)."""
    from oscar_amd import ops

    history, n = 15360, 9256
    c = cases.make_case([history], [n], seed=20261206)
    kc = torch.from_numpy(c["k8"]).view(torch.int8).cuda()
    vc = torch.from_numpy(c["v8"]).view(torch.int8).cuda()
    stage = tuple(torch.from_numpy(a).cuda() for a in c["stage"])
    lse = torch.empty(n, 6, dtype=torch.float32, device="cuda")
    tq, tk, tv = (torch.from_numpy(c[x]).bfloat16().cuda() for x in ("q", "k", "v"))
    out = ops.attention_prefill(tq, tk, tv, c["scale"], head_dim=256, history=history, k_cache=kc,
                                v_cache=vc, block_table_row=torch.from_numpy(c["bt"][0]).cuda(),
                                stage=stage, lse=lse)
    torch.cuda.synchronize()
    rows = continuation_rows(history, n)
    assert {r // (128 // 6) for r in rows} == set(range(-(-n // (128 // 6))))  # every query tile
    ref_o, ref_l = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                 c["seqs"], c["scale"], c["stage"], rows=rows)
    check_attention(out.cpu().numpy(), lse.cpu().numpy(), ref_o, ref_l,
                    f"continuation {history}+{n} ({len(rows)} sampled rows)", rows=rows)


def test_config5_batched_forward(cuda):
    """One impl.forward over the whole config-5 batch: the continuation (15360 + 9256),
    16 decodes over 8192-token histories and a history-free 2048-token prefill."""
    dev = cuda
    d, hq, hk = 256, 6, 1
    prefixes = [15360] + [8192] * 16 + [0]
    lengths = [9256] + [1] * 16 + [2048]
    c = cases.make_case(prefixes, lengths, seed=20261207)
    impl = make_impl(dev)
    layer = _Layer()
    rk, rv = cases.hadamard_rotation(d, 21), cases.qr_rotation(d, 22)
    layer._oscar_rots = (torch.from_numpy(rk).to(dev), torch.from_numpy(rv).to(dev))
    caches = [torch.from_numpy(c[x]).view(torch.int8).to(dev) for x in ("k8", "v8")]
    adopt_case_state(impl, layer, caches, c, dev)
    oracle_layer = oracle_layer_for_case(c, rk, rv)
    qsl, seqs, bs = c["qsl"], c["seqs"], 128
    slots = []
    for r, (p, n) in enumerate(zip(prefixes, lengths)):
        pos = np.arange(p, p + n)
        slots.append(c["bt"][r, pos // bs].astype(np.int64) * bs + pos % bs)
    slots = np.concatenate(slots)
    N = qsl[-1]
    md = metadata(dev, slots, qsl, seqs, c["bt"])
    out = torch.empty(N, hq * d, dtype=torch.bfloat16, device=dev)
    tq, tk, tv = (torch.from_numpy(c[x]).bfloat16().to(dev) for x in ("q", "k", "v"))
    impl.forward(layer, tq.view(N, -1), tk.view(N, -1), tv.view(N, -1), caches, md, output=out)
    torch.cuda.synchronize()
    rows = continuation_rows(prefixes[0], lengths[0]) + list(range(qsl[1], qsl[-1]))
    ref = ob.forward(oracle_layer, c["q"], c["k"], c["v"], slots, qsl, seqs, c["bt"], rows=rows)
    check_output(out.float().view(N, hq, d).cpu().numpy(), ref,
                 f"config 5 batched forward ({len(rows)} rows)", rows=rows)
    assert np.array_equal(np_u8(caches[0]), oracle_layer.k8)
    assert np.array_equal(np_u8(caches[1]), oracle_layer.v8)
    assert np.array_equal(layer._oscar_slot_owner.cpu().numpy(), oracle_layer.staging.owner)
    assert_window_close(layer._oscar_stage_v.cpu().numpy(), oracle_layer.staging.stage_v, [c["v"]], rv, "V window")


# ---------------------------------------------------------------- the reference's probe cases
# delivery/probe_streaming.py:100-119 (kernel_cases) through the impl's read routing
# (decode, cache-only split, continuation prefill, fresh-only prefill) with identity
# rotations, so the impl's output is the rotated-domain attention the oracle evaluates.
PROBE_CASES = [
    ("mixed", [0, 129, 1025, 0], [1, 4, 3, 0], {}),
    ("batch32", [128 + i % 3 for i in range(32)], [4] * 32, {}),
    ("batch16", [129] * 16, [4] * 16, {}),
    ("batch64", [129] * 64, [4] * 64, {}),
    ("cached_prefill", [129], [1024], {}),
    ("long_24k", [24579], [4], {}),
    ("cache_only_empty", [0, 257], [1, 1], {"fresh": False}),
    ("cache_only_multi", [3, 263], [7, 9], {"fresh": False}),
    ("slab_boundary_prefill", [8193], [257], {}),
    ("multi_kv_legacy", [129], [7], {"hk": 2, "legacy": True}),
    ("fp16", [1537], [4], {"qdt": torch.float16}),
    ("large-page", [1537], [4], {"bs": 1536}),
    ("fp16-large-page", [1537], [4], {"bs": 1536, "qdt": torch.float16}),
]


@pytest.mark.parametrize("name,prefixes,lengths,opts", PROBE_CASES, ids=[p[0] for p in PROBE_CASES])
def test_reference_probe_cases_through_impl(cuda, name, prefixes, lengths, opts):
    dev = cuda
    hk, d, bs = opts.get("hk", 1), 256, opts.get("bs", 128)
    hq = 6 * hk
    qdt = opts.get("qdt", torch.bfloat16)
    fresh = opts.get("fresh", True)
    c = cases.make_case(prefixes, lengths, hk=hk, bs=bs, fresh=fresh, legacy=opts.get("legacy", False))
    impl = make_impl(dev, d, hq, hk)
    layer = _Layer()
    eye = torch.eye(d, dtype=torch.float32, device=dev)
    layer._oscar_rots = (eye, eye)
    cdt = torch.bfloat16 if opts.get("legacy") else torch.int8
    caches = [torch.from_numpy(c[x]).view(cdt).to(dev) for x in ("k8", "v8")]
    impl._set_caches(caches)
    adopt_case_state(impl, layer, caches, c, dev)
    N = c["qsl"][-1]
    md = metadata(dev, np.zeros(N, np.int64), c["qsl"], c["seqs"], c["bt"])
    out = torch.empty(N, hq * d, dtype=qdt, device=dev)
    tq = torch.from_numpy(c["q"]).to(dev).to(qdt)
    tk = None if c["k"] is None else torch.from_numpy(c["k"]).to(dev).to(qdt)
    tv = None if c["v"] is None else torch.from_numpy(c["v"]).to(dev).to(qdt)
    # the read path alone (no store): the case's history and window are the state
    impl._streaming_attention(layer, tq.view(N, -1), None if tk is None else tk.view(N, -1),
                              None if tv is None else tv.view(N, -1), caches, md, out)
    torch.cuda.synchronize()
    q_dtype = "f16" if qdt == torch.float16 else "bf16"
    ref_o, _ = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"], c["seqs"],
                             c["scale"], c["stage"], d=d, q_dtype=q_dtype)
    ulp = BF16_ULP if qdt == torch.bfloat16 else 2.0 ** -10
    check_output(out.float().view(N, hq, d).cpu().numpy(), fmt.round_to(ref_o, q_dtype), name, ulp)
