"""GPU parity of the read path (decode split-K kernel, prefill kernel, merge, rotation).

Tolerances (stated by the task for this path): attention output within max-abs
2e-2 of the oracle, natural-log LSE within 1e-3 of an FP32 evaluation of the
reference math.  The oracle evaluates softmax exactly (float64) at the
reference's rounding points (history values rounded fp16 -> bf16).
"""
import math

import numpy as np
import pytest
import torch

from oracle import cases, fmt
from oracle.attention import attention_ref, causal_prefill_ref

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-2
LSE_TOL = 1e-3


def dev(x, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).cuda()


def run_decode(c, d=256, hk=1, group=6, target=256, hint=None, qdt=torch.bfloat16):
    """hint: the planner's window hint; default the window make_case stages (sink 128,
    recent 256) when the case has one.  qdt: the query (and current K/V) dtype."""
    from oscar_amd import ops

    kc = torch.from_numpy(c["k8"]).view(torch.int8).cuda()
    vc = torch.from_numpy(c["v8"]).view(torch.int8).cuda()
    stage = None if c["stage"] is None else tuple(torch.from_numpy(a).cuda() for a in c["stage"])
    if hint is None:
        hint = (128, 256) if c["stage"] is not None else (0, 0)
    plan = ops.plan_decode(c["qsl"], c["seqs"], has_new=c["k"] is not None, num_kv_heads=hk,
                           group=group, head_dim=d, device=torch.device("cuda"), target_items=target,
                           window=hint)
    out, lse = ops.attention_decode(dev(c["q"], qdt), None if c["k"] is None else dev(c["k"], qdt),
                                    None if c["v"] is None else dev(c["v"], qdt),
                                    kc, vc, torch.from_numpy(c["bt"]).cuda(), plan, c["scale"],
                                    stage, head_dim=d)
    torch.cuda.synchronize()
    return out.cpu().numpy(), lse.cpu().numpy(), plan


def check(out, lse, ref_out, ref_lse, label):
    fin = np.isfinite(ref_lse)
    assert np.array_equal(fin, np.isfinite(lse)), f"{label}: empty-row pattern differs"
    err_o = np.abs(out - ref_out).max() if out.size else 0.0
    err_l = np.abs(lse[fin] - ref_lse[fin]).max() if fin.any() else 0.0
    print(f"{label}: max|dO|={err_o:.3e} max|dLSE|={err_l:.3e}", flush=True)
    assert err_o <= OUT_TOL, f"{label}: output error {err_o}"
    assert err_l <= LSE_TOL, f"{label}: lse error {err_l}"
    assert np.all(out[~fin] == 0)


DECODE_CASES = [
    ("mtp_mixed_window", [129, 1025, 3, 300], [4, 3, 1, 2], {}),
    ("batch16", [129] * 16, [4] * 16, {}),
    ("long_24k", [24579], [4], {}),
    ("cache_only", [0, 257, 3, 263], [1, 1, 4, 5], {"fresh": False}),
    ("no_window", [1025, 2048], [4, 4], {"window": False}),
    ("d128_hk2", [129, 700], [4, 2], {"d": 128, "hk": 2, "group": 4}),
    # few items of up to 256 tiles: slow tiles (sink/recent window, ragged end, current
    # chunk) at item-tile indices past 32 and 64
    ("few_long_items", [9000], [1], {"fresh": False, "target": 2}),
    ("few_long_items_mtp", [8000, 3001], [4, 2], {"target": 3}),
    # keys growing along the history: each item's running max moves many times
    # (the fast tiles' rescale of O, l and z)
    ("rising_scores", [6000, 2500], [4, 1], {"key_ramp": 4.0, "target": 4}),
    # the planner's window hint is only a hint: none, and one far wider than the
    # staged window (window items that hold plain history tiles)
    ("hint_off", [1025, 2048, 5000], [4, 4, 1], {"hint": (0, 0), "target": 24}),
    # pages of 32 and 64 tokens: every tile is a whole page, or half of one
    ("pages_32", [1000, 77], [4, 1], {"bs": 32, "target": 16}),
    ("pages_64", [3000, 129], [4, 2], {"bs": 64}),
    # other profiles: 1536-token pages; the legacy bf16-width cache (512-byte slots)
    # with two KV heads
    ("pages_1536", [5000, 300], [4, 2], {"bs": 1536}),
    ("legacy_hk2", [700, 2000], [4, 1], {"legacy": True, "hk": 2, "group": 3}),
    ("hint_wide", [3000, 5000], [4, 1], {"hint": (512, 2048), "target": 24}),
    # chunks of more than 32 rows per KV head: sub-requests of 5 (4 at group 8) query
    # tokens, whose later sub-requests see the chunk's earlier keys as current rows
    ("chunk_240_rows", [3000, 500], [40, 7], {}),
    ("chunk_d128_hk2", [1500, 40], [20, 9], {"d": 128, "hk": 2, "group": 4}),
    ("chunk_no_window", [2000], [33], {"window": False, "target": 16}),
    ("cache_only_long", [2000, 100], [12, 20], {"fresh": False}),
    # items of one tile each, history and window tiles alike: wave 0's state is the
    # item's partial (no cross-wave merge)
    ("one_tile_items", [4000, 40], [1, 3], {"fresh": False, "target": 200, "hint": (0, 0), "one_tile": True}),
]


@pytest.mark.parametrize("name,prefixes,lengths,opts", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_decode_matches_oracle(cuda, name, prefixes, lengths, opts):
    d = opts.get("d", 256)
    hk = opts.get("hk", 1)
    group = opts.get("group", 6)
    c = cases.make_case(prefixes, lengths, d=d, hk=hk, group=group, bs=opts.get("bs", 128),
                        fresh=opts.get("fresh", True), window=opts.get("window", True),
                        key_ramp=opts.get("key_ramp", 0.0), legacy=opts.get("legacy", False))
    out, lse, plan = run_decode(c, d, hk, group, opts.get("target", 256), opts.get("hint"))
    if opts.get("one_tile"):
        counts = plan.host_items.reshape(plan.num_items, -1)[:, 4]  # tiles per item (record word 4)
        assert (counts == 1).sum() >= 100, f"{name}: {(counts == 1).sum()} one-tile items"
    ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                     c["seqs"], c["scale"], c["stage"], d=d)
    check(out, lse, ref_out, ref_lse, name)


@pytest.mark.parametrize("name,prefixes,lengths,opts", [
    ("mtp_mixed_window", [129, 1025, 3, 300], [4, 3, 1, 2], {}),
    ("cache_only", [0, 257, 3, 263], [1, 1, 4, 5], {"fresh": False}),
    ("d128_hk2", [129, 700], [4, 2], {"d": 128, "hk": 2, "group": 4}),
    ("long_items", [9000, 2100], [4, 1], {"target": 6}),
], ids=lambda v: v if isinstance(v, str) else None)
def test_decode_fp16_queries_match_oracle(cuda, name, prefixes, lengths, opts):
    """fp16 queries (probe_streaming.py:100-107 profiles): history values rounded
    fp16(x), fp16 MFMA operands; the oracle evaluates the reference math with q_dtype
    fp16.  The case values sit on the bf16 grid, which fp16 holds exactly."""
    d, hk, group = opts.get("d", 256), opts.get("hk", 1), opts.get("group", 6)
    c = cases.make_case(prefixes, lengths, d=d, hk=hk, group=group, fresh=opts.get("fresh", True))
    out, lse, _ = run_decode(c, d, hk, group, opts.get("target", 256), qdt=torch.float16)
    ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                     c["seqs"], c["scale"], c["stage"], d=d, q_dtype="f16")
    check(out, lse, ref_out, ref_lse, f"fp16 {name}")


@pytest.mark.parametrize("seed", range(6))
def test_decode_random_batches_match_oracle(cuda, seed):
    """Seeded random batches: request count, history lengths (0 to 6000), query
    lengths, fresh or cache-only, window or none, Hk, group, head dim, page size and
    the planner's target, each against the oracle."""
    rng = np.random.default_rng(4100 + seed)
    d = int(rng.choice([128, 256]))
    hk = int(rng.choice([1, 2]))
    group = int(rng.choice([2, 3, 4, 6]))
    fresh = bool(rng.integers(2))
    nreq = int(rng.integers(1, 7))
    prefixes = rng.integers(0 if not fresh else 1, 6000, nreq).tolist()
    lengths = rng.integers(1, 32 // group + 1, nreq).tolist()
    bs = int(rng.choice([32, 64, 128, 256]))
    window = bool(rng.integers(2))
    target = int(rng.choice([8, 64, 256]))
    label = f"seed {seed}: d={d} hk={hk} group={group} fresh={fresh} bs={bs} window={window} " \
            f"target={target} prefixes={prefixes} lengths={lengths}"
    print(label, flush=True)
    c = cases.make_case(prefixes, lengths, d=d, hk=hk, group=group, bs=bs, fresh=fresh,
                        window=window, seed=200 + seed)
    out, lse, _ = run_decode(c, d, hk, group, target)
    ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                     c["seqs"], c["scale"], c["stage"], d=d)
    check(out, lse, ref_out, ref_lse, label)


@pytest.mark.parametrize("gain", [1e3, 1e4], ids=["v1e3", "v1e4"])
def test_decode_large_value_scales(cuda, gain):
    """V magnitudes of 1e3 and 1e4 (per-token V scales far above 256): the reference's
    rounding fp16(x) -> bf16 stays finite up to |V| = 65504, so the output must too.
    The absolute tolerance scales with the value magnitude (2e-2 per unit of V)."""
    c = cases.make_case([3000, 700, 129], [4, 1, 3], v_gain=gain)
    out, lse, _ = run_decode(c, target=16)
    ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                     c["seqs"], c["scale"], c["stage"])
    assert np.isfinite(out).all(), "non-finite output"
    err_o = np.abs(out - ref_out).max()
    err_l = np.abs(lse - ref_lse).max()
    print(f"V x {gain:g}: max|dO|={err_o:.3e} (max|V| {np.abs(c['v']).max():.0f}) "
          f"max|dLSE|={err_l:.3e}", flush=True)
    assert err_o <= OUT_TOL * gain
    assert err_l <= LSE_TOL


def test_decode_nan_propagates_through_merge(cuda):
    """A NaN in one staged window value: the rows of that request that see the token are
    NaN (out and LSE) after the split-K merge; every other request is unaffected
    (slab_attention.py:341-356: NaN propagates)."""
    c = cases.make_case([2000, 1500, 300], [4, 2, 1])
    sk, sv, owner = c["stage"]
    # request 1's first position is a staged sink token
    blk = int(c["bt"][1, 0])
    row = blk % owner.shape[0]
    assert owner[row, 0] == blk
    sk[row, 0, 0, 7] = np.nan
    out, lse, _ = run_decode(c, target=64)
    ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                     c["seqs"], c["scale"], c["stage"])
    nan_rows = np.isnan(ref_lse)
    assert nan_rows[4:6].all() and not nan_rows[:4].any() and not nan_rows[6:].any()
    assert np.array_equal(np.isnan(lse), nan_rows), "NaN LSE rows differ"
    assert np.isnan(out[nan_rows]).all(), "NaN rows not NaN in the output"
    ok = ~nan_rows
    err_o = np.abs(out[ok] - ref_out[ok]).max()
    err_l = np.abs(lse[ok] - ref_lse[ok]).max()
    print(f"nan case: other rows max|dO|={err_o:.3e} max|dLSE|={err_l:.3e}", flush=True)
    assert err_o <= OUT_TOL and err_l <= LSE_TOL


def test_decode_bad_plan_records_poison_only_their_rows(cuda):
    """Records that break the planner's rules (a group whose item range runs past the
    plan, an item whose key tiles run past its sequence) turn that group's rows into NaN
    (output and LSE) instead of reading out of bounds; every other group is unaffected."""
    import dataclasses
    from oscar_amd import ops

    c = cases.make_case([2000, 1500, 300, 700], [4, 2, 1, 3])
    out, lse, plan = run_decode(c, target=48)
    ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                     c["seqs"], c["scale"], c["stage"])
    check(out, lse, ref_out, ref_lse, "good plan")
    groups = plan.host_groups.reshape(-1, 8).copy()
    items = plan.host_items.reshape(-1, 8).copy()
    groups[1, 3] = plan.num_items + 5                      # group 1: item range past the plan
    g2 = groups[2]
    it = items[(items[:, 0] == g2[0]) & (items[:, 6] == g2[4])][0]
    idx = int(np.nonzero((items == it).all(axis=1))[0][0])
    items[idx, 2] = 10 ** 6                                 # group 2: one item's tiles past its sequence
    bad = dataclasses.replace(plan, host_items=items.reshape(-1), host_groups=groups.reshape(-1))
    bad.adopt(ops.upload(bad.host_parts(), torch.device("cuda")))
    kc = torch.from_numpy(c["k8"]).view(torch.int8).cuda()
    vc = torch.from_numpy(c["v8"]).view(torch.int8).cuda()
    stage = tuple(torch.from_numpy(a).cuda() for a in c["stage"])
    o2, l2 = ops.attention_decode(dev(c["q"]), dev(c["k"]), dev(c["v"]), kc, vc, torch.from_numpy(c["bt"]).cuda(),
                                  bad, c["scale"], stage, head_dim=256)
    torch.cuda.synchronize()
    o2, l2 = o2.cpu().numpy(), l2.cpu().numpy()
    rows = {r: np.arange(c["qsl"][r], c["qsl"][r + 1]) for r in range(4)}
    for r in (1, 2):
        assert np.isnan(l2[rows[r]]).all() and np.isnan(o2[rows[r]]).all(), f"request {r} not poisoned"
    for r in (0, 3):
        assert np.array_equal(np.isnan(l2[rows[r]]), np.zeros_like(l2[rows[r]], bool))
        assert np.abs(o2[rows[r]] - ref_out[rows[r]]).max() <= OUT_TOL


def test_decode_plan_covers_each_history_token_once(cuda):
    c = cases.make_case([24579] * 8, [4] * 8)
    from oscar_amd import ops

    plan = ops.plan_decode(c["qsl"], c["seqs"], has_new=True, num_kv_heads=1, group=6,
                           head_dim=256, device=torch.device("cuda"), target_items=256,
                           window=(128, 256))
    items = np.array(plan.host_items).reshape(-1, 8)
    assert plan.num_items <= 256 and items[:, 4].max() <= 32
    for r, seq in enumerate(c["seqs"]):
        rows = items[items[:, 0] == r]
        cover = np.zeros((seq + 31) // 32, np.int32)
        for _, kvh_nq, first, stride, count, *_ in rows:
            cover[first + stride * np.arange(count)] += 1
            assert kvh_nq >> 16 == 4
        assert (cover == 1).all()
        assert len(set(rows[:, 5])) == len(rows)


def test_prefill_fresh_only_matches_sdpa(cuda):
    from oscar_amd import ops

    for n, hq, hk in ((300, 6, 1), (129, 8, 2), (1100, 6, 1)):  # 1100: key ranges split in 3 chunks
        q = cases.bf16_normal((n, hq, 256), 71)
        k = cases.bf16_normal((n, hk, 256), 72)
        v = cases.bf16_normal((n, hk, 256), 73)
        out = ops.attention_prefill(dev(q), dev(k), dev(v), 1 / 16, head_dim=256)
        torch.cuda.synchronize()
        ref = causal_prefill_ref(q, k, v, 1 / 16)
        err = np.abs(out.float().cpu().numpy() - ref).max()
        print(f"fresh prefill n={n}: max|dO|={err:.3e}", flush=True)
        assert err <= OUT_TOL


@pytest.mark.parametrize("prefix,n,ramp", [(1025, 100, 0.0), (8193, 257, 0.0), (129, 1024, 0.0),
                                           (3000, 300, 4.0)])
def test_prefill_continuation_matches_oracle(cuda, prefix, n, ramp):
    from oscar_amd import ops

    c = cases.make_case([prefix], [n], key_ramp=ramp)
    kc = torch.from_numpy(c["k8"]).view(torch.int8).cuda()
    vc = torch.from_numpy(c["v8"]).view(torch.int8).cuda()
    stage = tuple(torch.from_numpy(a).cuda() for a in c["stage"])
    lse = torch.empty(n, 6, dtype=torch.float32, device="cuda")
    out = ops.attention_prefill(dev(c["q"]), dev(c["k"]), dev(c["v"]), c["scale"], head_dim=256,
                                history=prefix, k_cache=kc, v_cache=vc,
                                block_table_row=torch.from_numpy(c["bt"][0]).cuda(), stage=stage,
                                lse=lse)
    torch.cuda.synchronize()
    ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                     c["seqs"], c["scale"], c["stage"])
    check(out.cpu().numpy(), lse.cpu().numpy(), ref_out, ref_lse, f"continuation {prefix}+{n}")


@pytest.mark.parametrize("prefix,n,d,hk,group,qdt", [
    (8193, 257, 256, 1, 6, "bf16"), (0, 1100, 256, 1, 6, "bf16"), (1025, 700, 256, 1, 6, "bf16"),
    (2000, 600, 128, 2, 4, "bf16"), (0, 900, 128, 2, 4, "f16"), (3000, 200, 256, 1, 6, "f16")])
def test_prefill_split_matches_unsplit_and_oracle(cuda, prefix, n, d, hk, group, qdt):
    """The balanced split (chunks of the query tiles' key ranges, partials merged by
    prefill_merge_kernel) against one workgroup per query tile and the oracle, at both
    head dims, GQA 4 over two KV heads and fp16 queries."""
    import ctypes as C
    from oscar_amd import _lib, ops

    hq = hk * group
    out = (C.c_int32 * 64)()
    assert _lib.load().oscar_prefill_plan_v1(prefix, n, hq, hk, out, 64) == 0 and out[0] >= 2
    c = cases.make_case([prefix], [n], fresh=True, seed=prefix + n, hk=hk, group=group, d=d)
    tdt = torch.float16 if qdt == "f16" else torch.bfloat16
    kw = dict(head_dim=d)
    if prefix:
        kw.update(history=prefix, k_cache=torch.from_numpy(c["k8"]).view(torch.int8).cuda(),
                  v_cache=torch.from_numpy(c["v8"]).view(torch.int8).cuda(),
                  block_table_row=torch.from_numpy(c["bt"][0]).cuda(),
                  stage=tuple(torch.from_numpy(a).cuda() for a in c["stage"]))
    res = {}
    for split in (True, False):
        lse = torch.empty(n, hq, dtype=torch.float32, device="cuda")
        o = ops.attention_prefill(dev(c["q"], tdt), dev(c["k"], tdt), dev(c["v"], tdt), c["scale"], lse=lse,
                                  split=split, **kw)
        torch.cuda.synchronize()
        res[split] = (o.float().cpu().numpy(), lse.cpu().numpy())
    if prefix:
        ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                         c["seqs"], c["scale"], c["stage"], q_dtype=qdt)
        for split in (True, False):
            check(*res[split], ref_out, ref_lse, f"continuation {prefix}+{n} d={d} {qdt} split={split}")
        tol = 1e-3
    else:
        ref = causal_prefill_ref(c["q"], c["k"], c["v"], c["scale"], q_dtype=qdt)
        for split in (True, False):
            err = np.abs(res[split][0] - ref).max()
            print(f"fresh {n} d={d} {qdt} split={split}: max|dO|={err:.3e}", flush=True)
            assert err <= OUT_TOL
        unit = 2.0 ** -10 if qdt == "f16" else 2.0 ** -7  # one output ulp of the largest value
        tol = unit * max(1.0, float(np.abs(ref).max()))
    d_out = np.abs(res[True][0] - res[False][0]).max()
    d_lse = np.abs(res[True][1] - res[False][1]).max()
    print(f"split vs unsplit {prefix}+{n}: max|dO| {d_out:.3e}, max|dLSE| {d_lse:.3e}", flush=True)
    assert d_out <= tol and d_lse <= 1e-4


def test_prefill_fp16_queries(cuda):
    """fp16 q/k/v: the fresh-only prefill returns fp16 (original domain); the
    continuation rounds the history fp16(x) (oracle with q_dtype f16)."""
    from oscar_amd import ops

    q = cases.bf16_normal((300, 6, 256), 81)
    k = cases.bf16_normal((300, 1, 256), 82)
    v = cases.bf16_normal((300, 1, 256), 83)
    out = ops.attention_prefill(dev(q, torch.float16), dev(k, torch.float16), dev(v, torch.float16), 1 / 16,
                                head_dim=256)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    err = np.abs(out.float().cpu().numpy() - causal_prefill_ref(q, k, v, 1 / 16)).max()
    print(f"fp16 fresh prefill: max|dO|={err:.3e}", flush=True)
    assert err <= OUT_TOL
    prefix, n = 3000, 300
    c = cases.make_case([prefix], [n], key_ramp=4.0)
    kc = torch.from_numpy(c["k8"]).view(torch.int8).cuda()
    vc = torch.from_numpy(c["v8"]).view(torch.int8).cuda()
    stage = tuple(torch.from_numpy(a).cuda() for a in c["stage"])
    lse = torch.empty(n, 6, dtype=torch.float32, device="cuda")
    out = ops.attention_prefill(dev(c["q"], torch.float16), dev(c["k"], torch.float16),
                                dev(c["v"], torch.float16), c["scale"], head_dim=256, history=prefix,
                                k_cache=kc, v_cache=vc, block_table_row=torch.from_numpy(c["bt"][0]).cuda(),
                                stage=stage, lse=lse)
    torch.cuda.synchronize()
    ref_out, ref_lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"],
                                     c["seqs"], c["scale"], c["stage"], q_dtype="f16")
    check(out.cpu().numpy(), lse.cpu().numpy(), ref_out, ref_lse, "fp16 continuation 3000+300")


def test_rotate_matches_fp32_reference(cuda):
    from oscar_amd import ops

    x = np.random.default_rng(81).standard_normal((333, 256)).astype(np.float32)
    r = cases.qr_rotation(256, 82)
    for transpose in (False, True):
        got = ops.rotate(dev(x, torch.float32), torch.from_numpy(r).cuda(), transpose=transpose).cpu().numpy()
        ref = x.astype(np.float64) @ (r.T if transpose else r).astype(np.float64)
        err = np.abs(got - ref).max()
        assert err < 1e-4, err


@pytest.mark.parametrize("d,hk,group,mode", [(256, 1, 6, "write"), (128, 2, 4, "write"), (256, 1, 6, "write_clip"),
                                             (128, 2, 4, "invalidate")])
def test_decode_write_sees_the_window_as_the_store_leaves_it(cuda, d, hk, group, mode):
    """oscar_decode_write_v1 (store + decode in one call, the small store's quantization
    in the merge launch): request 1's new tokens are written onto the window seats of
    request 0's last four history tokens (an 8-row arena), whose keys dominate request
    0's scores (key ramp).  The decode must see those seats as the store leaves them --
    the old tokens back on their INT2 codes -- and the window, tags and bytes must end
    as the oracle's."""
    import copy
    import math
    from oscar_amd import ops
    from oscar_amd._lib import STAGE_INVALIDATE, STAGE_WRITE
    from oracle.store import Staging, clip, store_ref

    bs, prefixes = 128, [3000, 700]
    c = cases.make_case(prefixes, [4, 4], fresh=True, seed=93, key_ramp=4.0, hk=hk, group=group, d=d)
    bt = c["bt"]
    st = Staging(bs, hk, d, 128, 256, 1024)  # 8 rows: blocks share rows
    sk0, sv0, own0 = c["stage"]
    # request 0's four staged window tokens with the largest scores (over its query rows)
    # are the ones request 1's new tokens will evict
    win = np.arange(prefixes[0] - 256, prefixes[0])
    q0 = c["q"][c["qsl"][0]:c["qsl"][1]].reshape(-1, hk, group, d)
    kw = np.stack([sk0[int(bt[0, q // bs]) % own0.shape[0], q % bs] for q in win])  # [256, hk, d]
    score = np.max(np.stack([(q0[:, h] @ kw[:, h].T).max(axis=(0, 1)) for h in range(hk)]), axis=0)
    p = np.sort(win[np.argsort(score)[-4:]])
    last = {(int(bt[0, q // bs]), int(q % bs)) for q in p}
    staged = [(int(b), col, r0) for r0 in range(own0.shape[0]) for col in range(bs) if (b := own0[r0, col]) >= 0]
    for b, col, r0 in sorted(staged, key=lambda x: (x[0], x[1]) in last):  # the chosen tokens win
        st.owner[b % st.rows, col] = b
        st.stage_k[b % st.rows, col], st.stage_v[b % st.rows, col] = sk0[r0, col], sv0[r0, col]
    used = set(bt[0, :math.ceil(c["seqs"][0] / bs)].tolist()) | set(bt[1, :math.ceil(c["seqs"][1] / bs)].tolist())
    free = [b for b in range(c["k8"].shape[0]) if b not in used]
    blk = [int(bt[0, q // bs]) for q in p]
    target = [next(b for b in free if b % st.rows == x % st.rows) for x in blk]
    pos0 = np.arange(prefixes[0], prefixes[0] + 4)
    slots = np.concatenate([bt[0, pos0 // bs].astype(np.int64) * bs + pos0 % bs,
                            np.array(target, np.int64) * bs + (p % bs).astype(np.int64)])
    # the oracle: the window after the store (identity rotations), then the attention
    post = copy.deepcopy(st)
    if mode == "invalidate":  # a standalone KV update: the rewritten seats lose their copies
        post.invalidate(slots)
        assert all(post.owner[b % st.rows, q % bs] == -1 for b, q in zip(blk, p))
    else:
        post.write(c["k"], c["v"], slots, c["qsl"], c["seqs"])
        assert all(post.owner[b % st.rows, q % bs] == t for b, q, t in zip(blk, p, target))
    ref_o, ref_l = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], bt, c["qsl"], c["seqs"], c["scale"],
                                 post.arrays())
    pre_o, _ = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], bt, c["qsl"], c["seqs"], c["scale"],
                             st.arrays())
    gap = np.abs(ref_o - pre_o).max()
    print(f"window before vs after the store: max|dO| {gap:.3e}", flush=True)
    assert gap > 5 * OUT_TOL  # the case tells the two windows apart
    kc = torch.from_numpy(c["k8"].copy()).view(torch.int8).cuda()
    vc = torch.from_numpy(c["v8"].copy()).view(torch.int8).cuda()
    sk, sv, own = (torch.from_numpy(a.copy()).cuda() for a in st.arrays())
    n, hq = c["q"].shape[:2]
    q_rot = torch.empty(n, hq, d, dtype=torch.bfloat16, device="cuda")
    k_rot = torch.empty(n, hk, d, dtype=torch.bfloat16, device="cuda")
    v_rot = torch.empty_like(k_rot)
    plan = ops.plan_decode(c["qsl"], c["seqs"], has_new=True, num_kv_heads=hk, group=group, head_dim=d,
                           device=torch.device("cuda"), window=(st.sink_eff, 256))
    clips = (0.96, 0.92) if mode == "write_clip" else (0.0, 0.0)
    win_kw = dict(stage_mode=STAGE_INVALIDATE) if mode == "invalidate" else dict(
        stage_mode=STAGE_WRITE, qsl_dev=torch.tensor(c["qsl"], dtype=torch.int32, device="cuda"),
        seqs_dev=torch.tensor(c["seqs"], dtype=torch.int32, device="cuda"), num_reqs=2, recent_tokens=256,
        sink_tokens_eff=st.sink_eff)
    store = ops.store_args(dev(c["k"]), dev(c["v"]), kc, vc, torch.from_numpy(slots).cuda(), head_dim=d,
                           k_clip=clips[0], v_clip=clips[1], stage=(sk, sv, own), query=dev(c["q"]),
                           query_rot=q_rot, key_rot=k_rot, value_rot=v_rot, **win_kw)
    out, lse = ops.attention_decode(q_rot, k_rot, v_rot, kc, vc, torch.from_numpy(bt).cuda(), plan, c["scale"],
                                    (sk, sv, own), head_dim=d, store=store)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), lse.cpu().numpy(), ref_o, ref_l, f"decode_write over rewritten seats ({mode})")
    k8, v8 = c["k8"].copy(), c["v8"].copy()
    if clips[0]:
        store_ref(clip(c["k"], clips[0]), clip(c["v"], clips[1]), k8, v8, slots)
    else:
        store_ref(c["k"], c["v"], k8, v8, slots)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v8)
    assert np.array_equal(own.cpu().numpy(), post.owner)
    assert np.array_equal(sk.cpu().numpy(), post.stage_k)
    assert np.array_equal(sv.cpu().numpy(), post.stage_v)
