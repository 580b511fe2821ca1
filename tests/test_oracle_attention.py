"""Pins the oracle's read path (oracle/attention.py, oracle/backend.py) on the CPU.

Closed forms restate the reference's lifecycle tests
(tests/test_streaming_backend.py:58-185, tests/test_backend.py:303-370) with the
reference fixture's geometry (D=64, block 4, 8 blocks, Hk=1, Hq=2, sink 4,
recent 4, staging 8, identity rotation, fp32 queries).  The softmax itself is
checked against torch's scaled_dot_product_attention in float64 over
independently decoded history, and the LSE merge against hand-derived values
and the split-softmax identity.
"""
import math

import numpy as np
import pytest
import torch

from oracle import cases, fmt
from oracle.attention import attention_ref, merge_ref, causal_prefill_ref
from oracle.backend import OracleLayer, do_kv_cache_update, forward, staging_write
from oracle.store import store_ref

D, BS, NB = 64, 4, 8
BT = [[0, 1, 2, 3]]


def layer(window=True, rk=None, rv=None):
    eye = np.eye(D, dtype=np.float32)
    return OracleLayer(k8=np.zeros((NB, BS, 1, D), np.uint8), v8=np.zeros((NB, BS, 1, D), np.uint8),
                       rk=eye if rk is None else rk, rv=eye if rv is None else rv, hq=2, hk=1, d=D,
                       scale=D ** -0.5, sink_tokens=4, recent_tokens=4, staging_tokens=8,
                       window_enabled=window)


def const(rows, value):
    return np.full((rows, 1, D), value, np.float32)


def run(L, q, k, v, slots, ends, seqs, bt=BT, **kw):
    return forward(L, q, k, v, slots, [0] + ends, seqs, np.asarray(bt), q_dtype="f32", **kw)


# ------------------------------------------------------------- closed forms
def test_cache_only_update_invalidates_window_mean_is_3():
    # tests/test_streaming_backend.py:58-78: staged ones, token 1 rewritten to 9
    L = layer()
    old = const(4, 1.0)
    do_kv_cache_update(L, old, old, np.arange(4))
    staging_write(L, old, old, [0, 1, 2, 3], [0, 4], [4])
    do_kv_cache_update(L, const(1, 9.0), const(1, 9.0), [1])
    out = run(L, np.zeros((1, 2, D), np.float32), None, None, [], [1], [4], num_actual_tokens=1)
    assert np.array_equal(out, np.full_like(out, 3.0))  # mean(1, 9, 1, 1)


def test_rejected_mtp_tail_and_recycled_blocks_cannot_leak():
    # tests/test_streaming_backend.py:81-144
    L = layer()
    oldv = np.broadcast_to(np.arange(6, dtype=np.float32)[:, None, None], (6, 1, D)).copy()
    oldk = np.zeros_like(oldv)
    do_kv_cache_update(L, oldk, oldv, np.arange(6))
    staging_write(L, oldk, oldv, list(range(6)), [0, 6], [6])
    firstv = np.broadcast_to(np.array([10.0, 100.0, 1000.0, 10000.0], np.float32)[:, None, None],
                             (4, 1, D)).copy()
    run(L, np.zeros((4, 2, D), np.float32), np.zeros_like(firstv), firstv, [6, 7, 8, 9], [4], [10])
    # only token 6 was accepted: positions 7 and 8 are replaced, 9 is invisible
    secondv = np.broadcast_to(np.array([20.0, 30.0], np.float32)[:, None, None], (2, 1, D)).copy()
    out = run(L, np.zeros((2, 2, D), np.float32), np.zeros_like(secondv), secondv, [7, 8], [2], [9])
    assert np.allclose(out[0], 45 / 8, rtol=1e-6) and np.allclose(out[1], 75 / 9, rtol=1e-6)
    # a new request recycles the same pages: fresh prefill ignores the old data
    out = run(L, np.zeros((4, 2, D), np.float32), const(4, 0.0), const(4, -3.0), [0, 1, 2, 3], [4], [4])
    assert np.array_equal(out, np.full_like(out, -3.0))
    out = run(L, np.zeros((1, 2, D), np.float32), const(1, 0.0), const(1, -8.0), [4], [1], [5])
    assert np.array_equal(out, np.full_like(out, -4.0))  # mean(-3, -3, -3, -3, -8)


def test_cached_long_prefill_sees_history_and_chunk():
    # tests/test_streaming_backend.py:147-158
    L = layer(window=False)
    old = const(4, 1.0)
    do_kv_cache_update(L, old, old, np.arange(4))
    new = const(20, 1.0)
    out = run(L, np.zeros((20, 2, D), np.float32), new, new, list(range(4, 24)), [20], [24],
              bt=[[0, 1, 2, 3, 4, 5]])
    assert np.array_equal(out, np.ones_like(out))


def test_mixed_prefix_free_prefill_and_continuation():
    # tests/test_streaming_backend.py:172-206
    L = layer(window=False)
    old = const(6, 1.0)
    do_kv_cache_update(L, old, old, [24, 25, 26, 27, 28, 29])
    cur = const(21, 1.0)
    out = run(L, np.zeros((21, 2, D), np.float32), cur, cur, list(range(17)) + [30, 31, 20, 21],
              [17, 21], [17, 10], bt=[[0, 1, 2, 3, 4], [6, 7, 5, 0, 0]])
    assert np.array_equal(out, np.ones_like(out))


def test_fresh_prefill_equals_sdpa():
    # tests/test_backend.py:303-334, first step: history-free request == causal SDPA
    g = np.random.default_rng(21)
    q = g.standard_normal((4, 2, D)).astype(np.float32)
    k = g.standard_normal((4, 1, D)).astype(np.float32)
    v = g.standard_normal((4, 1, D)).astype(np.float32)
    out = run(layer(), q, k, v, [0, 1, 2, 3], [4], [4])
    t = lambda x: torch.from_numpy(x).double().transpose(0, 1)
    want = torch.nn.functional.scaled_dot_product_attention(
        t(q), t(k).repeat_interleave(2, 0), t(v).repeat_interleave(2, 0), is_causal=True,
        scale=D ** -0.5).transpose(0, 1).numpy()
    np.testing.assert_allclose(out, want, atol=1e-6, rtol=1e-6)


def test_rotated_forward_equals_original_domain_attention():
    # orthogonal R_k, R_v, history fully staged (fp32, then fp16 as the reference
    # reads it): the rotated path must reproduce original-domain attention
    rk, rv = cases.qr_rotation(D, 22), cases.qr_rotation(D, 23)
    L = layer(rk=rk, rv=rv)
    L.sink_tokens, L.recent_tokens = 0, 16
    g = np.random.default_rng(24)
    oldk, oldv = (g.standard_normal((8, 1, D)).astype(np.float32) for _ in range(2))
    do_kv_cache_update(L, oldk, oldv, np.arange(8))
    staging_write(L, oldk, oldv, list(range(8)), [0, 8], [8])
    assert (L.staging.owner[:2] >= 0).all()
    q = g.standard_normal((3, 2, D)).astype(np.float32)
    k, v = (g.standard_normal((3, 1, D)).astype(np.float32) for _ in range(2))
    out = run(L, q, k, v, [8, 9, 10], [3], [11])
    keys = np.concatenate([oldk, k]).astype(np.float64)[:, 0]
    vals = np.concatenate([oldv, v]).astype(np.float64)[:, 0]
    for i in range(3):
        for h in range(2):
            s = keys[:9 + i] @ q[i, h] * D ** -0.5
            p = np.exp(s - s.max())
            want = p @ vals[:9 + i] / p.sum()
            np.testing.assert_allclose(out[i, h], want, atol=5e-3)


# ------------------------------------------------------------- staging hit rule
def test_history_value_source_follows_owner_tag():
    # cache holds 2.0 everywhere; the window holds 5.0 for block 0 only
    L = layer()
    do_kv_cache_update(L, const(8, 2.0), const(8, 2.0), np.arange(8))
    st = L.ensure_staging()
    st.owner[0, :] = 0
    st.stage_v[0] = 5.0
    st.owner[1, :] = 7  # tag of another physical block: ignored
    st.stage_v[1] = 100.0
    out = run(L, np.zeros((1, 2, D), np.float32), None, None, [], [1], [8], bt=[[0, 1]],
              num_actual_tokens=1)
    assert np.allclose(out, (4 * 5.0 + 4 * 2.0) / 8, rtol=1e-6)


# ------------------------------------------------------------- softmax vs SDPA
@pytest.mark.parametrize("window", [False, True])
def test_attention_ref_matches_sdpa_on_decoded_history(window):
    # tests/test_numeric.py:106-130: same INT2 data, independent decode and softmax
    c = cases.make_case([9, 21, 0, 5], [2, 3, 1, 4], d=D, hk=2, group=3, bs=4, sink=4, recent=4,
                        window=window, seed=25)
    out, lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"], c["seqs"],
                             c["scale"], c["stage"], d=D)
    for r, (a, b, seq) in enumerate(zip(c["qsl"][:-1], c["qsl"][1:], c["seqs"])):
        n, prefix = b - a, seq - (b - a)
        pos = np.arange(prefix)
        blk = c["bt"][r, pos // 4]
        slots = np.zeros((prefix, 2, fmt.SLOT_SIZE), np.uint8)  # logical 160-byte slots
        slots[..., :32 + D // 4] = c["k8"][blk, pos % 4, :, :32 + D // 4]
        slots[..., 96:96 + D // 4] = c["v8"][blk, pos % 4, :, :D // 4]
        kh, vh = fmt.parse_slot_bytes(slots, D)
        if window:
            sk, sv, owner = c["stage"]
            hit = owner[blk % owner.shape[0], pos % 4] == blk
            kh[hit] = sk[blk % owner.shape[0], pos % 4][hit]
            vh[hit] = sv[blk % owner.shape[0], pos % 4][hit]
        kh, vh = fmt.bf16_round(fmt.f16_round(kh)), fmt.bf16_round(fmt.f16_round(vh))
        keys = torch.from_numpy(np.concatenate([kh, c["k"][a:b]])).double().transpose(0, 1)
        vals = torch.from_numpy(np.concatenate([vh, c["v"][a:b]])).double().transpose(0, 1)
        q = torch.from_numpy(c["q"][a:b]).double().transpose(0, 1)
        mask = torch.arange(seq)[None, :] < (prefix + 1 + torch.arange(n))[:, None]
        want = torch.nn.functional.scaled_dot_product_attention(
            q, keys.repeat_interleave(3, 0), vals.repeat_interleave(3, 0), attn_mask=mask,
            scale=c["scale"]).transpose(0, 1).numpy()
        np.testing.assert_allclose(out[a:b], want, atol=1e-6, rtol=1e-5)
        s = torch.einsum("hqd,hkd->hqk", q, keys.repeat_interleave(3, 0)) * c["scale"]
        want_lse = torch.logsumexp(s.masked_fill(~mask, -math.inf), -1).transpose(0, 1).numpy()
        np.testing.assert_allclose(lse[a:b], want_lse, atol=1e-6, rtol=1e-6)


def test_empty_rows_and_leading_empty_queries():
    # tests/test_slab_attention.py:38-46: cache-only rows that see nothing
    c = cases.make_case([3, 35, 0], [7, 17, 2], d=D, bs=4, fresh=False, window=False, seed=26,
                        group=2)
    out, lse = attention_ref(c["q"], None, None, c["k8"], c["v8"], c["bt"], c["qsl"], c["seqs"],
                             c["scale"], None, d=D)
    # request 0: seq 3, 7 queries -> query i sees 3 - 7 + i + 1 keys: the first 4 see none
    assert (out[:4] == 0).all() and np.isneginf(lse[:4]).all()
    assert np.isfinite(lse[4:7]).all()
    assert (out[-2:] == 0).all() and np.isneginf(lse[-2:]).all()


def test_nan_query_propagates():
    # tests/test_streaming_attention.py:250-256: invalid scores are not ignored
    c = cases.make_case([9], [2], d=D, bs=4, window=False, seed=27, group=2)
    c["q"][0, 0, 0] = np.nan
    out, lse = attention_ref(c["q"], c["k"], c["v"], c["k8"], c["v8"], c["bt"], c["qsl"], c["seqs"],
                             c["scale"], None, d=D)
    assert np.isnan(out[0, 0]).all() and np.isnan(lse[0, 0])
    assert np.isfinite(out[1]).all()


def test_causal_prefill_ref_gqa_matches_sdpa():
    g = np.random.default_rng(28)
    q, k, v = (g.standard_normal((7, h, 32)).astype(np.float32) for h in (4, 2, 2))
    out = causal_prefill_ref(q, k, v, 0.3, q_dtype="f32")
    t = lambda x: torch.from_numpy(x).double().transpose(0, 1)
    want = torch.nn.functional.scaled_dot_product_attention(
        t(q), t(k).repeat_interleave(2, 0), t(v).repeat_interleave(2, 0), is_causal=True,
        scale=0.3).transpose(0, 1).numpy()
    np.testing.assert_allclose(out, want, atol=1e-6, rtol=1e-6)


# ------------------------------------------------------------- LSE merge
def test_merge_known_answers():
    # slab_attention.py:341-356 semantics, values derived by hand
    g = np.random.default_rng(29)
    out = g.standard_normal((3, 2, 8)).astype(np.float32)
    lse = np.array([[-np.inf, 1000.0], [2.0, -np.inf], [1.0, 3.0]], np.float32)
    part = g.standard_normal((3, 2, 8)).astype(np.float32)
    plse = np.array([[-np.inf, -1000.0], [np.nan, 4.0], [3.0, -np.inf]], np.float32)
    out[0, 0] = part[0, 0] = np.nan  # values of empty rows are unspecified
    o0, p0 = out.copy(), part.copy()
    merge_ref(out, lse, part, plse, np.arange(3))
    assert (out[0, 0] == 0).all() and np.isneginf(lse[0, 0])           # empty + empty
    assert np.array_equal(out[0, 1], o0[0, 1]) and lse[0, 1] == 1000.0  # e^-2000 underflows
    assert np.isnan(out[1, 0]).all() and np.isnan(lse[1, 0])            # NaN propagates
    assert np.array_equal(out[1, 1], p0[1, 1]) and lse[1, 1] == 4.0     # empty old row
    a = math.exp(-2.0)
    np.testing.assert_allclose(out[2, 0], (o0[2, 0] * a + p0[2, 0]) / (1 + a), rtol=1e-6)
    np.testing.assert_allclose(lse[2, 0], 3 + math.log1p(a), rtol=1e-7)
    assert np.array_equal(out[2, 1], o0[2, 1]) and lse[2, 1] == 3.0     # empty part


def test_merge_of_split_softmax_equals_full_softmax():
    g = np.random.default_rng(30)
    s = g.standard_normal((5, 40)) * 4
    v = g.standard_normal((40, 16))

    def part(lo, hi):
        m = s[:, lo:hi].max(1)
        p = np.exp(s[:, lo:hi] - m[:, None])
        return (p @ v[lo:hi] / p.sum(1)[:, None]).astype(np.float32), (m + np.log(p.sum(1))).astype(np.float32)

    o, l = part(0, 40)
    acc = np.zeros((5, 16), np.float32)
    acc_lse = np.full(5, -np.inf, np.float32)
    for lo, hi in ((0, 7), (7, 31), (31, 40)):
        po, pl = part(lo, hi)
        merge_ref(acc, acc_lse, po, pl, np.arange(5))
    np.testing.assert_allclose(acc, o, atol=1e-5)
    np.testing.assert_allclose(acc_lse, l, atol=1e-5)
