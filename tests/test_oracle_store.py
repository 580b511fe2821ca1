"""Pins the oracle's write path (oracle/store.py, oracle/backend.py) on the CPU.

Known answers restate the reference's own tests for this path
(tests/test_backend.py:56-118, tests/test_numeric.py:82-103 and :354-367,
tests/test_backend.py:436-451) with the reference fixture's geometry
(D=64, block 4, 8 blocks, Hk=1, sink 4, recent 4, staging 8); the rotation is
checked against exact rational arithmetic.
"""
from fractions import Fraction

import numpy as np
import pytest

from oracle import cases, fmt
from oracle.backend import OracleLayer, do_kv_cache_update, staging_write
from oracle.store import Staging, clip, rotate, staging_order, store_ref

D, BS, NB, HK = 64, 4, 8, 1


def fp32_nearest(fr: Fraction) -> np.float32:
    """Correctly rounded float32 of an exact rational (ties to even)."""
    c = np.float32(float(fr))
    best = c
    for cand in (np.nextafter(c, np.float32(-np.inf)), np.nextafter(c, np.float32(np.inf))):
        e_best, e_cand = abs(Fraction(float(best)) - fr), abs(Fraction(float(cand)) - fr)
        if e_cand < e_best or (e_cand == e_best and int(cand.view(np.uint32)) % 2 == 0):
            best = cand
    return best


def layer(window=True, d=D, rk=None, rv=None):
    eye = np.eye(d, dtype=np.float32)
    return OracleLayer(k8=np.zeros((NB, BS, HK, d), np.uint8), v8=np.zeros((NB, BS, HK, d), np.uint8),
                       rk=eye if rk is None else rk, rv=eye if rv is None else rv, hq=2, hk=HK, d=d,
                       scale=d ** -0.5, sink_tokens=4, recent_tokens=4, staging_tokens=8,
                       window_enabled=window)


# ------------------------------------------------------------------ rotation
def test_rotate_is_correctly_rounded_exact_dot_product():
    g = np.random.default_rng(11)
    x = fmt.bf16_round(g.standard_normal((5, 8)).astype(np.float32))
    r = g.standard_normal((8, 8)).astype(np.float32)  # not symmetric: catches R^T
    got = rotate(x, r)
    for i in range(5):
        for j in range(8):
            exact = sum(Fraction(float(x[i, k])) * Fraction(float(r[k, j])) for k in range(8))
            assert got[i, j] == fp32_nearest(exact), (i, j)


def test_rotate_identity_and_hadamard_closed_form():
    x = cases.bf16_normal((3, 1, 64), 12)
    assert np.array_equal(rotate(x, np.eye(64, dtype=np.float32)), x)
    # e_k @ H = row k of H (entries +-1/8 for D=64)
    h = cases.hadamard(64).astype(np.float32)
    e = np.zeros((1, 64), np.float32)
    e[0, 5] = 1.0
    assert np.array_equal(rotate(e, h)[0], h[5])
    assert set(np.abs(h[5]).tolist()) == {0.125}


# ------------------------------------------------------------------ clip
def test_clip_order_statistic_known_answers():
    x = np.array([[1.0, -5.0, 3.0, 2.0]], np.float32)
    assert np.array_equal(clip(x, 0.5), [[1.0, -3.0, 3.0, 2.0]])    # idx 2 of |x| sorted [1,2,3,5]
    assert np.array_equal(clip(x, 0.25), [[1.0, -2.0, 2.0, 2.0]])   # idx 1
    assert np.array_equal(clip(x, 0.99), x)                          # idx min(3, 3) -> 5
    assert np.array_equal(clip(x, 0.0), x)                           # disabled


def test_clip_threshold_bounds_every_vector():
    # reference tests/test_numeric.py:354-367
    g = np.random.default_rng(13)
    x = (g.standard_normal((4, 1, 32)) * np.array([1.0, 3.0, 8.0, 24.0])[:, None, None]).astype(np.float32)
    y = clip(x, 0.75)
    thr = np.sort(np.abs(x), -1)[..., 24]
    assert (np.abs(y) <= thr[..., None]).all()
    assert np.array_equal(np.abs(y).max(-1), thr)


# ------------------------------------------------------------------ INT2 store
@pytest.mark.parametrize("width", [D, 2 * D])  # packed int8 cache / legacy bf16-sized cache
@pytest.mark.parametrize("hk", [1, 2, 4])
def test_negative_slots_are_skipped(width, hk):
    # reference tests/test_backend.py:56-75
    g = np.random.default_rng(14)
    k = g.standard_normal((3, hk, D)).astype(np.float32)
    v = g.standard_normal((3, hk, D)).astype(np.float32)
    kc, vc = np.zeros((NB, BS, hk, width), np.uint8), np.zeros((NB, BS, hk, width), np.uint8)
    store_ref(k, v, kc, vc, [-1, 2, -1])
    ek, ev = np.zeros_like(kc), np.zeros_like(vc)
    store_ref(k[1:2], v[1:2], ek, ev, [2])
    assert np.array_equal(kc, ek) and np.array_equal(vc, ev)
    before = (kc.copy(), vc.copy())
    store_ref(k, v, kc, vc, [-1, -1, -1])
    assert np.array_equal(kc, before[0]) and np.array_equal(vc, before[1])


def test_split_slot_bytes_equal_logical_slot():
    # reference tests/test_numeric.py:82-103 (bf16-sized cache: 64 bytes per head slot)
    d, h = 32, 2
    g = np.random.default_rng(15)
    k = (g.standard_normal((6, h, d)) * 1.5).astype(np.float32)
    v = (g.standard_normal((6, h, d)) * 1.5).astype(np.float32)
    kc, vc = np.zeros((3, BS, h, 2 * d), np.uint8), np.zeros((3, BS, h, 2 * d), np.uint8)
    store_ref(k, v, kc, vc, np.arange(6))
    want = fmt.make_slot_bytes(k, v)
    got = np.zeros_like(want)
    for t in range(6):
        b, o = divmod(t, BS)
        got[t, :, 0:8] = kc[b, o, :, 0:8]
        got[t, :, 32:32 + d // 4] = kc[b, o, :, 32:32 + d // 4]
        got[t, :, 96:96 + d // 4] = vc[b, o, :, 0:d // 4]
    assert np.array_equal(got, want)
    # nothing else was written: pad bytes and the rest of each slot stay zero
    assert (kc[:, :, :, 8:32] == 0).all() and (kc[:, :, :, 32 + d // 4:] == 0).all()
    assert (vc[:, :, :, d // 4:] == 0).all()


def logical_slot(kc, vc, b, o):
    slot = np.zeros((kc.shape[2], fmt.SLOT_SIZE), np.uint8)
    slot[:, :32 + D // 4] = kc[b, o, :, :32 + D // 4]
    slot[:, 96:96 + D // 4] = vc[b, o, :, :D // 4]
    return slot


def test_repeated_slot_last_writer_wins():
    k = np.stack([np.full((1, D), 1.0), np.full((1, D), 2.0), np.full((1, D), 3.0)]).astype(np.float32)
    kc, vc = np.zeros((NB, BS, 1, D), np.uint8), np.zeros((NB, BS, 1, D), np.uint8)
    store_ref(k, k, kc, vc, [9, 5, 9])
    kr, _ = fmt.parse_slot_bytes(logical_slot(kc, vc, 2, 1), D)
    assert (kr == 3.0).all()
    kr, _ = fmt.parse_slot_bytes(logical_slot(kc, vc, 1, 1), D)
    assert (kr == 2.0).all()


# ------------------------------------------------------------------ staging
def test_staging_geometry():
    st = Staging(BS, HK, D, 4, 4, 8)
    # rows = max(ceil(8/4), sink_pages 1 + tail_pages (ceil(4/4) + 1) + 2) = 5
    assert st.rows == 5 and st.sink_eff == 4
    assert st.owner.shape == (5, 4) and (st.owner == -1).all()
    assert Staging(128, 1, 256, 64, 256, 8192).rows == 64
    assert Staging(128, 1, 256, 64, 256, 8192).sink_eff == 0  # sink rounded down to pages


def test_staging_persists_and_invalidates_recycled_slots():
    # reference tests/test_backend.py:78-96
    L = layer()
    g = np.random.default_rng(16)
    k, v = g.standard_normal((4, 1, D)).astype(np.float32), g.standard_normal((4, 1, D)).astype(np.float32)
    staging_write(L, k, v, [0, 1, 2, 3], [0, 4], [4])
    st = L.staging
    staging_write(L, k[:1] + 5, v[:1], [4], [0, 1], [5])
    assert L.staging is st
    assert np.array_equal(st.stage_k[0], k) and (st.owner[0] == 0).all()
    assert (st.owner[1, 0] == 1) and np.array_equal(st.stage_k[1, 0], k[0] + 5)
    # old physical slots reused by middle tokens (positions 88..99 of a 100-token
    # sequence: only 96..99 are in the recent window) lose their staged copies
    staging_write(L, g.standard_normal((12, 1, D)), g.standard_normal((12, 1, D)), list(range(12)),
                  [0, 12], [100])
    assert (st.owner[0] == -1).all() and (st.owner[1] == -1).all()
    assert (st.owner[2] == 2).all()


def test_staging_collision_owner_matches_value_and_padding_is_ignored():
    # reference tests/test_backend.py:99-109: blocks 0 and `rows` share seat 0
    L = layer()
    L.ensure_staging()
    slot = L.staging.rows * BS
    k = np.stack([np.ones((1, D)), np.full((1, D), 7.0)]).astype(np.float32)
    staging_write(L, k, k, [0, slot], [0, 1, 2, 4], [1, 1, 1])  # third request is padding
    assert L.staging.owner[0, 0] == slot // BS
    assert np.array_equal(L.staging.stage_k[0, 0], k[1])


def test_standalone_update_invalidates_only_rewritten_seats():
    # reference tests/test_streaming_backend.py:62-71
    L = layer()
    old = np.ones((4, 1, D), np.float32)
    do_kv_cache_update(L, old, old, np.arange(4))
    staging_write(L, old, old, [0, 1, 2, 3], [0, 4], [4])
    assert L.staging.owner[0, 1] == 0
    do_kv_cache_update(L, np.full((1, 1, D), 9.0), np.full((1, 1, D), 9.0), [1])
    assert L.staging.owner[0, 1] == -1 and L.staging.owner[0, 0] == 0


def test_staging_values_are_unclipped_rotated_fp32():
    rk = cases.qr_rotation(D, 17)
    L = layer(rk=rk, rv=rk)
    L.k_clip = L.v_clip = 0.5
    x = cases.bf16_normal((1, 1, D), 18)
    do_kv_cache_update(L, x, x, [0])
    staging_write(L, x, x, [0], [0, 1], [1])
    assert np.array_equal(L.staging.stage_k[0, 0], rotate(x, rk)[0])
    # the cache holds the clipped value: its range is at most the clip threshold
    kr, _ = fmt.parse_slot_bytes(logical_slot(L.k8, L.v8, 0, 0), D)
    assert np.abs(kr).max() <= np.sort(np.abs(rotate(x, rk)), -1)[..., 32].max() + 1e-3


@pytest.mark.parametrize("capacity", [8192, 2 ** 24, 2 ** 24 + 2])
def test_staging_order_exact_and_stable_at_float32_boundary(capacity):
    # reference tests/test_backend.py:436-451: stable order of seat ids, exact above 2^24
    seats = np.array([capacity - 1, 0, capacity - 2, capacity - 1, 0])
    assert staging_order(seats, capacity).tolist() == [1, 4, 2, 0, 3]
    if capacity > 2 ** 24:
        # float32 keys would merge capacity-1 and capacity-2 (both round to 2^24)
        wrong = np.argsort(seats.astype(np.float32), kind="stable").tolist()
        assert wrong != [1, 4, 2, 0, 3]
