"""GPU parity of the INT2 write path (oscar_store_v1) against the CPU oracle.

Bar: bit-exact cache bytes (meta + codes, untouched bytes preserved) and owner
tags.  FP32 window values: bit-exact for calls of at most 64 tokens (the fp64
rotation); larger calls keep y~, the MFMA rotation, whose distance from the
correctly rounded y is bounded by 2^-20 ||x|| ||R_:d|| + 2^-22 |y~| (bf16 / fp16
inputs; the kernel's certification bound), unless the vector took the exact pass.
Read-path rotated copies: calls of at most 64 tokens
round the correctly rounded rotation to the input dtype (bit-exact); larger calls
round the MFMA rotation, which lies within 2^-20 ||x|| ||R_:d|| of it, so a copy
is within that bound plus one unit of the dtype, and rarely differs at all (the
reference's own copies come from an fp32 GEMM of unspecified order,
oscar_ascend/backend.py:370-373).
"""
import numpy as np
import pytest
import torch

from oracle import cases, fmt
from oracle.store import Staging, clip, rotate, rotate_f32gemm, store_ref
from window_check import assert_window_close

pytestmark = pytest.mark.gpu


def to_dev(x, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).cuda()


def cache_dev(a):
    return torch.from_numpy(a.copy()).view(torch.int8).cuda()


def slot_mapping(n, capacity, seed, neg=0.05, dup=0.02):
    """Shuffled distinct slots; `neg` of them -1, `dup` repeat an earlier position."""
    g = cases.rng(seed)
    slots = g.permutation(capacity)[:n].astype(np.int64)
    slots[g.random(n) < neg] = -1
    dups = np.nonzero(g.random(n) < dup)[0]
    for i in dups:
        if i > 0:
            slots[i] = slots[g.integers(0, i)]
    return slots


def assert_read_copy(got, x, r, n_tokens, unit=2.0 ** -8):
    """got: the read-path copy (as fp32) of x @ r in a dtype of relative unit `unit`
    (bf16 2^-8, fp16 2^-11): bit-exact for small calls, within the MFMA bound plus
    one unit otherwise."""
    exact = rotate(x, r)
    want = fmt.bf16_round(exact) if unit == 2.0 ** -8 else exact.astype(np.float16).astype(np.float32)
    if n_tokens <= 64:
        assert np.array_equal(got, want)
        return
    nx = np.linalg.norm(np.asarray(x, np.float64), axis=-1, keepdims=True)
    cn = np.linalg.norm(np.asarray(r, np.float64), axis=0)
    tol = 2.0 ** -20 * nx * cn + unit * np.abs(exact)
    assert np.all(np.abs(got.astype(np.float64) - exact) <= tol)
    assert (got != want).mean() < 1e-2, (got != want).mean()


def assert_window(got, want, x, r, n_tokens):
    """FP32 window values: bit-exact for calls of at most 64 tokens, else within the
    MFMA rotation bound (window_check)."""
    if n_tokens <= 64:
        assert np.array_equal(got, want)
    else:
        assert_window_close(got, want, [x], r)


def run_store(k, v, caches, slots, d, rk, rv, **kw):
    from oscar_amd import ops

    k8, v8 = caches
    kc, vc = cache_dev(k8), cache_dev(v8)
    ops.store(to_dev(k), to_dev(v), kc, vc, torch.from_numpy(slots).cuda(), head_dim=d,
              rk=None if rk is None else torch.from_numpy(rk).cuda(),
              rv=None if rv is None else torch.from_numpy(rv).cuda(), **kw)
    torch.cuda.synchronize()
    return kc.view(torch.uint8).cpu().numpy(), vc.view(torch.uint8).cpu().numpy()


# 1500 tokens: last writers via claim tables; 300 tokens: via the slot scan (two
# launches); 64 and 23 tokens: the one-launch path (column slices, last slice quantizes)
@pytest.mark.parametrize("n", [1500, 300, 64, 23])
@pytest.mark.parametrize("d,hk,rot", [(256, 1, "hadamard"), (256, 1, "identity"),
                                      (128, 2, "qr"), (64, 4, "hadamard")])
def test_store_bytes_bit_exact(cuda, d, hk, rot, n):
    bs, nb = 128, 16
    k = cases.kv_outliers(n, hk, d, cases.BASE_SEED + 1)
    v = cases.kv_outliers(n, hk, d, cases.BASE_SEED + 2)
    rk = {"hadamard": cases.hadamard_rotation(d, 3), "qr": cases.qr_rotation(d, 3),
          "identity": None}[rot]
    rv = {"hadamard": cases.hadamard_rotation(d, 4), "qr": cases.qr_rotation(d, 4),
          "identity": None}[rot]
    slots = slot_mapping(n, nb * bs, 5)
    # pre-fill the caches with noise: untouched bytes must survive
    g = cases.rng(6)
    k8, v8 = (g.integers(0, 256, (nb, bs, hk, d), dtype=np.uint8) for _ in range(2))
    got_k, got_v = run_store(k, v, (k8, v8), slots, d, rk, rv)
    eye = np.eye(d, dtype=np.float32)
    ek, ev = k8.copy(), v8.copy()
    store_ref(rotate(k, rk if rk is not None else eye), rotate(v, rv if rv is not None else eye),
              ek, ev, slots)
    assert np.array_equal(got_k, ek), f"K cache bytes differ at {np.argwhere(got_k != ek)[:5]}"
    assert np.array_equal(got_v, ev)


def exact_pass_count(n, hk, d):
    """Vectors the last large call sent to the fp64 pass: the K and V totals that open
    the store workspace of a call of more than 64 tokens (written by the exact pass)."""
    from oscar_amd import ops

    ws = ops.DeviceScratch.get(torch.device("cuda", torch.cuda.current_device())).store_ws
    return int(ws[:8].view(torch.int32).sum().item())


@pytest.mark.parametrize("n", [400, 1500])  # slot scan / claim tables
def test_store_boundary_vectors_take_the_exact_pass(cuda, n):
    """Rotated values that sit on the quantizer's code boundaries cannot be certified
    from the MFMA rotation: those vectors go through the fp64 pass and their bytes
    still equal the oracle's; the others are certified from the MFMA result."""
    d, hk, bs, nb = 256, 1, 128, 16
    g = cases.rng(71)
    r = cases.qr_rotation(d, 72)
    y = g.uniform(-1.0, 2.0, (n, hk, d))
    y[..., 0], y[..., 1] = -1.0, 2.0  # zero -1, scale 1: code boundaries at -0.5, 0.5, 1.5
    edge = np.arange(n) % 2 == 0
    y[edge, :, 2:40] = g.choice([-0.5, 0.5, 1.5], (int(edge.sum()), hk, 38))
    x = (y @ r.astype(np.float64).T).astype(np.float32)  # x R lies within ~1e-7 of y
    slots = slot_mapping(n, nb * bs, 73, neg=0.0, dup=0.0)
    k8, v8 = cases.empty_caches(nb, bs, hk, d)
    from oscar_amd import ops

    kc, vc = cache_dev(k8), cache_dev(v8)
    rd = torch.from_numpy(r).cuda()
    ops.store(to_dev(x, torch.float32), to_dev(x, torch.float32), kc, vc,
              torch.from_numpy(slots).cuda(), head_dim=d, rk=rd, rv=rd)
    torch.cuda.synchronize()
    count = exact_pass_count(n, hk, d)
    yr = rotate(x, r)
    store_ref(yr, yr, k8, v8, slots)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v8)
    assert 2 * edge.sum() <= count < 2 * edge.sum() + 0.2 * n, count


def test_store_fp16_large_call_bit_exact(cuda):
    """fp16 inputs (two bf16 planes per element) through the MFMA path."""
    d, hk, n, bs, nb = 128, 2, 900, 128, 16
    # full 11-bit fp16 significands: the second bf16 plane of x is not zero
    k = (cases.rng(81).standard_normal((n, hk, d)) * 3).astype(np.float16).astype(np.float32)
    v = (cases.rng(82).standard_normal((n, hk, d)) * 3).astype(np.float16).astype(np.float32)
    rk, rv = cases.hadamard_rotation(d, 83), cases.qr_rotation(d, 84)
    slots = slot_mapping(n, nb * bs, 85)
    k8, v8 = cases.empty_caches(nb, bs, hk, d)
    from oscar_amd import ops

    kc, vc = cache_dev(k8), cache_dev(v8)
    k_rot = torch.empty(n, hk, d, dtype=torch.float16, device="cuda")
    ops.store(to_dev(k, torch.float16), to_dev(v, torch.float16), kc, vc,
              torch.from_numpy(slots).cuda(), head_dim=d, rk=torch.from_numpy(rk).cuda(),
              rv=torch.from_numpy(rv).cuda(), key_rot=k_rot)
    torch.cuda.synchronize()
    store_ref(rotate(k, rk), rotate(v, rv), k8, v8, slots)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v8)
    assert_read_copy(k_rot.float().cpu().numpy(), k, rk, n, unit=2.0 ** -11)


@pytest.mark.parametrize("d,hk", [(256, 1), (256, 2), (128, 1)])
def test_store_small_call_rewrites_bit_exact(cuda, d, hk):
    """One-launch calls (<= 64 tokens) with many rewrites of one slot and skipped
    slots: the last writer's bytes land, the others' never do; two calls in a row
    (the arrival counters are left at zero by the first)."""
    bs, nb, n = 128, 4, 48
    rk, rv = cases.qr_rotation(d, 13), cases.hadamard_rotation(d, 14)
    g = cases.rng(15)
    k8, v8 = (g.integers(0, 256, (nb, bs, hk, d), dtype=np.uint8) for _ in range(2))
    ek, ev = k8.copy(), v8.copy()
    for call in range(2):
        k = cases.kv_outliers(n, hk, d, cases.BASE_SEED + 20 + call)
        v = cases.kv_outliers(n, hk, d, cases.BASE_SEED + 30 + call)
        slots = slot_mapping(n, nb * bs, 16 + call, neg=0.1, dup=0.3)
        slots[[5, 17, 40]] = slots[3]  # one slot written four times
        got_k, got_v = run_store(k, v, (k8, v8), slots, d, rk, rv)
        store_ref(rotate(k, rk), rotate(v, rv), ek, ev, slots)
        assert np.array_equal(got_k, ek), f"call {call}: K bytes differ at {np.argwhere(got_k != ek)[:5]}"
        assert np.array_equal(got_v, ev), f"call {call}: V bytes differ"
        k8, v8 = got_k, got_v


def test_store_prerotated_reference_sgemm_bits(cuda):
    """With R = identity the kernel quantizes the reference's own fp32 sgemm output."""
    d, n, bs, nb = 256, 800, 128, 8
    k = cases.kv_outliers(n, 1, d, 11)
    v = cases.kv_outliers(n, 1, d, 12)
    r = cases.hadamard_rotation(d, 13)
    k_rot, v_rot = rotate_f32gemm(k, r), rotate_f32gemm(v, r)
    slots = slot_mapping(n, nb * bs, 14)
    k8, v8 = cases.empty_caches(nb, bs, 1, d)
    from oscar_amd import ops

    kc, vc = cache_dev(k8), cache_dev(v8)
    ops.store(to_dev(k_rot, torch.float32), to_dev(v_rot, torch.float32), kc, vc,
              torch.from_numpy(slots).cuda(), head_dim=d)
    torch.cuda.synchronize()
    store_ref(k_rot, v_rot, k8, v8, slots)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v8)


# the serve defaults 0.96 / 0.92 (delivery/serve_oscar.sh:32-33): calls of <= 64 tokens
# take the one-launch path (clip on the vector handed over by the last column slice),
# 300 tokens the two-launch path
@pytest.mark.parametrize("n", [4, 23, 64, 300])
@pytest.mark.parametrize("d,hk", [(256, 1), (256, 2), (128, 1)])
def test_store_clip_bit_exact(cuda, d, hk, n):
    bs, nb = 128, 4
    k = cases.kv_outliers(n, hk, d, 21)
    v = cases.kv_outliers(n, hk, d, 22)
    rk, rv = cases.hadamard_rotation(d, 23), cases.qr_rotation(d, 24)
    slots = slot_mapping(n, nb * bs, 25)
    k8, v8 = cases.empty_caches(nb, bs, hk, d)
    got_k, got_v = run_store(k, v, (k8, v8), slots, d, rk, rv, k_clip=0.96, v_clip=0.92)
    store_ref(clip(rotate(k, rk), 0.96), clip(rotate(v, rv), 0.92), k8, v8, slots)
    assert np.array_equal(got_k, k8), f"K bytes differ at {np.argwhere(got_k != k8)[:5]}"
    assert np.array_equal(got_v, v8)


def tie_heavy(n, hk, d, seed):
    """Rows whose rotated values tie often: +-1 and +-2 (exact in bf16; no zeros before
    the rotation); every 4th token has one lane's
    whole span of a 16-lane row (elements 2E .. 3E - 1) at a large equal value, so that
    its largest magnitudes all sit in one lane; every 5th token is all zeros (every
    magnitude ties, a zero scale and zero)."""
    g = cases.rng(seed)
    x = g.choice(np.array([-2.0, -1.0, 1.0, 2.0], dtype=np.float32), (n, hk, d))
    e = d // 16
    x[::4, :, 2 * e:3 * e] = 7.0
    x[1::5] = 0.0
    return x


# The sort-clip threshold (the (D - idx)-th largest magnitude) by bisection from a
# lower bound: the one-launch path (<= 64 tokens, one wave per vector) and the large
# path (16-lane rows in the fused launch, the exact pass for the rows it leaves), at
# ratios whose bound is a lane's largest (need <= D / 16), its second largest, or 0
# (need > D / 8), and at need = 1.  (A threshold of exactly 0 over a row with values of
# both signs clips them to -0 and +0, and the sign of their minimum -- the zero point --
# is then whatever the min reduction gives, in the reference's torch amin as here: the
# Hadamard rotations of these rows hold up to 9.4% exact zeros, so the smallest ratio
# here is 0.125.)
@pytest.mark.parametrize("clips", [(0.96, 0.92), (0.5, 0.999), (0.125, 0.5)])
@pytest.mark.parametrize("rot", ["identity", "hadamard"])
@pytest.mark.parametrize("n", [23, 300])
@pytest.mark.parametrize("d,hk", [(256, 1), (128, 2)])
def test_store_clip_threshold_ties_and_bounds(cuda, d, hk, n, rot, clips):
    bs, nb = 128, 4
    k, v = tie_heavy(n, hk, d, 41), tie_heavy(n, hk, d, 42)
    r = cases.hadamard_rotation(d, 43) if rot == "hadamard" else None
    eye = np.eye(d, dtype=np.float32)
    slots = slot_mapping(n, nb * bs, 44)
    k8, v8 = cases.empty_caches(nb, bs, hk, d)
    kc_, vc_ = clips
    got_k, got_v = run_store(k, v, (k8, v8), slots, d, r, r, k_clip=kc_, v_clip=vc_)
    rr = r if r is not None else eye
    store_ref(clip(rotate(k, rr), kc_), clip(rotate(v, rr), vc_), k8, v8, slots)
    assert np.array_equal(got_k, k8), f"K bytes differ at {np.argwhere(got_k != k8)[:5]}"
    assert np.array_equal(got_v, v8), f"V bytes differ at {np.argwhere(got_v != v8)[:5]}"


# the last request of each case is empty; with 100 blocks over 64 staging rows,
# blocks b and b + 64 share seats (collisions resolved by the last writer)
@pytest.mark.parametrize("qsl,seqs,nb", [([0, 700, 705, 1200, 1200], [700, 2000, 496, 10], 32),
                                         ([0, 300, 305, 600, 600], [300, 2000, 496, 10], 100),
                                         ([0, 4, 8, 9, 9], [700, 2000, 496, 10], 100)])  # one launch
def test_store_window_tags_values_and_rotated_outputs(cuda, qsl, seqs, nb):
    """Forward write: codes + owner tags + FP32 window + rotated q/k/v for the read."""
    from oscar_amd import ops
    from oscar_amd._lib import STAGE_WRITE

    d, hk, hq, bs = 256, 1, 6, 128
    n = qsl[-1]
    k = cases.kv_outliers(n, hk, d, 31)
    v = cases.kv_outliers(n, hk, d, 32)
    q = cases.bf16_normal((n, hq, d), 33)
    rk, rv = cases.hadamard_rotation(d, 34), cases.hadamard_rotation(d, 35)
    slots = slot_mapping(n, nb * bs, 36)
    st = Staging(bs, hk, d, 128, 256, 8192)
    # earlier window contents that the collisions / rewrites must replace
    st.owner[:] = np.arange(st.rows)[:, None]
    st.stage_k[:] = 7.0
    k8, v8 = cases.empty_caches(nb, bs, hk, d)
    kc, vc = cache_dev(k8), cache_dev(v8)
    sk, sv, own = (torch.from_numpy(a.copy()).cuda() for a in st.arrays())
    q_rot = torch.empty(n, hq, d, dtype=torch.bfloat16, device="cuda")
    k_rot = torch.empty(n, hk, d, dtype=torch.bfloat16, device="cuda")
    v_rot = torch.empty_like(k_rot)
    ops.store(to_dev(k), to_dev(v), kc, vc, torch.from_numpy(slots).cuda(), head_dim=d,
              rk=torch.from_numpy(rk).cuda(), rv=torch.from_numpy(rv).cuda(),
              stage=(sk, sv, own), stage_mode=STAGE_WRITE,
              qsl_dev=torch.tensor(qsl, dtype=torch.int32, device="cuda"),
              seqs_dev=torch.tensor(seqs, dtype=torch.int32, device="cuda"), num_reqs=len(seqs),
              recent_tokens=256, sink_tokens_eff=st.sink_eff, query=to_dev(q),
              query_rot=q_rot, key_rot=k_rot, value_rot=v_rot)
    torch.cuda.synchronize()
    kr, vr = rotate(k, rk), rotate(v, rv)
    store_ref(kr, vr, k8, v8, slots)
    st.write(kr, vr, slots, qsl, seqs)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v8)
    assert np.array_equal(own.cpu().numpy(), st.owner)
    assert_window(sk.cpu().numpy(), st.stage_k, k, rk, n)
    assert_window(sv.cpu().numpy(), st.stage_v, v, rv, n)
    assert_read_copy(q_rot.float().cpu().numpy(), q, rk, n)
    assert_read_copy(k_rot.float().cpu().numpy(), k, rk, n)
    assert_read_copy(v_rot.float().cpu().numpy(), v, rv, n)


@pytest.mark.parametrize("clips", [(0.0, 0.0), (0.96, 0.92)])
@pytest.mark.parametrize("qsl,seqs", [([0, 700, 705, 1500, 1500], [700, 2000, 1000, 10]),
                                      ([0, 100, 105, 300, 300], [100, 2000, 400, 10]),
                                      ([0, 4, 8, 23, 23], [700, 2000, 496, 10])])
def test_store_window_odd_geometry(cuda, qsl, seqs, clips):
    """Block size, head counts and staging rows that are not powers of two (the
    kernels divide slots, vector indexes and block numbers by them): 48-slot blocks,
    3 KV heads, 5 query heads, 50 blocks over 21 staging rows; with and without the
    serve defaults' sort clip (the bytes of clipped values, the window unclipped)."""
    from oscar_amd import ops
    from oscar_amd._lib import STAGE_WRITE

    d, hk, hq, bs, nb = 128, 3, 5, 48, 50
    n = qsl[-1]
    k = cases.kv_outliers(n, hk, d, 51)
    v = cases.kv_outliers(n, hk, d, 52)
    q = cases.bf16_normal((n, hq, d), 53)
    rk, rv = cases.qr_rotation(d, 54), cases.hadamard_rotation(d, 55)
    slots = slot_mapping(n, nb * bs, 56)
    st = Staging(bs, hk, d, 96, 200, 1000)
    assert st.rows == 21
    st.owner[:] = np.arange(st.rows)[:, None]
    st.stage_k[:] = 7.0
    k8, v8 = cases.empty_caches(nb, bs, hk, d)
    kc, vc = cache_dev(k8), cache_dev(v8)
    sk, sv, own = (torch.from_numpy(a.copy()).cuda() for a in st.arrays())
    q_rot = torch.empty(n, hq, d, dtype=torch.bfloat16, device="cuda")
    k_rot = torch.empty(n, hk, d, dtype=torch.bfloat16, device="cuda")
    v_rot = torch.empty_like(k_rot)
    ops.store(to_dev(k), to_dev(v), kc, vc, torch.from_numpy(slots).cuda(), head_dim=d,
              rk=torch.from_numpy(rk).cuda(), rv=torch.from_numpy(rv).cuda(),
              stage=(sk, sv, own), stage_mode=STAGE_WRITE,
              qsl_dev=torch.tensor(qsl, dtype=torch.int32, device="cuda"),
              seqs_dev=torch.tensor(seqs, dtype=torch.int32, device="cuda"), num_reqs=len(seqs),
              recent_tokens=200, sink_tokens_eff=st.sink_eff, query=to_dev(q),
              query_rot=q_rot, key_rot=k_rot, value_rot=v_rot, k_clip=clips[0], v_clip=clips[1])
    torch.cuda.synchronize()
    kr, vr = rotate(k, rk), rotate(v, rv)
    store_ref(clip(kr, clips[0]), clip(vr, clips[1]), k8, v8, slots)
    st.write(kr, vr, slots, qsl, seqs)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v8)
    assert np.array_equal(own.cpu().numpy(), st.owner)
    assert_window(sk.cpu().numpy(), st.stage_k, k, rk, n)
    assert_window(sv.cpu().numpy(), st.stage_v, v, rv, n)
    assert_read_copy(q_rot.float().cpu().numpy(), q, rk, n)
    assert_read_copy(k_rot.float().cpu().numpy(), k, rk, n)
    assert_read_copy(v_rot.float().cpu().numpy(), v, rv, n)


@pytest.mark.parametrize("n", [23, 1500])  # one-launch path / three launches
def test_store_capacity_past_31_bits(cuda, n):
    """A cache of 2^31 + 2048 slots, where the kernels split slots into block and offset
    with 64-bit division: every block aliases one real block (block stride 0) and the
    tokens' slots lie at distinct offsets of far blocks, so the bytes land in the real
    block at those offsets; seats and owner tags follow the far blocks."""
    import ctypes as C

    from oscar_amd import _lib, ops
    from oscar_amd._lib import STAGE_WRITE

    d, hk, bs = 256, 1, 2048
    nb = (1 << 31) // bs + 1
    g = cases.rng(61)
    offs = g.permutation(bs)[:n].astype(np.int64)
    blocks = (nb - 1 - g.integers(0, 5000, n)).astype(np.int64)
    blocks[::3] = nb - 1  # slots at and past 2^31
    slots = blocks * bs + offs
    slots[g.random(n) < 0.05] = -1
    assert slots.max() >= 1 << 31
    k = cases.kv_outliers(n, hk, d, 62)
    v = cases.kv_outliers(n, hk, d, 63)
    rk, rv = cases.hadamard_rotation(d, 64), cases.qr_rotation(d, 65)
    st = Staging(bs, hk, d, 0, 256, 4 * bs)
    qsl, seqs = [0, n], [n + 100]
    k8, v8 = cases.empty_caches(1, bs, hk, d)
    kc, vc = cache_dev(k8), cache_dev(v8)
    sk, sv, own = (torch.from_numpy(a.copy()).cuda() for a in st.arrays())
    args, keep = ops.store_args(
        to_dev(k), to_dev(v), kc, vc, torch.from_numpy(slots).cuda(), head_dim=d,
        rk=torch.from_numpy(rk).cuda(), rv=torch.from_numpy(rv).cuda(), stage=(sk, sv, own),
        stage_mode=STAGE_WRITE, qsl_dev=torch.tensor(qsl, dtype=torch.int32, device="cuda"),
        seqs_dev=torch.tensor(seqs, dtype=torch.int32, device="cuda"), num_reqs=1,
        recent_tokens=256, sink_tokens_eff=0)
    args.cache.num_blocks = nb
    args.cache.k_stride[0] = 0
    args.cache.v_stride[0] = 0
    claims = torch.zeros(nb * bs, dtype=torch.int64, device="cuda")  # 16 GiB, one per slot
    args.slot_claims = claims.data_ptr()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.load().oscar_store_v1(C.byref(args), stream), "oscar_store_v1")
    torch.cuda.synchronize()
    del claims, keep
    kr, vr = rotate(k, rk), rotate(v, rv)
    store_ref(kr, vr, k8, v8, np.where(slots >= 0, slots % bs, -1))
    st.write(kr, vr, slots, qsl, seqs)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v8)
    assert np.array_equal(own.cpu().numpy(), st.owner)
    assert_window(sk.cpu().numpy(), st.stage_k, k, rk, n)
    assert_window(sv.cpu().numpy(), st.stage_v, v, rv, n)


def test_standalone_update_invalidates_written_seats(cuda):
    from oscar_amd import ops
    from oscar_amd._lib import STAGE_INVALIDATE

    d, bs, nb = 128, 128, 8
    st = Staging(bs, 1, d, 64, 256, 1024)
    st.owner[:] = 5
    slots = np.array([3, -1, 130, 131, 3, 1000], np.int64)
    k = cases.kv_outliers(len(slots), 1, d, 41)
    k8, v8 = cases.empty_caches(nb, bs, 1, d)
    kc, vc = cache_dev(k8), cache_dev(v8)
    sk, sv, own = (torch.from_numpy(a.copy()).cuda() for a in st.arrays())
    ops.store(to_dev(k), to_dev(k), kc, vc, torch.from_numpy(slots).cuda(), head_dim=d,
              stage=(sk, sv, own), stage_mode=STAGE_INVALIDATE)
    torch.cuda.synchronize()
    st.invalidate(slots)
    assert np.array_equal(own.cpu().numpy(), st.owner)
    store_ref(k, k, k8, v8, slots)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)


def test_negative_slots_only_is_a_no_op(cuda):
    d, bs, nb = 256, 128, 2
    k = cases.kv_outliers(5, 1, d, 51)
    g = cases.rng(52)
    k8, v8 = (g.integers(0, 256, (nb, bs, 1, d), dtype=np.uint8) for _ in range(2))
    got_k, got_v = run_store(k, k, (k8, v8), np.full(5, -1, np.int64), d, None, None)
    assert np.array_equal(got_k, k8) and np.array_equal(got_v, v8)


def test_legacy_bf16_geometry(cuda):
    """bf16 caches: 512-byte slots, same packed placement in the first bytes."""
    from oscar_amd import ops

    d, n, bs, nb = 256, 200, 128, 4
    k = cases.kv_outliers(n, 1, d, 61)
    v = cases.kv_outliers(n, 1, d, 62)
    slots = slot_mapping(n, nb * bs, 63, dup=0.0)
    k8, v8 = cases.empty_caches(nb, bs, 1, d, legacy=True)
    kc = torch.from_numpy(k8.copy()).view(torch.bfloat16).cuda()
    vc = torch.from_numpy(v8.copy()).view(torch.bfloat16).cuda()
    ops.store(to_dev(k), to_dev(v), kc, vc, torch.from_numpy(slots).cuda(), head_dim=d)
    torch.cuda.synchronize()
    store_ref(k, v, k8, v8, slots)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k8)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v8)
