"""Pins the oracle's INT2 slot contract (oracle/fmt.py) on the CPU.

Every expectation here is derived by hand from the published format
(oscar_ascend/format.py:19-167) or checked against an independent routine
(torch's bf16 conversion, float64 brute force), never by re-running the
oracle's own formula.
"""
import itertools

import numpy as np
import pytest
import torch

from oracle import fmt


def test_pack_unpack_exhaustive_over_all_bytes():
    # format.py:84-87 / :99-110: byte b holds q[4b+k] in bits 2k..2k+1
    codes = np.array(list(itertools.product(range(4), repeat=4)))[:, ::-1]  # q0 fastest
    packed = fmt.pack(codes)
    assert packed.dtype == np.uint8
    assert np.array_equal(packed[:, 0], np.arange(256, dtype=np.uint8))
    assert np.array_equal(fmt.unpack(np.arange(256, dtype=np.uint8)[:, None], 4), codes)


def test_pack_known_bytes():
    assert fmt.pack(np.array([0, 1, 2, 3]))[0] == 0xE4
    assert fmt.pack(np.array([3, 0, 0, 0]))[0] == 0x03
    assert fmt.pack(np.array([0, 0, 0, 3]))[0] == 0xC0
    assert list(fmt.pack(np.array([1, 1, 1, 1, 2, 2, 2, 2]))) == [0x55, 0xAA]


def test_slot_bytes_known_answer():
    # D=4: K = [0,1,2,3] -> scale (3-0)/3 = 1.0 (fp16 0x3C00), zero 0, codes 0,1,2,3
    #      V = [-1,-1,-1,5] -> scale 2.0 (0x4000), zero -1 (0xBC00), codes 0,0,0,3
    k = np.array([[[0.0, 1.0, 2.0, 3.0]]], np.float32)
    v = np.array([[[-1.0, -1.0, -1.0, 5.0]]], np.float32)
    slot = fmt.make_slot_bytes(k, v)[0, 0]
    assert slot.shape == (160,)
    assert list(slot[:8]) == [0x00, 0x3C, 0x00, 0x00, 0x00, 0x40, 0x00, 0xBC]
    assert (slot[8:32] == 0).all()
    assert slot[32] == 0xE4 and (slot[33:96] == 0).all()
    assert slot[96] == 0xC0 and (slot[97:] == 0).all()
    kr, vr = fmt.parse_slot_bytes(slot[None, None], 4)
    assert np.array_equal(kr[0, 0], k[0, 0]) and np.array_equal(vr[0, 0], v[0, 0])


def test_rounding_is_floor_plus_half_not_banker():
    # zero 0, scale 1: 0.5 -> 1 and 2.5 -> 3 (round-half-even would give 0 and 2)
    q, s, z = fmt.quantize_codes(np.array([0.0, 0.5, 2.5, 3.0], np.float32))
    assert s[0] == 1.0 and z[0] == 0.0
    assert list(q) == [0, 1, 3, 3]


def test_scale_is_fp16_rounded_before_coding():
    # range 1 -> scale 1/3, fp16(1/3) = 1365/4096.  x = 1.5 * s16 is exactly on the
    # 1|2 boundary with the fp16 scale (code 2); with the fp32 scale it would be 1.
    s16 = 1365 / 4096
    x = np.array([0.0, 1.5 * s16, 1.0, 1.0], np.float32)
    q, s, z = fmt.quantize_codes(x)
    assert s[0] == np.float32(s16) and z[0] == 0.0
    assert list(q) == [0, 2, 3, 3]


def test_zero_is_fp16_rounded_minimum():
    x = np.array([0.1, 0.2, 0.3, 0.4], np.float32)
    _, s, z = fmt.quantize_codes(x)
    assert z[0] == np.float32(np.float16(0.1))
    assert np.float16(z[0]).view(np.uint16) == 0x2E66
    assert s[0] == np.float32(np.float16(np.float32(0.4 - np.float32(0.1)) / 3))


@pytest.mark.parametrize("value", [0.0, 1.0, -1.25, 1e-7])
def test_constant_vector_quantization(value):
    # reference tests/test_backend.py:139-146
    x = np.full((2, 1, 64), value, np.float32)
    packed, scale, zero = fmt.quantize(x)
    assert np.isfinite(scale).all() and (scale > 0).all()
    assert (scale == np.float32(2.0 ** -14)).all()  # the floor: fp16 0x0400
    lo, hi = fmt.f16_le(scale)
    assert (lo == 0x00).all() and (hi == 0x04).all()
    out = fmt.dequant(packed, scale, zero, 64)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, x, atol=1e-5, rtol=1e-3)


def test_codes_are_nearest_level_brute_force():
    g = np.random.default_rng(5)
    x = (g.standard_normal((64, 256)) * g.uniform(0.1, 10, (64, 1))).astype(np.float32)
    x[::7, ::13] *= 8  # outlier channels
    q, s, z = fmt.quantize_codes(x)
    t = (x.astype(np.float64) - z) / s  # exact-ish position on the level grid
    want = np.clip(np.floor(t + 0.5), 0, 3)
    near_tie = np.abs(t + 0.5 - np.round(t + 0.5)) < 1e-5
    assert np.array_equal(q[~near_tie], want[~near_tie])
    # every code's level is within half a step of the value (or clamped at an end)
    err = np.abs(x - (q * s + z)) / s
    inside = (t > -0.5) & (t < 3.5)
    assert (err[inside] <= 0.5 + 1e-5).all()


def test_bf16_round_matches_torch():
    g = np.random.default_rng(6)
    x = np.concatenate([
        g.standard_normal(4096).astype(np.float32) * 100,
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 1.0 + 2 ** -8,
                  1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20], np.float32)])
    want = torch.from_numpy(x).bfloat16().float().numpy()
    assert np.array_equal(fmt.bf16_round(x), want)
    assert np.isnan(fmt.bf16_round(np.array([np.nan], np.float32))).all()


def test_f16_le_round_trip_and_sign():
    x = np.array([1.0, -2.0, 65504.0, 2.0 ** -14, -0.0], np.float32)
    lo, hi = fmt.f16_le(x)
    assert (lo[0], hi[0]) == (0x00, 0x3C)
    assert (lo[1], hi[1]) == (0x00, 0xC0)
    assert (lo[2], hi[2]) == (0xFF, 0x7B)
    assert (lo[4], hi[4]) == (0x00, 0x80)
    assert np.array_equal(fmt.f16_from_le(lo, hi), x)


def test_check_d_limits():
    fmt.check_d(256)
    with pytest.raises(ValueError):
        fmt.check_d(258)  # not a multiple of 4
    with pytest.raises(ValueError):
        fmt.check_d(260)  # 65 code bytes exceed the 64-byte K region
