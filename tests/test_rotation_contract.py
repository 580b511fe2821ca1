"""The store's rotation contract against the reference's fp32 sgemm (backend.py:130-148).

The store writes the codes, scales and zeros of the correctly rounded rotation
y = RN(x @ R) (the oracle's ``store.rotate``); the reference writes those of torch's
CPU sgemm result (``store.rotate_f32gemm``), whose last bits depend on the BLAS
blocking.  At config-2 inputs (15360 tokens, N(0, 1) bf16 with four x8 outlier
channels, K and V, with and without the serve defaults' clip 0.96):

* a seeded random-sign Hadamard R gives identical bytes for every vector;
* a seeded QR rotation gives different bytes for at most 1 vector in 1000, and only for
  vectors whose correctly rounded y lies within the sgemm's own error of a decision of
  the quantizer (format.py:51-88): the fp16 rounding of the zero or of the scale, or a
  code boundary.  The clip threshold is an order statistic, 1-Lipschitz in the values,
  so clipping moves no element by more than the largest element error.
"""
import numpy as np
import pytest

from oracle import cases, fmt, store

N, D = 15360, 256
BOUND = N // 1000  # differing vectors allowed per kind with a non-Hadamard rotation


def _bytes(y):
    """Per-vector concatenation of the stored bytes' sources: codes, scale, zero."""
    packed, scale, zero = fmt.quantize(y)
    return np.concatenate([packed.reshape(N, -1).astype(np.float32), scale.reshape(N, -1),
                           zero.reshape(N, -1)], axis=1)


def _f16_margin(v):
    """Distance of fp32 values v >= 0 to the nearest fp16 rounding midpoint."""
    v = np.asarray(v, np.float64)
    h = v.astype(np.float16)
    up = np.nextafter(h, np.float16(np.inf)).astype(np.float64)
    dn = np.nextafter(h, np.float16(-np.inf)).astype(np.float64)
    hf = h.astype(np.float64)
    return np.minimum(np.abs(v - (hf + up) / 2), np.abs(v - (hf + dn) / 2))


def _near_a_boundary(y, err):
    """Vectors whose quantizer decisions could change when every element moves by at most
    err (per vector): the zero's or the scale's fp16 rounding, or a code boundary at
    t = 1, 2, 3 of t = (y - zero) / scale + 0.5, with a few fp32 ulps of slack for the
    quantizer's own roundings."""
    y = y.reshape(N, D).astype(np.float64)
    e = err.reshape(N).astype(np.float64)
    vmin, vmax = y.min(-1), y.max(-1)
    raw = (vmax - vmin) / 3
    ulp = np.spacing(np.float32(np.maximum(np.abs(raw), 2.0 ** -14))).astype(np.float64)
    near_scale = (raw > 2.0 ** -14 - 2 * e / 3) & (_f16_margin(raw) <= 2 * e / 3 + 4 * ulp)
    near_zero = _f16_margin(np.abs(vmin)) <= e + np.spacing(np.float32(np.abs(vmin)))
    packed, scale, zero = fmt.quantize(y.astype(np.float32).reshape(N, 1, D))
    s = scale.reshape(N, 1).astype(np.float64)
    z = zero.reshape(N, 1).astype(np.float64)
    t = (y - z) / s + 0.5
    dist = np.min(np.abs(t[..., None] - np.array([1.0, 2.0, 3.0])), axis=-1)
    near_code = (dist <= e[:, None] / s + 2.0 ** -19 * np.maximum(np.abs(t), 1)).any(-1)
    return near_scale | near_zero | near_code


ROTATIONS = {
    "hadamard": lambda: cases.hadamard_rotation(D, cases.BASE_SEED + 2),
    "qr": lambda: cases.qr_rotation(D, cases.BASE_SEED + 12),
}


@pytest.mark.parametrize("clip", [0.0, 0.96])
@pytest.mark.parametrize("name", sorted(ROTATIONS))
def test_store_bytes_follow_the_reference_sgemm_except_at_decision_boundaries(name, clip):
    r = ROTATIONS[name]()
    for seed in (cases.BASE_SEED + 20, cases.BASE_SEED + 21):  # K and V inputs
        x = cases.kv_outliers(N, 1, D, seed)
        exact = store.clip(store.rotate(x, r), clip)
        sgemm = store.clip(store.rotate_f32gemm(x, r), clip)
        differ = (_bytes(exact) != _bytes(sgemm)).any(-1)
        if name == "hadamard":
            assert not differ.any()
            continue
        assert differ.sum() <= BOUND, differ.sum()
        err = np.abs(exact - sgemm).reshape(N, D).max(-1)
        near = _near_a_boundary(exact, err)
        # the differences are the boundary cases the sgemm's error can reach ...
        assert not (differ & ~near).any(), np.flatnonzero(differ & ~near)
        # ... and the boundary set is a small fraction, so the inclusion pins something
        assert near.sum() < 0.05 * N, near.sum()
        # the sgemm's error itself stays far below the attention tolerance
        assert (err <= 2.0 ** -20 * np.linalg.norm(x.reshape(N, D), axis=-1) * 8).all()
