"""FP32 staging-window comparison shared by the GPU tests (not a test module).

Calls of at most 64 tokens write the window from the fp64 rotation (bit-exact with the
oracle); larger calls write y~, the certified MFMA rotation, whose distance from the
correctly rounded y is bounded by 2^-20 ||x|| ||R_:d|| + 2^-22 |y| for bf16 / fp16
inputs (the bound the store kernel certifies its bytes with).  The check takes the
largest ||x|| of the inputs written and the largest column norm of R; seats no call
wrote keep their earlier values, which the bound compares exactly enough (their error
is 0)."""
import numpy as np


def assert_window_close(got, want, xs, r, label="window"):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    nx = max(np.linalg.norm(np.asarray(x, np.float64).reshape(-1, np.shape(x)[-1]), axis=-1).max() for x in xs)
    cn = np.linalg.norm(np.asarray(r, np.float64), axis=0).max()
    tol = 2.0 ** -20 * nx * cn + 2.0 ** -22 * np.abs(want) + 2.0 ** -126
    err = np.abs(got - want)
    assert np.all(err <= tol), f"{label}: error {err.max():.3g} above the rotation bound"
    print(f"{label}: {(got != want).mean():.3%} of values differ, max error {err.max():.3g}", flush=True)
