"""Helpers shared by the GPU parity tests: case setup through the oracle
(checker) and the HIP backend (product)."""
import numpy as np

import oracle as O

ATOL, RTOL = 2e-3, 1e-2  # fp32 attention output tolerance (max-abs / rel)


def assert_close(got, want, atol=ATOL, rtol=RTOL, what="output"):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    if bad.any():
        i = int(np.argmax(err - (atol + rtol * np.abs(want))))
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside atol={atol} rtol={rtol}; "
                             f"worst index {i}: got {got.flat[i]!r} want {want.flat[i]!r}; max abs err {err.max():.3e}")
    return float(err.max())


def assert_bits_equal(got, want, what="rows"):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    diff = got != want
    if diff.any():
        i = int(np.argmax(diff.reshape(-1)))
        raise AssertionError(f"{what}: {int(diff.sum())} of {diff.size} differ; first at {i}: "
                             f"got {int(got.reshape(-1)[i]):#06x} want {int(want.reshape(-1)[i]):#06x}")
