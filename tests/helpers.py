"""Assertion helpers shared by the test modules."""

import numpy as np


def assert_close(actual, expected, rtol=1e-3, atol=1e-4, what=""):
    """The fp32 parity bar: |a - e| <= atol + rtol * |e| elementwise."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    err = np.abs(actual - expected)
    bound = atol + rtol * np.abs(expected)
    bad = ~(err <= bound)
    if bad.any():
        i = int(np.flatnonzero(bad.reshape(-1))[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside rtol={rtol} atol={atol}; first at flat "
            f"index {i}: got {actual.reshape(-1)[i]!r}, want {expected.reshape(-1)[i]!r}; "
            f"max abs err {float(err.max()):.3e}")
