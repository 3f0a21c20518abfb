"""Pins the oracle's int8 matvec and row dequantization.

Mirrors the reference's own CQ tests (tests/cq.test.ts:74-99): batch equals
single with a row range, and the direct matvec equals a dot with the
dequantized row, on the same input vectors (cos(i + 0.5), sin(i + 0.25)).
Adds closed forms (W == c, x == e_k) and float64 numpy matmuls.
"""

import numpy as np
import pytest

import oracle
from helpers import assert_close


def mat(rng, n, k, g):
    w = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s = rng.uniform(0.001, 0.02, size=(n, k // g)).astype(np.float32)
    return w, s


def dense(w, s, g):
    n, k = w.shape
    return w.astype(np.float64) * np.repeat(s.astype(np.float64), g, axis=1)


def test_direct_equals_dequantized_row_dot(rng):
    w, s = mat(rng, 2, 8 * 16, 16)
    x = np.cos(np.arange(128) + 0.5).astype(np.float32)
    y = oracle.matvec_i8(w, s, 16, x)
    for r in range(2):
        row = oracle.row_i8(w, s, 16, r)
        assert abs(float(y[r]) - float(np.dot(row.astype(np.float64), x))) < 1e-4


def test_batch_and_range_equal_single(rng):
    w, s = mat(rng, 6, 64, 32)
    x = np.sin(np.arange(64) + 0.25).astype(np.float32)
    full = oracle.matvec_i8(w, s, 32, x)
    part = oracle.matvec_i8(w, s, 32, x, row_start=1, row_count=3)
    assert np.array_equal(part, full[1:4])
    xb = np.stack([x, -x, 2 * x])
    yb = oracle.matvec_i8(w, s, 32, xb)
    for b in range(3):
        assert np.array_equal(yb[b], oracle.matvec_i8(w, s, 32, xb[b]))


@pytest.mark.parametrize("n,k,g", [(7, 64, 16), (16, 512, 512), (33, 256, 32)])
def test_against_float64_matmul(rng, n, k, g):
    w, s = mat(rng, n, k, g)
    x = rng.normal(size=(3, k)).astype(np.float32)
    ref = x.astype(np.float64) @ dense(w, s, g).T
    got = oracle.matvec_i8(w, s, g, x)
    assert_close(got, ref, rtol=1e-6, atol=1e-6, what="oracle vs float64 matmul")
    # The oracle's f32 store is a single rounding of a float64 sum.
    assert np.max(np.abs(got - ref.astype(np.float32))) <= np.max(np.abs(ref)) * 2e-7


def test_closed_forms(rng):
    n, k, g = 4, 128, 32
    w = np.full((n, k), 3, np.int8)
    s = rng.uniform(0.001, 0.02, size=(n, k // g)).astype(np.float32)
    x = rng.normal(size=k).astype(np.float32)
    y = oracle.matvec_i8(w, s, g, x)
    gs = x.astype(np.float64).reshape(k // g, g).sum(axis=1)
    expect = 3 * (s.astype(np.float64) * gs[None, :]).sum(axis=1)
    assert_close(y, expect, rtol=1e-7, atol=1e-7)
    w2, s2 = mat(rng, n, k, g)
    for col in (0, 31, 32, 127):
        e = np.zeros(k, np.float32)
        e[col] = 1
        y = oracle.matvec_i8(w2, s2, g, e)
        assert np.array_equal(y, (w2[:, col].astype(np.float64) * s2[:, col // g]).astype(np.float32))


def test_row_is_exact_product(rng):
    w, s = mat(rng, 5, 96, 32)
    for r in range(5):
        expect = (w[r].astype(np.float64) * np.repeat(s[r], 32)).astype(np.float32)
        assert np.array_equal(oracle.row_i8(w, s, 32, r), expect)


def test_invalid_ranges(rng):
    w, s = mat(rng, 4, 32, 16)
    with pytest.raises(oracle.OracleError):
        oracle.matvec_i8(w, s, 16, np.zeros(32, np.float32), row_start=3, row_count=2)
