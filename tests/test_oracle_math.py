"""Pins the oracle's scalar math (model/math.ts, backends/cq.ts:8-27).

FWHT against the Sylvester Hadamard matrix (scipy.linalg.hadamard) and the
reference's own self-inverse test (tests/cq.test.ts:64-72); RMS norms by
their closed form; RoPE as a complex multiplication by e^{i p theta^(-2j/d)}
on (x_j, x_{j+d/2}) pairs; Sinkhorn's output doubly stochastic; the Hadamard
MLP as explicit matrix products; softmax and sigmoid against scipy.
"""

import numpy as np
import pytest
from scipy.linalg import hadamard
from scipy.special import expit, softmax as sp_softmax

import oracle
from helpers import assert_close


def test_fwht_reference_case():
    out = oracle.fwht(oracle.fwht(np.arange(1, 9, dtype=np.float32)))
    assert np.allclose(out, np.arange(1, 9) * 8, atol=1e-5)


@pytest.mark.parametrize("n", [2, 8, 64, 512])
def test_fwht_is_sylvester_hadamard(rng, n):
    x = rng.normal(size=n).astype(np.float32)
    assert_close(oracle.fwht(x), hadamard(n) @ x.astype(np.float64), rtol=1e-5, atol=1e-4)


def test_fwht_rejects_non_power_of_two():
    with pytest.raises(oracle.OracleError):
        oracle.fwht(np.zeros(12, np.float32))


def test_rms_norm_closed_form(rng):
    x = rng.normal(size=512).astype(np.float32)
    s = rng.uniform(-0.1, 0.1, size=512).astype(np.float32)
    xd = x.astype(np.float64)
    inv = 1 / np.sqrt(np.mean(xd * xd) + 1e-6)
    assert_close(oracle.rms_norm(x, s), (1 + s.astype(np.float64)) * xd * inv, rtol=1e-6, atol=1e-7)
    u = oracle.rms_unit(x)
    assert abs(np.sqrt(np.mean(u.astype(np.float64) ** 2)) - 1) < 1e-5


@pytest.mark.parametrize("position", [0, 1, 17, 2047])
def test_rope_is_complex_rotation(rng, position):
    heads, d = 3, 64
    x = rng.normal(size=heads * d).astype(np.float32)
    got = oracle.rope(x, heads, d, position, 10000.0).reshape(heads, d)
    xr = x.astype(np.float64).reshape(heads, d)
    j = np.arange(d // 2)
    ang = position * 10000.0 ** (-(2 * j) / d)
    z = (xr[:, : d // 2] + 1j * xr[:, d // 2:]) * np.exp(1j * ang)
    expect = np.concatenate([z.real, z.imag], axis=1)
    assert_close(got, expect, rtol=1e-5, atol=1e-5)
    assert_close(np.linalg.norm(got, axis=1), np.linalg.norm(xr, axis=1), rtol=1e-6, atol=1e-6)


def test_sinkhorn_doubly_stochastic(rng):
    logits = rng.normal(size=16).astype(np.float32)
    m = oracle.sinkhorn(logits, 4).reshape(4, 4).astype(np.float64)
    assert np.all(m > 0)
    assert_close(m.sum(axis=0), np.ones(4), rtol=1e-5, atol=1e-6)
    assert_close(m.sum(axis=1), np.ones(4), rtol=1e-3, atol=1e-4)


def test_hadamard_mlp_matrix_form(rng):
    n = h = 64
    x = rng.normal(size=n).astype(np.float32)
    d1, d2, d3 = (rng.uniform(0.5, 1.5, size=h).astype(np.float32) for _ in range(3))
    H = hadamard(h) / np.sqrt(h)
    z = H @ (d1.astype(np.float64) * x)
    z = z * d2
    z = z * expit(z)
    expect = d3 * (H @ z)
    assert_close(oracle.hadamard_mlp(x, d1, d2, d3, h), expect, rtol=1e-5, atol=1e-5)


def test_softmax_and_sigmoid(rng):
    x = rng.normal(size=100).astype(np.float32) * 5
    assert_close(oracle.softmax(x), sp_softmax(x.astype(np.float64)), rtol=1e-6, atol=1e-9)
    for v in [-800.0, -30.0, -1.0, 0.0, 0.5, 30.0, 800.0]:
        assert abs(oracle.sigmoid(v) - expit(v)) <= 1e-15
    assert oracle.softmax(np.zeros(0, np.float32)).size == 0
