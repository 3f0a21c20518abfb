"""Pins of the oracle's Cactus-Quant functions (CPU only).

What fixes them, beyond the oracle's own text:
  * binary16 decoding: the patterns of the reference's fp16 tests
    (tests/fp16.test.ts:4-20) and numpy's float16 decoding of all 65536
    patterns;
  * the activation rotation: explicit Sylvester Hadamard matrices
    (scipy.linalg.hadamard) per group, and the FWHT self-inverse property of
    tests/cq.test.ts:64-72;
  * the matvec and the row dequantization: the reference's fixture matrices
    (tests/cq.test.ts:20-61: group 8, two rows, norms 1.25 / 0.75, indices
    i % 2^bits, ternary trits 0, 1, 2 stored as crumbs 3, 0, 1) with its
    identity "direct matvec equals a dequantized row dot", codes unpacked
    independently with numpy bit operations times explicit Hadamard
    products, and a closed form for a constant code;
  * packing: the byte values of known code sequences.
"""

import numpy as np
import pytest
from scipy.linalg import hadamard

import oracle
from needle_hip import pack_codes, synth

TERNARY = 5
REF_CODEBOOK = np.concatenate([  # tests/cq.test.ts:35-38
    np.array([-0.5, -0.15, 0.15, 0.5], np.float32),
    np.array([-0.6, -0.4, -0.2, -0.05, 0.05, 0.2, 0.4, 0.6], np.float32),
    ((np.arange(16) - 7.5) / 12).astype(np.float32),
]).astype(np.float32)
SLICE = {2: (0, 4), 3: (4, 12), 4: (12, 28)}


def reference_fixture(bits):
    """The matrix(bits) fixture of tests/cq.test.ts:20-61 (2 rows x group 8)."""
    group, rows = 8, 2
    top = 3 if bits == TERNARY else 1 << bits
    indices = np.arange(rows * group) % top
    encoded = np.where(indices == 0, 3, indices - 1) if bits == TERNARY else indices
    packed = pack_codes(encoded.reshape(rows, group), bits)
    norms = np.array([[np.float16(1.25).view(np.uint16)], [np.float16(0.75).view(np.uint16)]],
                     dtype=np.uint16)
    return packed, norms


def unpack_codes(packed, kpad, bits):
    """Codes [n][kpad] from packed rows: numpy bit unpacking (independent of
    the oracle's shift-and-mask reads)."""
    pb = 2 if bits == TERNARY else bits
    planes = np.unpackbits(packed, axis=1, bitorder="little")[:, : kpad * pb]
    planes = planes.reshape(packed.shape[0], kpad, pb).astype(np.int64)
    return (planes << np.arange(pb)).sum(axis=2)


def dense_weights(packed, norms, codebook, k, g, bits):
    """The effective weight matrix [n][kpad] in the rotated basis:
    codebook value times the group norm, float64."""
    kpad = -(-k // g) * g
    codes = unpack_codes(packed, kpad, bits)
    if bits == TERNARY:
        c = 1.2240064 / np.sqrt(g)
        values = np.array([0.0, c, 0.0, -c])[codes]
    else:
        lo, hi = SLICE[bits]
        values = codebook[lo:hi].astype(np.float64)[codes]
    scale = np.repeat(norms.view(np.float16).astype(np.float64), g, axis=1)
    return values * scale


def rotate(x, k, g):
    """Zero-pad to whole groups, then H_g / sqrt(g) on each group (float64)."""
    kpad = -(-k // g) * g
    v = np.zeros(kpad)
    v[:k] = x
    return (v.reshape(-1, g) @ hadamard(g).T / np.sqrt(g)).reshape(-1)


# --------------------------------------------------------------- binary16

def test_f16_reference_patterns():
    # tests/fp16.test.ts:6-12
    assert oracle.f16_to_f32(0x0000) == 0.0
    assert np.signbit(oracle.f16_to_f32(0x8000)) and oracle.f16_to_f32(0x8000) == 0.0
    assert oracle.f16_to_f32(0x3C00) == 1.0
    assert oracle.f16_to_f32(0xC000) == -2.0
    assert oracle.f16_to_f32(0x7C00) == np.inf
    assert np.isnan(oracle.f16_to_f32(0x7E00))
    assert oracle.f16_to_f32(0x0001) == 2.0**-24
    assert oracle.f16_to_f32(0x7BFF) == 65504.0


def test_f16_all_patterns_match_numpy():
    patterns = np.arange(65536, dtype=np.uint32)
    ours = np.array([oracle.f16_to_f32(int(p)) for p in patterns], dtype=np.float32)
    numpy = patterns.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = ~np.isnan(numpy)
    assert np.array_equal(ours[finite].view(np.uint32), numpy[finite].view(np.uint32))
    assert np.isnan(ours[~finite]).all()


# ------------------------------------------------------- rotated activations

@pytest.mark.parametrize("k,g", [(8, 8), (64, 8), (40, 16), (256, 32), (300, 64), (1024, 128),
                                 (4096, 256)])
def test_prepare_is_grouped_hadamard(k, g):
    x = np.random.default_rng(k * 7 + g).standard_normal(k).astype(np.float32)
    got = oracle.cq_prepare(x, g)
    want = rotate(x, k, g)
    assert got.shape == want.shape
    # float32 butterflies: log2(g) roundings of partial sums of |x| size.
    bound = 4e-7 * np.log2(g) * np.abs(x).sum() / np.sqrt(g) + 1e-7
    assert np.abs(got - want).max() <= bound


def test_prepare_unit_vector_and_self_inverse():
    g = 16
    for i in range(g):
        e = np.zeros(g, np.float32)
        e[i] = 1.0
        got = oracle.cq_prepare(e, g)
        assert np.array_equal(np.abs(got), np.full(g, np.float32(1 / np.sqrt(g))))
    # tests/cq.test.ts:64-72: H(Hx) = n x; here applied to the normalized
    # transform twice it is the identity.
    x = np.arange(1, 9, dtype=np.float32)
    twice = oracle.cq_prepare(oracle.cq_prepare(x, 8), 8)
    np.testing.assert_allclose(twice, x, rtol=0, atol=1e-5)


# ------------------------------------------------------------------ matvec

@pytest.mark.parametrize("bits", [2, 3, 4, TERNARY])
def test_reference_fixture_direct_equals_row_dot(bits):
    packed, norms = reference_fixture(bits)
    x = np.sin(np.arange(8) + 0.25).astype(np.float32)
    direct = oracle.cq_matvec(packed, norms, REF_CODEBOOK, 8, 8, bits, x)
    for row in range(2):
        w = oracle.cq_row(packed, norms, REF_CODEBOOK, 8, 8, bits, row)
        expected = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
        assert abs(direct[row] - expected) < 0.5e-4  # toBeCloseTo(expected, 4)


def test_reference_fixture_batch_and_range():
    # tests/cq.test.ts:74-86 with cos(i + 0.5) inputs.
    packed, norms = reference_fixture(2)
    x = np.cos(np.arange(8) + 0.5).astype(np.float32)
    full = oracle.cq_matvec(packed, norms, REF_CODEBOOK, 8, 8, 2, x)
    part = oracle.cq_matvec(packed, norms, REF_CODEBOOK, 8, 8, 2, x, 1, 1)
    assert part[0] == full[1]
    both = oracle.cq_matvec(packed, norms, REF_CODEBOOK, 8, 8, 2, np.stack([x, 2 * x]))
    assert np.array_equal(both[0], full)


@pytest.mark.parametrize("bits", [2, 3, 4, TERNARY])
@pytest.mark.parametrize("n,k,g", [(8, 64, 8), (5, 40, 16), (9, 256, 32), (4, 300, 64),
                                   (3, 1024, 128)])
def test_matvec_equals_dense_rotated_product(bits, n, k, g):
    packed, norms = synth.cq_matrix(11, f"o{n}x{k}g{g}b{bits}", n, k, g, bits)
    codebook = synth.cq_codebook()
    x = np.random.default_rng(n + k + g + bits).standard_normal((2, k)).astype(np.float32)
    got = oracle.cq_matvec(packed, norms, codebook, k, g, bits, x)
    w = dense_weights(packed, norms, codebook, k, g, bits)
    want = np.stack([w @ rotate(xb, k, g) for xb in x])
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(w).sum(axis=1).max())


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_matvec_constant_code_closed_form(bits):
    # Every code c, every norm 1: a group contributes cb[c] * sum(H x / sqrt g)
    # = cb[c] * sqrt(g) * x[first column of the group].
    n, k, g = 3, 256, 32
    codebook = synth.cq_codebook()
    c = (1 << bits) - 2
    packed = pack_codes(np.full((n, k), c), bits)
    norms = np.full((n, k // g), np.float16(1.0).view(np.uint16), np.uint16)
    x = np.random.default_rng(bits).standard_normal(k).astype(np.float32)
    got = oracle.cq_matvec(packed, norms, codebook, k, g, bits, x)
    lo, _ = SLICE[bits]
    want = float(codebook[lo + c]) * np.sqrt(g) * x[::g].astype(np.float64).sum()
    np.testing.assert_allclose(got, np.full(n, want), rtol=1e-5, atol=1e-5)


def test_ternary_crumb_values():
    # One group of 8 with crumbs 0,1,2,3 twice, norm 1, x = e_0 after the
    # rotation's inverse: the matvec reads back sum of crumb values times
    # the rotated basis vector; against the dense table [0, c, 0, -c].
    g = 8
    packed = pack_codes(np.array([[0, 1, 2, 3, 0, 1, 2, 3]]), TERNARY)
    norms = np.array([[np.float16(1.0).view(np.uint16)]], np.uint16)
    c = 1.2240064 / np.sqrt(g)
    table = np.array([0.0, c, 0.0, -c])[[0, 1, 2, 3, 0, 1, 2, 3]]
    row = oracle.cq_row(packed, norms, REF_CODEBOOK, g, g, TERNARY, 0)
    np.testing.assert_allclose(row, hadamard(g) @ table / np.sqrt(g), rtol=1e-6, atol=1e-7)


# -------------------------------------------------------------------- rows

@pytest.mark.parametrize("bits", [2, 3, 4, TERNARY])
@pytest.mark.parametrize("n,k,g", [(4, 64, 8), (3, 40, 16), (2, 300, 64), (2, 2048, 256)])
def test_row_equals_explicit_hadamard(bits, n, k, g):
    packed, norms = synth.cq_matrix(5, f"r{n}x{k}g{g}b{bits}", n, k, g, bits)
    codebook = synth.cq_codebook()
    w = dense_weights(packed, norms, codebook, k, g, bits)
    for row in range(n):
        got = oracle.cq_row(packed, norms, codebook, k, g, bits, row)
        want = (w[row].reshape(-1, g) @ hadamard(g).T / np.sqrt(g)).reshape(-1)[:k]
        np.testing.assert_allclose(got, want, rtol=1e-5,
                                   atol=2e-7 * np.log2(g) * np.abs(w[row]).sum())


def test_row_constant_code_closed_form():
    g, k = 32, 64
    codebook = synth.cq_codebook()
    packed = pack_codes(np.full((1, k), 5), 4)
    norms = np.full((1, 2), np.float16(0.5).view(np.uint16), np.uint16)
    row = oracle.cq_row(packed, norms, codebook, k, g, 4, 0)
    v = np.float32(np.float32(codebook[12 + 5]) * np.float32(0.5))  # f32(cb * norm)
    head = np.float32(float(np.float32(v * g)) / np.sqrt(g))
    expect = np.zeros(k, np.float32)
    expect[::g] = head
    assert np.array_equal(row, expect)


def test_pack_codes_known_bytes():
    assert pack_codes(np.array([[0, 1, 2, 3]]), 2).tolist() == [[0xE4]]
    assert pack_codes(np.array([list(range(8))]), 3).tolist() == [[0x88, 0xC6, 0xFA]]
    assert pack_codes(np.array([[1, 15]]), 4).tolist() == [[0xF1]]
    assert pack_codes(np.array([[3, 0, 1, 2]]), TERNARY).tolist() == [[0b10010011]]
