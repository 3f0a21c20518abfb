"""GPU parity of Cactus-Quant matrices (CQ2 / CQ3 / CQ4 / ternary) against
the oracle, through the C ABI.

Bars: matvec outputs within 1e-3 relative / 1e-4 absolute of the oracle's
float64 restatement of cqMatvec; dequantized rows bit-exact (dequantizeCqRow
stores float32 after every step, and the HIP kernel makes the same
roundings in the same order).
"""

import ctypes as C
import sys

import numpy as np
import pytest

import oracle
from helpers import DeviceArray, assert_close
from needle_hip import (CqMatrix, Int8Matrix, MatrixRowRange, MatvecRequest, NeedleError,
                        pack_codes, parse_cact, synth, write_cact)
from needle_hip import cact as K
from needle_hip import lib as L

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4
TERNARY = 5
CODEBOOK = synth.cq_codebook()
BOOKS = {b: CODEBOOK[lo:hi] for b, (lo, hi) in K.CODEBOOK_SLICES.items()}


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


def cq(seed, n, k, g, bits):
    packed, norms = synth.cq_matrix(seed, f"cq{n}x{k}g{g}b{bits}", n, k, g, bits)
    return CqMatrix(packed, norms, BOOKS, n, k, g, bits)


def ref_matvec(m, x, row_start=0, row_count=None):
    return oracle.cq_matvec(m.packed.reshape(m.output_size, -1), m.norms, CODEBOOK, m.input_size,
                            m.group_size, m.bits, x, row_start, row_count)


def ref_row(m, row):
    return oracle.cq_row(m.packed.reshape(m.output_size, -1), m.norms, CODEBOOK, m.input_size,
                         m.group_size, m.bits, row)


# (n, k, g): the isolated workload; padded rows (k < kpad, kpad % 32 != 0);
# k % 4 != 0 (scalar input loads); groups of 8 / 16 (several per 32-code
# unit), 64 .. 2048 (rotation across lanes) and 4096 (separate rotation
# kernel); ragged row counts.
SHAPES = [(4096, 4096, 32), (512, 300, 64), (100, 40, 8), (64, 8192, 128), (33, 1024, 16),
          (257, 96, 32), (1000, 2048, 256), (50, 301, 32), (40, 4096, 2048), (30, 4100, 4096),
          (129, 1022, 8)]


@pytest.mark.parametrize("bits", [2, 3, 4, TERNARY])
@pytest.mark.parametrize("n,k,g", SHAPES)
def test_cq_matvec_matches_oracle(hip, n, k, g, bits):
    say("cq matvec", n, k, g, bits)
    m = cq(1, n, k, g, bits)
    x = np.random.default_rng(n + k + g + bits).standard_normal((3, k)).astype(np.float32)
    assert_close(hip.matvec(m, x[0]), ref_matvec(m, x[0]), RTOL, ATOL, f"cq {n}x{k} g{g} b{bits}")
    assert_close(hip.matvec(m, x), ref_matvec(m, x), RTOL, ATOL, f"cq b3 {n}x{k} g{g} b{bits}")


@pytest.mark.parametrize("bits", [2, 3, 4, TERNARY])
@pytest.mark.parametrize("n,k,g", [(40, 300, 64), (9, 40, 8), (17, 8192, 32), (5, 1000, 16)])
def test_cq_row_bit_exact(hip, n, k, g, bits):
    say("cq row", n, k, g, bits)
    m = cq(2, n, k, g, bits)
    for row in sorted({0, n // 2, n - 1}):
        got = hip.row(m, row)
        want = ref_row(m, row)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (row, got[:4], want[:4])


@pytest.mark.parametrize("bits", [2, 3, 4, TERNARY])
def test_reference_fixture_matrices(hip, bits):
    # The matrix(bits) fixture of needle.js tests/cq.test.ts:20-61: two rows,
    # one group of 8 (stored padded to 32 codes), norms 1.25 and 0.75.
    say("reference fixture", bits)
    top = 3 if bits == TERNARY else 1 << bits
    idx = np.arange(16) % top
    codes = np.where(idx == 0, 3, idx - 1) if bits == TERNARY else idx
    norms = np.array([[np.float16(1.25).view(np.uint16)], [np.float16(0.75).view(np.uint16)]],
                     np.uint16)
    m = CqMatrix(pack_codes(codes.reshape(2, 8), bits), norms, BOOKS, 2, 8, 8, bits)
    x = np.sin(np.arange(8) + 0.25).astype(np.float32)
    assert_close(hip.matvec(m, x), ref_matvec(m, x), RTOL, ATOL, f"fixture b{bits}")
    for row in range(2):
        assert np.array_equal(hip.row(m, row), ref_row(m, row))
        # "direct matvec equals a dequantized row dot" (tests/cq.test.ts:88-99)
        assert abs(hip.matvec(m, x)[row] - float(np.dot(hip.row(m, row), x))) < 0.5e-4


def test_cq_ranges_batches_and_mixed_requests(hip):
    say("cq ranges")
    m2 = cq(3, 700, 512, 32, 2)
    m4 = cq(3, 300, 512, 64, 4)
    w, s = synth.int8_matrix(3, "mixed", 256, 512, 32)
    i8 = Int8Matrix(w, s, 32)
    x = np.random.default_rng(5).standard_normal((11, 512)).astype(np.float32)
    # batch 11: one launch (a grid row per batch row); with groups of 4096 the
    # separate rotation kernel runs in chunks of 8 and 3 rows.
    assert_close(hip.matvec(m2, x), ref_matvec(m2, x), RTOL, ATOL, "cq batch 11")
    wide = cq(3, 20, 4096, 4096, 3)
    xw = np.random.default_rng(7).standard_normal((11, 4096)).astype(np.float32)
    assert_close(hip.matvec(wide, xw), ref_matvec(wide, xw), RTOL, ATOL, "cq g4096 batch 11")
    part = hip.matvec(m4, x[:2], MatrixRowRange(37, 200))
    assert_close(part, ref_matvec(m4, x[:2], 37, 200), RTOL, ATOL, "cq range")
    assert hip.matvec(m4, x[0], MatrixRowRange(300, 0)).shape == (0,)
    outs = hip.matvec_batch([
        MatvecRequest(m2, x[0]),
        MatvecRequest(i8, x[0], MatrixRowRange(8, 16)),
        MatvecRequest(m4, x[0], MatrixRowRange(1, 1)),
        MatvecRequest(m2, x[1], MatrixRowRange(699, 1)),
    ])
    assert_close(outs[0], ref_matvec(m2, x[0]), RTOL, ATOL, "batch job 0")
    assert_close(outs[1], oracle.matvec_i8(w, s, 32, x[0], 8, 16), RTOL, ATOL, "batch job 1")
    assert_close(outs[2], ref_matvec(m4, x[0], 1, 1), RTOL, ATOL, "batch job 2")
    assert_close(outs[3], ref_matvec(m2, x[1], 699, 1), RTOL, ATOL, "batch job 3")


def test_cq_device_pointer_entry_points(hip):
    say("cq _d entry points")
    m = cq(4, 1024, 2048, 128, 3)
    h = hip.upload(m)
    x = np.random.default_rng(6).standard_normal((10, 2048)).astype(np.float32)
    dx = DeviceArray(x)
    dy = DeviceArray(np.zeros((10, 1024), np.float32))
    drow = DeviceArray(np.zeros(2048, np.float32))
    try:
        hip._check(hip.lib.nd_matvec_d(hip.ctx, h, dx.ptr, 10, 0, 1024, dy.ptr, None))
        hip._check(hip.lib.nd_row_d(hip.ctx, h, 517, drow.ptr, None))
        hip._check(hip.lib.nd_sync(hip.ctx))
        assert_close(dy.read(), ref_matvec(m, x), RTOL, ATOL, "nd_matvec_d cq")
        assert np.array_equal(drow.read(), ref_row(m, 517))
        bits, kpad, row_bytes = C.c_uint32(), C.c_uint32(), C.c_uint32()
        assert hip.lib.nd_mat_cq_info(h, C.byref(bits), C.byref(kpad), C.byref(row_bytes)) == 0
        assert (bits.value, kpad.value, row_bytes.value) == (3, 2048, 768)
    finally:
        for d in (dx, dy, drow):
            d.free()


def test_cq_archive_round_trip_on_device(hip):
    say("cq archive")
    tensors = [cq(7, 96, 256, 32, b) for b in (2, 3, 4, TERNARY)]
    geometry = dict(vocabulary_size=96, model_dimension=256, number_of_heads=4,
                    number_of_kv_heads=2, head_dimension=64, hadamard_dimension=256)
    archive = parse_cact(write_cact(geometry, CODEBOOK, tensors))
    x = np.random.default_rng(8).standard_normal(256).astype(np.float32)
    for parsed, original in zip(archive.tensors, tensors):
        assert_close(hip.matvec(parsed, x), ref_matvec(original, x), RTOL, ATOL,
                     f"archive b{original.bits}")
        assert np.array_equal(hip.row(parsed, 95), ref_row(original, 95))


def test_cq_rejections(hip):
    say("cq rejections")
    packed, norms = synth.cq_matrix(9, "g4", 4, 64, 8, 2)
    handle = C.c_void_p()
    st = hip.lib.nd_mat_upload_cq(hip.ctx, L.ptr(packed), L.ptr(norms), L.ptr(BOOKS[2]), 4, 64, 4,
                                  2, C.byref(handle))
    assert st == L.ND_ERR_UNSUPPORTED
    st = hip.lib.nd_mat_upload_cq(hip.ctx, L.ptr(packed), L.ptr(norms), L.ptr(BOOKS[2]), 4, 64, 24,
                                  2, C.byref(handle))
    assert st == L.ND_ERR_UNSUPPORTED and b"power-of-two" in hip.lib.nd_last_error(hip.ctx)
    st = hip.lib.nd_mat_upload_cq(hip.ctx, L.ptr(packed), L.ptr(norms), L.ptr(BOOKS[2]), 4, 64, 8,
                                  6, C.byref(handle))
    assert st == L.ND_ERR_UNSUPPORTED
    wide = cq(9, 2, 8200, 8, 2)
    with pytest.raises(NeedleError) as e:
        hip.matvec(wide, np.zeros(8200, np.float32))
    assert e.value.code == "UNSUPPORTED_CACT"
    m = cq(9, 64, 64, 64, 4)
    h = hip.upload(m)
    y = np.zeros((1, 64), np.float32)
    assert hip.lib.nd_matmul(hip.ctx, h, L.ptr(np.zeros((1, 64), np.float32)), 1,
                             L.ptr(y)) == L.ND_ERR_INVALID
    with pytest.raises(NeedleError) as e:
        hip.matvec(m, np.zeros(64, np.float32), MatrixRowRange(60, 5))
    assert e.value.code == "INVALID_CACT"


def test_needle2_archive_matrices_on_device(hip):
    # A synthetic archive in the Needle 2 order: its parsed CQ matrices run
    # on the device as the reference's backends would run them.
    from needle_hip.cact import parse_cact_weights, synthetic_needle2_archive

    say("needle2 archive matrices")
    geo = dict(kv_window=8, kv_bits=8, vocabulary_size=256, model_dimension=128,
               number_of_heads=4, number_of_kv_heads=2, number_of_layers=2, head_dimension=64,
               maximum_sequence_length=64, hadamard_dimension=128, mhc_lanes=4, engram_slots=64,
               engram_sub_dimension=32, number_of_engram_tables=4, engram_convolution_taps=4,
               engram_convolution_dilation=1, engram_orders=[2, 3], engram_layers=[0, 1],
               rope_theta=10000.0)
    for bits in (3, 5):
        w = parse_cact_weights(synthetic_needle2_archive(geo, 9, bits=bits, group=64))
        x = np.random.default_rng(bits).standard_normal(128).astype(np.float32)
        for m in (w.layers[0].query_projection, w.layers[1].key_projection, w.mhc_phi_pre,
                  w.engrams[0].key_projection):
            xx = np.resize(x, m.input_size).astype(np.float32)
            assert_close(hip.matvec(m, xx), ref_matvec(m, xx), RTOL, ATOL, f"archive b{bits}")
        for tok in (0, 255):
            assert np.array_equal(hip.row(w.embedding, tok), ref_row(w.embedding, tok))
