""".cact archive parsing and writing (host logic, CPU only).

The first three cases are the reference's parser tests (tests/cact.test.ts:
5-21); the rest check that every tensor kind survives write -> parse and
that the parser's length and kind checks raise the reference's codes.
"""

import struct

import numpy as np
import pytest

from needle_hip import CqMatrix, NeedleError, parse_cact, synth, write_cact
from needle_hip import cact as K


def test_rejects_truncated_header():
    with pytest.raises(NeedleError, match="(?i)header") as e:
        parse_cact(bytes(12))
    assert e.value.code == "INVALID_CACT"


def test_rejects_bad_magic():
    with pytest.raises(NeedleError, match="(?i)tag"):
        parse_cact(bytes(120))


def test_validates_codebook_before_directory():
    head = bytearray(120)
    struct.pack_into("<III", head, 0, K.CACT_TAG, 1, 4)
    with pytest.raises(NeedleError, match="(?i)codebook") as e:
        parse_cact(bytes(head))
    assert e.value.code == "UNSUPPORTED_CACT"


GEOMETRY = dict(kv_window=256, kv_bits=8, vocabulary_size=64, model_dimension=32,
                number_of_heads=2, number_of_kv_heads=1, number_of_layers=1, head_dimension=16,
                maximum_sequence_length=512, hadamard_dimension=32, mhc_lanes=2,
                engram_slots=4, engram_sub_dimension=8, number_of_engram_tables=2,
                engram_convolution_taps=3, engram_convolution_dilation=1,
                engram_orders=[2, 3], engram_layers=[0], rope_theta=10000.0)


def sample_tensors():
    codebook = synth.cq_codebook()
    books = {b: codebook[lo:hi] for b, (lo, hi) in K.CODEBOOK_SLICES.items()}
    tensors = []
    for i, (n, k, g, bits) in enumerate([(16, 64, 32, 2), (8, 40, 8, 3), (4, 256, 128, 4),
                                         (6, 96, 32, 5)]):
        packed, norms = synth.cq_matrix(3, f"t{i}", n, k, g, bits)
        tensors.append(CqMatrix(packed, norms, books, n, k, g, bits))
    f16 = K.CactTensorRecord(0, K.DTYPE_FLOAT16, (3, 5), 0, 0, 0, 0)
    tensors.append(K.DenseTensor((3, 5), np.linspace(-2, 2, 15).astype(np.float16)
                                 .astype(np.float32), f16))
    tensors.append(K.DenseTensor((7,), np.arange(7, dtype=np.float32) / 3))
    tensors.append(K.RawTensor((9,), np.arange(9, dtype=np.uint8)))
    return codebook, tensors


def test_write_parse_round_trip():
    codebook, tensors = sample_tensors()
    archive = parse_cact(write_cact(GEOMETRY, codebook, tensors))
    assert archive.geometry == GEOMETRY
    assert np.array_equal(archive.codebook, codebook)
    assert len(archive.tensors) == len(tensors)
    for index, (got, want) in enumerate(zip(archive.tensors, tensors)):
        assert got.kind == want.kind and tuple(got.shape) == tuple(want.shape)
        assert got.record.index == index
        if want.kind == "cq":
            assert (got.group_size, got.bits, got.input_size_padded, got.row_byte_length) == (
                want.group_size, want.bits, want.input_size_padded, want.row_byte_length)
            assert np.array_equal(got.packed, want.packed)
            assert np.array_equal(got.norms, want.norms)
            if want.bits != 5:
                assert np.array_equal(got.codebook, want.codebook)
        else:
            assert np.array_equal(got.data, want.data)
    assert archive.tensors[4].record.dtype == K.DTYPE_FLOAT16


def test_cq_geometry_matches_the_parser_rules():
    codebook, tensors = sample_tensors()
    m = tensors[1]  # 8 x 40, group 8, 3-bit
    assert (m.input_size_padded, m.row_byte_length) == (40, 15)
    t = tensors[3]  # ternary: 2-bit crumbs
    assert t.row_byte_length == 96 * 2 // 8 and t.codebook is None


def test_rejects_inconsistent_cq_length():
    codebook, tensors = sample_tensors()
    blob = bytearray(write_cact(GEOMETRY, codebook, tensors[:1]))
    directory = K.CACT_HEADER_BYTES + codebook.size * 4
    length = struct.unpack_from("<Q", blob, directory + 28)[0]
    struct.pack_into("<Q", blob, directory + 28, length - 2)
    with pytest.raises(NeedleError, match="inconsistent packed/norm length"):
        parse_cact(bytes(blob))


@pytest.mark.parametrize("field,value,code,pattern", [
    (36, 24, "UNSUPPORTED_CACT", "non-power-of-two group"),
    (40, 6, "UNSUPPORTED_CACT", "unsupported record width"),
    (0, 9, "UNSUPPORTED_CACT", "unknown dtype"),
])
def test_rejects_unsupported_records(field, value, code, pattern):
    codebook, tensors = sample_tensors()
    blob = bytearray(write_cact(GEOMETRY, codebook, tensors[:1]))
    directory = K.CACT_HEADER_BYTES + codebook.size * 4
    if field == 0:
        blob[directory] = value
    else:
        struct.pack_into("<I", blob, directory + field, value)
    with pytest.raises(NeedleError, match=pattern) as e:
        parse_cact(bytes(blob))
    assert e.value.code == code


def test_rejects_out_of_range_blob_and_heads():
    codebook, tensors = sample_tensors()
    blob = bytearray(write_cact(GEOMETRY, codebook, tensors[:1]))
    with pytest.raises(NeedleError, match="outside the archive"):
        parse_cact(bytes(blob[:-1]))
    bad = dict(GEOMETRY, number_of_heads=3, number_of_kv_heads=2)
    with pytest.raises(NeedleError, match="positive multiple of KV heads"):
        parse_cact(write_cact(bad, codebook, tensors[:1]))
