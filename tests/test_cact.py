""".cact archive parsing and writing (host logic, CPU only).

The first three cases are the reference's parser tests (tests/cact.test.ts:
5-21); the rest check that every tensor kind survives write -> parse, that
the parser's length and kind checks raise the reference's codes, and that
a Needle 2 archive parses into its named weights (cact.ts:398-562) with the
reference's structure checks.
"""

import struct

import numpy as np
import pytest

from needle_hip import CqMatrix, NeedleError, parse_cact, synth, write_cact
from needle_hip import cact as K
from needle_hip.cact import parse_cact_weights, synthetic_needle2_archive

import oracle


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


# ------------------------------------------------------ named Needle 2 weights

N2_GEOMETRY = dict(kv_window=8, kv_bits=8, vocabulary_size=256, model_dimension=128,
                   number_of_heads=4, number_of_kv_heads=2, number_of_layers=2, head_dimension=64,
                   maximum_sequence_length=64, hadamard_dimension=128, mhc_lanes=4,
                   engram_slots=64, engram_sub_dimension=32, number_of_engram_tables=4,
                   engram_convolution_taps=4, engram_convolution_dilation=1,
                   engram_orders=[2, 3], engram_layers=[0, 1], rope_theta=10000.0)


def test_archive_weights_for_the_runtime_step_on_the_oracle():
    """weights_from_cact maps a parsed archive onto the runtime's weight
    layout: the oracle steps it, and its float64 model (dequantized CQ
    matrices) agrees."""
    from needle_hip.needle2 import weights_from_cact
    from test_oracle_needle2 import NumpyNeedle2

    w = weights_from_cact(parse_cact_weights(synthetic_needle2_archive(N2_GEOMETRY, 3)))
    g = w.geometry
    assert (g.vocab, g.dim, g.layers, g.sites, g.orders) == (256, 128, 2, (0, 1), (2, 3))
    assert w.norm_input.shape == (2, 128) and w.d2.shape == (2, 128) and len(w.eg_tables) == 2
    assert w.confidence is not None and w.confidence.probe_count == 8
    rt = oracle.Needle2(w).runtime(g.max_length, 0)
    ref = NumpyNeedle2(w, g.max_length, 0)
    for t in (5, 200, 17, 5, 200, 64):
        got, want = rt.step(t), ref.step(t)
        assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max(), t


def test_mixed_width_archive_records_and_oracle_step():
    """A mixed-width archive: every Cactus-Quant record keeps the width and
    group mixed_form gives it through write and parse, every width appears,
    and the oracle's step over the parsed weights agrees with the float64
    model of the dequantized matrices."""
    from needle_hip.cact import mixed_form
    from needle_hip.needle2 import weights_from_cact
    from test_oracle_needle2 import NumpyNeedle2

    pw = parse_cact_weights(synthetic_needle2_archive(N2_GEOMETRY, 6, mixed=True))
    seen = set()
    for l, layer in enumerate(pw.layers):
        for role, m in (("wq", layer.query_projection), ("wk", layer.key_projection),
                        ("wv", layer.value_projection), ("wgate", layer.gate_projection),
                        ("wo", layer.output_projection)):
            assert (m.bits, m.group_size) == mixed_form(role, l), (role, l)
            seen.add(m.bits)
    for role, m in (("embedding", pw.embedding), ("phi_pre", pw.mhc_phi_pre),
                    ("phi_post", pw.mhc_phi_post), ("phi_res", pw.mhc_phi_residual)):
        assert (m.bits, m.group_size) == mixed_form(role), role
    for s, e in enumerate(pw.engrams):
        assert (e.tables.bits, e.tables.group_size) == mixed_form("eg_tables", s)
        assert (e.key_projection.bits, e.key_projection.group_size) == mixed_form("eg_key", s)
        assert (e.value_projection.bits, e.value_projection.group_size) == mixed_form("eg_value", s)
    assert seen == {2, 3, 4, 5}
    w = weights_from_cact(pw)
    rt = oracle.Needle2(w).runtime(w.geometry.max_length, 0)
    ref = NumpyNeedle2(w, w.geometry.max_length, 0)
    for t in (5, 200, 17, 5, 200, 64):
        got, want = rt.step(t), ref.step(t)
        assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max(), t


def test_needle2_archive_named_structure():
    w = parse_cact_weights(synthetic_needle2_archive(N2_GEOMETRY, 3))
    g = N2_GEOMETRY
    assert w.embedding.shape == (256, 128) and len(w.layers) == 2
    layer = w.layers[1]
    assert layer.query_projection.shape == (256, 128)
    assert layer.key_projection.shape == (128, 128)
    assert layer.output_projection.shape == (128, 256)
    assert layer.query_norm.shape == (64,) and layer.hadamard_d2.shape == (128,)
    assert isinstance(layer.attention_gate, float)
    assert w.mhc_phi_residual.shape == (2 * 16, 4 * 128) and w.mhc_b_residual.shape == (32,)
    assert len(w.engrams) == 2 and w.engrams[0].tables.shape == (4 * 64, 32)
    assert w.engrams[1].taps.size == 4 * 128
    head = w.heads["confidence"]
    assert (head.probe_count, head.output_size) == (8, 1) and head.projection.shape == (1, 1024)
    assert w.tokenizer_blob.tobytes() == b"synthetic-sp-mdl"
    assert w.geometry["engram_layers"] == g["engram_layers"]


def _rewrite(tensors_edit):
    archive = K.parse_cact(synthetic_needle2_archive(N2_GEOMETRY, 4))
    tensors = list(archive.tensors)
    tensors_edit(tensors)
    return write_cact(archive.geometry, archive.codebook, tensors)


@pytest.mark.parametrize("edit,code,pattern", [
    (lambda t: t.pop(), "INVALID_CACT", "tokenizer"),
    (lambda t: t.append(K.RawTensor((1,), np.zeros(1, np.uint8))), "INVALID_CACT",
     "more than one RAW"),
    (lambda t: t.insert(len(t) - 1, K.DenseTensor((1,), np.ones(1, np.float32))),
     "UNSUPPORTED_CACT", "Unexpected trailing tensor"),
    (lambda t: t.__setitem__(0, t[1]), "INVALID_CACT", "embedding must be a Cactus-Quant"),
    (lambda t: t.__setitem__(-5, K.DenseTensor((1,), np.array([3.0], np.float32))),
     "UNSUPPORTED_CACT", "probe-head manifest code 3"),
])
def test_needle2_archive_checks(edit, code, pattern):
    with pytest.raises(NeedleError, match=pattern) as e:
        parse_cact_weights(_rewrite(edit))
    assert e.value.code == code


def test_needle2_archive_embedding_shape_checked():
    g = dict(N2_GEOMETRY, vocabulary_size=300)
    data = bytearray(synthetic_needle2_archive(N2_GEOMETRY, 5))
    struct.pack_into("<I", data, 5 * 4, g["vocabulary_size"])
    with pytest.raises(NeedleError, match="Embedding shape"):
        parse_cact_weights(bytes(data))
