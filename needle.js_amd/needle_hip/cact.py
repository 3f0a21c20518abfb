"""The `.cact` deployment archive and its Cactus-Quant matrices.

Mirrors model/cact.ts of needle.js: the 120-byte header (tag, tensor count,
codebook length, geometry words), the shared fp32 codebook (CQ2 entries
[0, 4), CQ3 [4, 12), CQ4 [12, 28)), the 44-byte tensor directory, and the
tensor kinds (fp16 / fp32 dense, raw bytes, Cactus-Quant matrices).  Packed
matrices stay views of the archive bytes, as the reference keeps them
(cact.ts:183-186); HipBackend uploads a CqMatrix to HBM on first use and
multiplies it there without expanding it.

`parse_cact_weights` continues as parseCact does (cact.ts:398-562): the
tensors in archive order become the named Needle 2 weights (embedding,
layers, mHC, engram sites, final norm, probe heads, tokenizer blob) with
the reference's kind, shape and manifest checks.  `write_cact` builds an
archive from tensors: the inverse of `parse_cact`, for synthetic models and
round-trip tests (there is no writer in the reference; the layout is the
parser's); `synthetic_needle2_archive` writes one in the Needle 2 order.
"""

from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Union

import numpy as np

from .errors import NeedleError, invariant

CACT_TAG = 0x05E12A83  # model/cact.ts:4
CACT_HEADER_BYTES = 120  # cact.ts:5
CACT_RECORD_BYTES = 44  # cact.ts:6
DTYPE_FLOAT16 = 1  # CactDType, cact.ts:8-13
DTYPE_FLOAT32 = 2
DTYPE_CACTUS_QUANT = 3
DTYPE_RAW = 4
TERNARY_RECORD_BITS = 5  # backends/cq.ts:5
CODEBOOK_SLICES = {2: (0, 4), 3: (4, 12), 4: (12, 28)}  # cact.ts:272-276

_DTYPE_NAMES = {1: "FP16", 2: "FP32", 3: "CQ", 4: "RAW"}  # cact.ts:564-568
_GEOMETRY_WORDS = (  # header word index of each field, cact.ts:226-247
    ("kv_window", 3), ("kv_bits", 4), ("vocabulary_size", 5), ("model_dimension", 6),
    ("number_of_heads", 7), ("number_of_kv_heads", 8), ("number_of_layers", 9),
    ("head_dimension", 10), ("maximum_sequence_length", 11), ("hadamard_dimension", 12),
    ("mhc_lanes", 13), ("engram_slots", 14), ("engram_sub_dimension", 15),
    ("number_of_engram_tables", 16), ("engram_convolution_taps", 17),
    ("engram_convolution_dilation", 18),
)


@dataclass(frozen=True)
class CactTensorRecord:
    """One directory entry (CactTensorRecord, cact.ts:37-45)."""

    index: int
    dtype: int
    shape: tuple
    offset: int
    byte_length: int
    group_size: int
    bits: int


@dataclass
class DenseTensor:
    shape: tuple
    data: np.ndarray  # float32
    record: Optional[CactTensorRecord] = None
    kind: str = "dense"


@dataclass
class RawTensor:
    shape: tuple
    data: np.ndarray  # uint8 view of the archive
    record: Optional[CactTensorRecord] = None
    kind: str = "raw"


class CqMatrix:
    """A Cactus-Quant matrix (CqMatrix, cact.ts:61-75).

    packed: uint8 [output_size * row_byte_length], rows of input_size_padded
    codes of `bits` bits (2 bits for the ternary width 5), low bits first,
    3-bit rows one little-endian bit stream; norms: uint16 binary16 patterns
    [output_size][input_size_padded / group_size]; codebooks: {2: 4 floats,
    3: 8 floats, 4: 16 floats} (the archive's shared codebook).
    """

    kind = "cq"

    def __init__(self, packed, norms, codebooks, output_size: int, input_size: int,
                 group_size: int, bits: int, record: Optional[CactTensorRecord] = None):
        invariant(group_size > 0 and (group_size & (group_size - 1)) == 0, "UNSUPPORTED_CACT",
                  f"CQ tensor has non-power-of-two group {group_size}")
        invariant(bits in (2, 3, 4, 5), "UNSUPPORTED_CACT",
                  f"CQ tensor uses unsupported record width {bits}")
        padded = -(-input_size // group_size) * group_size
        packed_bits = 2 if bits == TERNARY_RECORD_BITS else bits
        invariant((padded * packed_bits) % 8 == 0, "INVALID_CACT",
                  "CQ tensor has a fractional packed row size")
        self.output_size = int(output_size)
        self.input_size = int(input_size)
        self.input_size_padded = padded
        self.group_size = int(group_size)
        self.bits = int(bits)
        self.row_byte_length = padded * packed_bits // 8
        self.packed = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8).reshape(-1))
        self.norms = np.ascontiguousarray(np.asarray(norms, dtype=np.uint16).reshape(
            self.output_size, padded // self.group_size))
        invariant(self.packed.size == self.output_size * self.row_byte_length, "INVALID_CACT",
                  "CQ tensor has an inconsistent packed/norm length")
        self.codebooks = {int(b): np.ascontiguousarray(c, dtype=np.float32)
                          for b, c in dict(codebooks).items()}
        if bits != TERNARY_RECORD_BITS:
            cb = self.codebooks.get(bits)
            invariant(cb is not None and cb.size == 1 << bits, "INVALID_CACT",
                      f"Codebook W{bits} is missing")
        self.record = record

    @property
    def shape(self):
        return (self.output_size, self.input_size)

    @property
    def codebook(self) -> Optional[np.ndarray]:
        """This width's codebook (None for ternary)."""
        return None if self.bits == TERNARY_RECORD_BITS else self.codebooks[self.bits]


CactTensor = Union[DenseTensor, RawTensor, CqMatrix]


@dataclass
class CactArchive:
    """Header geometry, the shared codebook and every tensor in directory
    order (the named layer structure of CactWeights is built from these in
    the same order, cact.ts:398-560)."""

    geometry: dict
    codebook: np.ndarray
    tensors: list = field(default_factory=list)


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Packs code rows [n][kpad] into archive bytes [n][kpad * pb / 8]: each
    code low bits first at bit position column * pb of its row (the `pack`
    helper of the reference's tests, cq.test.ts:8-18, row by row).  For the
    ternary width pass the 2-bit crumbs."""
    codes = np.asarray(codes, dtype=np.uint32)
    n, kpad = codes.shape
    pb = 2 if bits == TERNARY_RECORD_BITS else bits
    invariant((kpad * pb) % 8 == 0, "INVALID_CACT", "fractional packed row size")
    invariant(int(codes.max(initial=0)) < (1 << pb), "INVALID_CACT", "code out of range")
    shifts = np.arange(pb, dtype=np.uint32)
    bitplane = ((codes[:, :, None] >> shifts) & 1).astype(np.uint8).reshape(n, kpad * pb)
    return np.packbits(bitplane, axis=1, bitorder="little")


def _product(shape) -> int:
    result = 1
    for value in shape:
        invariant(value >= 0, "INVALID_CACT", f"Invalid tensor dimension {value}")
        result *= int(value)
    return result


def _assert_range(size: int, offset: int, length: int, label: str) -> None:
    invariant(offset >= 0 and length >= 0 and offset + length <= size, "INVALID_CACT",
              f"{label} is outside the archive")


def parse_cact(source) -> CactArchive:
    """parseCact (cact.ts:189-396) up to the tensor list: the header checks,
    the codebook, the directory and each tensor's kind and byte-length
    check, with the same NeedleError codes."""
    data = np.frombuffer(bytes(source) if not isinstance(source, np.ndarray) else source,
                         dtype=np.uint8)
    size = data.size
    _assert_range(size, 0, CACT_HEADER_BYTES, "CACT header")
    words = data[:CACT_HEADER_BYTES].view("<u4")
    tag = int(words[0])
    invariant(tag == CACT_TAG, "INVALID_CACT",
              f"Invalid .cact tag 0x{tag:x} (expected 0x{CACT_TAG:x})")
    number_of_tensors = int(words[1])
    codebook_length = int(words[2])
    invariant(number_of_tensors > 0, "INVALID_CACT", "The .cact archive has no tensors")
    invariant(codebook_length >= 28, "UNSUPPORTED_CACT",
              f"Needle 2 requires the CQ2/CQ3/CQ4 codebook (28 entries); archive has "
              f"{codebook_length}")
    number_of_orders = int(words[19])
    number_of_sites = int(words[24])
    invariant(number_of_orders <= 4 and number_of_sites <= 4, "UNSUPPORTED_CACT",
              "The current .cact format supports at most four engram orders and sites")
    geometry = {name: int(words[i]) for name, i in _GEOMETRY_WORDS}
    geometry["engram_orders"] = [int(words[20 + i]) for i in range(number_of_orders)]
    geometry["engram_layers"] = [int(words[25 + i]) for i in range(number_of_sites)]
    geometry["rope_theta"] = float(data[116:120].view("<f4")[0])
    invariant(geometry["model_dimension"] > 0 and geometry["vocabulary_size"] > 0,
              "INVALID_CACT", "Model geometry contains a zero-sized vocabulary or hidden dimension")
    heads, kv_heads = geometry["number_of_heads"], geometry["number_of_kv_heads"]
    invariant(heads > 0 and kv_heads > 0 and heads % kv_heads == 0, "UNSUPPORTED_CACT",
              "Attention heads must be a positive multiple of KV heads")
    invariant(heads * geometry["head_dimension"] > 0, "INVALID_CACT",
              "Invalid attention dimensions")
    hd = geometry["hadamard_dimension"]
    invariant(hd & (hd - 1) == 0, "UNSUPPORTED_CACT", "Hadamard dimension must be a power of two")

    codebook_offset = CACT_HEADER_BYTES
    _assert_range(size, codebook_offset, codebook_length * 4, "CQ codebook")
    codebook = data[codebook_offset:codebook_offset + codebook_length * 4].view("<f4").astype(
        np.float32)
    codebooks = {b: codebook[lo:hi].copy() for b, (lo, hi) in CODEBOOK_SLICES.items()}

    directory = codebook_offset + codebook_length * 4
    _assert_range(size, directory, number_of_tensors * CACT_RECORD_BYTES, "Tensor directory")
    tensors: list = []
    for index in range(number_of_tensors):
        at = directory + index * CACT_RECORD_BYTES
        raw = data[at:at + CACT_RECORD_BYTES].tobytes()
        dtype, dims = raw[0], raw[1]
        invariant(dims <= 4, "UNSUPPORTED_CACT",
                  f"Tensor {index} has {dims} dimensions; the format supports four")
        shape = struct.unpack_from("<4I", raw, 4)[:dims]
        offset, byte_length = struct.unpack_from("<QQ", raw, 20)
        group_size, bits = struct.unpack_from("<II", raw, 36)
        _assert_range(size, offset, byte_length, f"Tensor {index}")
        record = CactTensorRecord(index, dtype, tuple(shape), offset, byte_length, group_size,
                                  bits)
        blob = data[offset:offset + byte_length]
        count = _product(shape)
        if dtype == DTYPE_FLOAT16:
            invariant(byte_length == count * 2, "INVALID_CACT",
                      f"FP16 tensor {index} has an inconsistent byte length")
            tensors.append(DenseTensor(tuple(shape), blob.view("<f2").astype(np.float32), record))
        elif dtype == DTYPE_FLOAT32:
            invariant(byte_length == count * 4, "INVALID_CACT",
                      f"FP32 tensor {index} has an inconsistent byte length")
            tensors.append(DenseTensor(tuple(shape), blob.view("<f4").astype(np.float32), record))
        elif dtype == DTYPE_RAW:
            tensors.append(RawTensor(tuple(shape), blob, record))
        elif dtype == DTYPE_CACTUS_QUANT:
            invariant(len(shape) == 2, "INVALID_CACT", f"CQ tensor {index} is not a matrix")
            invariant(group_size > 0 and (group_size & (group_size - 1)) == 0,
                      "UNSUPPORTED_CACT",
                      f"CQ tensor {index} has non-power-of-two group {group_size}")
            invariant(bits in (2, 3, 4, 5), "UNSUPPORTED_CACT",
                      f"CQ tensor {index} uses unsupported record width {bits}")
            n, k = shape
            padded = -(-k // group_size) * group_size
            pb = 2 if bits == TERNARY_RECORD_BITS else bits
            invariant((padded * pb) % 8 == 0, "INVALID_CACT",
                      f"CQ tensor {index} has a fractional packed row size")
            packed_length = n * padded * pb // 8
            norm_count = n * (padded // group_size)
            invariant(byte_length == packed_length + norm_count * 2, "INVALID_CACT",
                      f"CQ tensor {index} has an inconsistent packed/norm length")
            tensors.append(CqMatrix(blob[:packed_length], blob[packed_length:].view("<u2"),
                                    codebooks, n, k, group_size, bits, record))
        else:
            raise NeedleError("UNSUPPORTED_CACT",
                              f"Tensor {index} uses unknown dtype "
                              f"{_DTYPE_NAMES.get(dtype, str(dtype))}")
    return CactArchive(geometry, codebook, tensors)


def write_cact(geometry: dict, codebook: np.ndarray, tensors: Sequence[CactTensor]) -> bytes:
    """Serializes tensors into a `.cact` archive that `parse_cact` (and the
    reference's parseCact) reads back: header, codebook, directory, then
    each blob 64-byte aligned."""
    codebook = np.ascontiguousarray(codebook, dtype="<f4")
    header = np.zeros(CACT_HEADER_BYTES // 4, dtype="<u4")
    header[0] = CACT_TAG
    header[1] = len(tensors)
    header[2] = codebook.size
    for name, i in _GEOMETRY_WORDS:
        header[i] = int(geometry.get(name, 0))
    orders = list(geometry.get("engram_orders", []))
    sites = list(geometry.get("engram_layers", []))
    header[19] = len(orders)
    header[20:20 + len(orders)] = orders
    header[24] = len(sites)
    header[25:25 + len(sites)] = sites
    header_bytes = bytearray(header.tobytes())
    header_bytes[116:120] = struct.pack("<f", float(geometry.get("rope_theta", 0.0)))

    blobs = []
    for t in tensors:
        if isinstance(t, CqMatrix):
            blobs.append((DTYPE_CACTUS_QUANT, t.shape, t.group_size, t.bits,
                          t.packed.tobytes() + t.norms.astype("<u2").tobytes()))
        elif isinstance(t, RawTensor):
            blobs.append((DTYPE_RAW, tuple(t.shape), 0, 0, np.asarray(t.data, np.uint8).tobytes()))
        else:
            arr = np.asarray(t.data, dtype=np.float32)
            dt = t.record.dtype if t.record is not None else DTYPE_FLOAT32
            payload = arr.astype("<f2" if dt == DTYPE_FLOAT16 else "<f4").tobytes()
            blobs.append((dt, tuple(t.shape), 0, 0, payload))

    directory = CACT_HEADER_BYTES + codebook.size * 4
    cursor = directory + CACT_RECORD_BYTES * len(blobs)
    records = bytearray()
    body = bytearray()
    for dtype, shape, group, bits, payload in blobs:
        cursor = (cursor + 63) // 64 * 64
        start = cursor
        rec = bytearray(CACT_RECORD_BYTES)
        rec[0] = dtype
        rec[1] = len(shape)
        struct.pack_into("<4I", rec, 4, *(list(shape) + [0] * (4 - len(shape))))
        struct.pack_into("<QQII", rec, 20, start, len(payload), group, bits)
        records += rec
        body += bytes(start - (directory + CACT_RECORD_BYTES * len(blobs)) - len(body))
        body += payload
        cursor = start + len(payload)
    return bytes(header_bytes) + codebook.tobytes() + bytes(records) + bytes(body)


# ------------------------------------------------------ named Needle 2 weights

@dataclass
class CactLayer:
    norm_input: np.ndarray
    query_projection: CqMatrix
    key_projection: CqMatrix
    value_projection: CqMatrix
    query_norm: np.ndarray
    key_norm: np.ndarray
    gate_projection: CqMatrix
    output_projection: CqMatrix
    post_attention_norm: np.ndarray
    attention_gate: float
    pre_hadamard_norm: np.ndarray
    hadamard_d1: np.ndarray
    hadamard_d2: np.ndarray
    hadamard_d3: np.ndarray


@dataclass
class CactEngramSite:
    tables: CqMatrix
    key_projection: CqMatrix
    value_projection: CqMatrix
    taps: np.ndarray


@dataclass
class CactProbeHead:
    """CactProbeHead (cact.ts:105-112)."""

    name: str
    probes: np.ndarray
    probe_count: int
    projection: np.ndarray
    output_size: int
    bias: np.ndarray


@dataclass
class CactWeights:
    """CactWeights (cact.ts:114-138)."""

    geometry: dict
    codebook: np.ndarray
    tensors: list
    embedding: CqMatrix
    layers: List[CactLayer]
    mhc_a_pre: np.ndarray
    mhc_a_post: np.ndarray
    mhc_a_residual: np.ndarray
    mhc_b_pre: np.ndarray
    mhc_b_post: np.ndarray
    mhc_b_residual: np.ndarray
    mhc_phi_pre: CqMatrix
    mhc_phi_post: CqMatrix
    mhc_phi_residual: CqMatrix
    engrams: List[CactEngramSite]
    final_norm: np.ndarray
    heads: dict
    tokenizer_blob: np.ndarray


def parse_cact_weights(source) -> CactWeights:
    """parseCact to the end (cact.ts:398-562)."""
    archive = parse_cact(source)
    geometry, tensors = archive.geometry, archive.tensors
    cursor = 0

    def take(name):
        nonlocal cursor
        invariant(cursor < len(tensors), "INVALID_CACT", f"Archive ended before {name}")
        t = tensors[cursor]
        cursor += 1
        return t

    def cq(t, name) -> CqMatrix:
        invariant(t.kind == "cq", "INVALID_CACT", f"{name} must be a Cactus-Quant matrix")
        return t

    def dense(t, name) -> np.ndarray:
        invariant(t.kind == "dense", "INVALID_CACT", f"{name} must be a dense tensor")
        return t.data

    embedding = cq(take("embedding"), "embedding")
    invariant(embedding.output_size == geometry["vocabulary_size"]
              and embedding.input_size == geometry["model_dimension"], "INVALID_CACT",
              "Embedding shape does not match model geometry")
    layers = []
    for layer in range(geometry["number_of_layers"]):
        pre = f"layer {layer}"
        norm_input = dense(take(f"{pre} input norm"), f"{pre} input norm")
        q = cq(take(f"{pre} query projection"), f"{pre} query projection")
        k = cq(take(f"{pre} key projection"), f"{pre} key projection")
        v = cq(take(f"{pre} value projection"), f"{pre} value projection")
        qn = dense(take(f"{pre} query norm"), f"{pre} query norm")
        kn = dense(take(f"{pre} key norm"), f"{pre} key norm")
        gate = cq(take(f"{pre} gate projection"), f"{pre} gate projection")
        out = cq(take(f"{pre} output projection"), f"{pre} output projection")
        post = dense(take(f"{pre} post-attention norm"), f"{pre} post-attention norm")
        ag = dense(take(f"{pre} attention gate"), f"{pre} attention gate")
        preh = dense(take(f"{pre} pre-Hadamard norm"), f"{pre} pre-Hadamard norm")
        d1 = dense(take(f"{pre} Hadamard d1"), f"{pre} Hadamard d1")
        d2 = dense(take(f"{pre} Hadamard d2"), f"{pre} Hadamard d2")
        d3 = dense(take(f"{pre} Hadamard d3"), f"{pre} Hadamard d3")
        layers.append(CactLayer(norm_input, q, k, v, qn, kn, gate, out, post,
                                float(ag[0]) if ag.size else 0.0, preh, d1, d2, d3))
    mhc = [dense(take(f"mHC {n}"), f"mHC {n}")
           for n in ("a_pre", "a_post", "a_res", "b_pre", "b_post", "b_res")]
    phi = [cq(take(f"mHC {n}"), f"mHC {n}") for n in ("phi_pre", "phi_post", "phi_res")]
    engrams = []
    for site in range(len(geometry["engram_layers"])):
        engrams.append(CactEngramSite(
            cq(take(f"engram {site} tables"), f"engram {site} tables"),
            cq(take(f"engram {site} key projection"), f"engram {site} key projection"),
            cq(take(f"engram {site} value projection"), f"engram {site} value projection"),
            dense(take(f"engram {site} taps"), f"engram {site} taps")))
    final_norm = dense(take("final norm"), "final norm")
    heads = {}
    if cursor < len(tensors) and tensors[cursor].kind == "dense":
        manifest = tensors[cursor].data
        cursor += 1
        for raw in manifest:
            code = math.floor(float(raw) + 0.5)  # Math.round
            name = "contrastive" if code == 1 else "confidence" if code == 2 else None
            invariant(name is not None, "UNSUPPORTED_CACT", f"Unknown probe-head manifest code {code}")
            pt, jt, bt = take(f"{name} probes"), take(f"{name} projection"), take(f"{name} bias")
            probes, proj, bias = (dense(pt, f"{name} probes"), dense(jt, f"{name} projection"),
                                  dense(bt, f"{name} bias"))
            count = pt.shape[0] if pt.shape else 0
            out = jt.shape[0] if jt.shape else bias.size
            d = geometry["model_dimension"]
            invariant(count > 0 and probes.size == count * d, "INVALID_CACT",
                      f"{name} probe shape is inconsistent")
            invariant(proj.size == out * count * d, "INVALID_CACT",
                      f"{name} projection shape is inconsistent")
            heads[name] = CactProbeHead(name, probes.reshape(count, d), count,
                                        proj.reshape(out, count * d), out, bias)
    blob = None
    while cursor < len(tensors):
        t = take("trailing tensor")
        if t.kind == "raw":
            invariant(blob is None, "INVALID_CACT", "Archive contains more than one RAW tokenizer tensor")
            blob = t.data
        else:
            raise NeedleError("UNSUPPORTED_CACT", f"Unexpected trailing tensor {t.record.index}")
    invariant(blob is not None, "INVALID_CACT", "Archive does not contain its RAW SentencePiece tokenizer")
    return CactWeights(geometry, archive.codebook, tensors, embedding, layers, *mhc, *phi, engrams,
                       final_norm, heads, blob)


_MIXED_WIDTHS = (4, 3, 2, 5)


def mixed_form(role: str, index: int = 0) -> tuple:
    """(bits, group) of one matrix of the mixed-width Needle 2 used in tests
    and the benchmark: the shipped archive is "mixed CQ2/CQ3/CQ4/ternary"
    (packages/needle.js/README.md:21) with every record carrying its own
    width and group (cact.ts:346-361).  Across layers every width (ternary
    as 5) meets every kind of matrix; a layer's q, k, v and gate share their
    group and Wo has groups of 128, as the reference's resident path expects
    of the archive (resident/compatibility.ts:19-36).  `index` is the layer
    (the engram site for the engram matrices)."""
    w = _MIXED_WIDTHS
    part = {"wq": 0, "wk": 1, "wv": 2, "wgate": 3}
    if role in part:
        return w[(index + part[role]) % 4], (32, 64)[index % 2]
    return {
        "embedding": (4, 32),
        "wo": (w[(index + 2) % 4], 128),
        "phi_pre": (2, 64),
        "phi_post": (5, 32),
        "phi_res": (3, 128),
        "eg_tables": ((3, 64), (5, 64))[index % 2],
        "eg_key": (2, 32),
        "eg_value": (4, 64),
    }[role]


def synthetic_needle2_archive(geometry: dict, run_seed: int = 2026, bits: int = 4,
                              group: int = 32, confidence: bool = True,
                              mixed: bool = False) -> bytes:
    """A .cact archive in the Needle 2 tensor order (cact.ts:410-540) with
    seeded Cactus-Quant matrices of one width and group (mixed: each matrix
    in its mixed_form), dense vectors near neutral, an optional confidence
    head and a placeholder tokenizer blob."""
    from . import synth

    g = geometry
    d, hd, L = g["model_dimension"], g["head_dimension"], g["number_of_layers"]
    H, Hkv, ln = g["number_of_heads"], g["number_of_kv_heads"], g["mhc_lanes"]
    codebook = synth.cq_codebook()
    books = {b: codebook[lo:hi] for b, (lo, hi) in CODEBOOK_SLICES.items()}
    tensors: list = []
    count = [0]

    def cqm(n, k, role="", index=0):
        count[0] += 1
        b, gr = mixed_form(role, index) if mixed else (bits, group)
        packed, norms = synth.cq_matrix(run_seed, f"arch{count[0]}", n, k, gr, b)
        tensors.append(CqMatrix(packed, norms, books, n, k, gr, b))

    def vec(shape, lo, hi):
        count[0] += 1
        data = synth.Stream(run_seed, f"arch{count[0]}").uniform(shape, lo, hi).reshape(-1)
        tensors.append(DenseTensor(tuple(shape), data.astype(np.float32)))

    cqm(g["vocabulary_size"], d, "embedding")
    for layer in range(L):
        vec((d,), -0.1, 0.1)
        cqm(H * hd, d, "wq", layer)
        cqm(Hkv * hd, d, "wk", layer)
        cqm(Hkv * hd, d, "wv", layer)
        vec((hd,), -0.1, 0.1)
        vec((hd,), -0.1, 0.1)
        cqm(H * hd, d, "wgate", layer)
        cqm(d, H * hd, "wo", layer)
        vec((d,), -0.1, 0.1)
        vec((1,), -1.0, 1.0)
        vec((d,), -0.1, 0.1)
        vec((d,), 0.5, 1.5)
        vec((g["hadamard_dimension"],), 0.5, 1.5)
        vec((d,), 0.5, 1.5)
    for shape in ((L,), (L,), (L,), (L * ln,), (L * ln,), (L * ln * ln,)):
        vec(shape, 0.02, 0.1)
    cqm(L * ln, ln * d, "phi_pre")
    cqm(L * ln, ln * d, "phi_post")
    cqm(L * ln * ln, ln * d, "phi_res")
    cat = g["number_of_engram_tables"] * g["engram_sub_dimension"]
    for site, _ in enumerate(g.get("engram_layers", [])):
        cqm(g["number_of_engram_tables"] * g["engram_slots"], g["engram_sub_dimension"],
            "eg_tables", site)
        cqm(d, cat, "eg_key", site)
        cqm(d, cat, "eg_value", site)
        vec((g["engram_convolution_taps"], d), -0.5, 0.5)
    vec((d,), -0.1, 0.1)
    if confidence:
        tensors.append(DenseTensor((1,), np.array([2.0], np.float32)))
        vec((8, d), -0.1, 0.1)
        vec((1, 8 * d), -0.003, 0.003)
        vec((1,), -0.2, 0.2)
    tensors.append(RawTensor((16,), np.frombuffer(b"synthetic-sp-mdl", np.uint8)))
    return write_cact(geometry, codebook, tensors)
