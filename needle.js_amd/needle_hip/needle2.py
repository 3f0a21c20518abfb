"""Needle 2 geometry and seeded int8 weights.

The shipped geometry (apps/website/src/content/docs/tutorials/model-structure.mdx:12-23;
packages/needle.js/tests/model.integration.test.ts:175-180): vocab 8192,
d 512, 27 layers, 8 query heads and 4 KV heads of 64, 4 mHC lanes, Hadamard
512, KV window 256, maximum sequence 2048, engram orders {2, 3} at layers
{2, 15} with 4 tables x 8192 slots x 128 and 4 taps.  The archive's RoPE
theta is not documented; 10000 is used.  Every Cactus-Quant matrix becomes an
int8 matrix with one fp32 scale per row (uniform codes in [-127, 127],
scales ~U(0.001, 0.02)); dense vectors are seeded near neutral (norm offsets
~U(-0.1, 0.1), Hadamard diagonals ~U(0.5, 1.5)).  The confidence probe head
has the shape the resident reference path accepts (resident/compatibility.ts:42-51):
8 probes of d, one output.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import synth
from .backend import Int8Matrix


@dataclass(frozen=True)
class Needle2Geometry:
    vocab: int = 8192
    dim: int = 512
    heads: int = 8
    kv_heads: int = 4
    layers: int = 27
    head_dim: int = 64
    max_length: int = 2048
    hadamard: int = 512
    lanes: int = 4
    engram_slots: int = 8192
    engram_sub: int = 128
    engram_tables: int = 4
    engram_taps: int = 4
    orders: tuple = (2, 3)
    sites: tuple = (2, 15)
    rope_theta: float = 10000.0
    kv_window: int = 256


class ProbeHead:
    """CactProbeHead (model/cact.ts:105-112): probes [count][dim],
    projection [output_size][count * dim], bias [output_size]."""

    def __init__(self, probes: np.ndarray, projection: np.ndarray, bias: np.ndarray):
        self.probes = np.ascontiguousarray(probes, dtype=np.float32)
        self.projection = np.ascontiguousarray(projection, dtype=np.float32)
        self.bias = np.ascontiguousarray(bias, dtype=np.float32)
        self.probe_count, dim = self.probes.shape
        self.output_size = self.bias.shape[0]
        assert self.projection.shape == (self.output_size, self.probe_count * dim)


def weights_from_cact(w) -> "Needle2Weights":
    """The runtime's weights from a parsed .cact archive (CactWeights,
    cact.ts:114-138, from parse_cact_weights): the archive's Cactus-Quant
    matrices as they are, the per-layer dense tensors stacked, the geometry
    from the header (cact.ts:398-562, runtime.ts:150-225)."""
    h = w.geometry
    g = Needle2Geometry(
        vocab=h["vocabulary_size"], dim=h["model_dimension"], heads=h["number_of_heads"],
        kv_heads=h["number_of_kv_heads"], layers=h["number_of_layers"],
        head_dim=h["head_dimension"], max_length=h["maximum_sequence_length"],
        hadamard=h["hadamard_dimension"], lanes=h["mhc_lanes"], engram_slots=h["engram_slots"],
        engram_sub=h["engram_sub_dimension"], engram_tables=h["number_of_engram_tables"],
        engram_taps=h["engram_convolution_taps"], orders=tuple(h["engram_orders"]),
        sites=tuple(h["engram_layers"]), rope_theta=float(h["rope_theta"]),
        kv_window=h["kv_window"])
    out = Needle2Weights.__new__(Needle2Weights)
    out.geometry = g
    out.embedding = w.embedding
    layers = w.layers
    out.wq = [l.query_projection for l in layers]
    out.wk = [l.key_projection for l in layers]
    out.wv = [l.value_projection for l in layers]
    out.wgate = [l.gate_projection for l in layers]
    out.wo = [l.output_projection for l in layers]

    def stack(name):
        return np.stack([np.asarray(getattr(l, name), np.float32).reshape(-1) for l in layers])

    out.norm_input = stack("norm_input")
    out.query_norm = stack("query_norm")
    out.key_norm = stack("key_norm")
    out.post_attn_norm = stack("post_attention_norm")
    out.attention_gate = np.array([l.attention_gate for l in layers], np.float32)
    out.pre_hadamard_norm = stack("pre_hadamard_norm")
    out.d1, out.d2, out.d3 = stack("hadamard_d1"), stack("hadamard_d2"), stack("hadamard_d3")
    out.phi_pre, out.phi_post, out.phi_res = w.mhc_phi_pre, w.mhc_phi_post, w.mhc_phi_residual
    f32 = lambda v: np.asarray(v, np.float32).reshape(-1)  # noqa: E731
    out.a_pre, out.a_post, out.a_res = f32(w.mhc_a_pre), f32(w.mhc_a_post), f32(w.mhc_a_residual)
    out.b_pre, out.b_post, out.b_res = f32(w.mhc_b_pre), f32(w.mhc_b_post), f32(w.mhc_b_residual)
    out.eg_tables = [e.tables for e in w.engrams]
    out.eg_key = [e.key_projection for e in w.engrams]
    out.eg_value = [e.value_projection for e in w.engrams]
    out.eg_taps = (np.stack([np.asarray(e.taps, np.float32).reshape(g.engram_taps, g.dim)
                             for e in w.engrams]) if w.engrams
                   else np.zeros((0, g.engram_taps, g.dim), np.float32))
    out.final_norm = np.asarray(w.final_norm, np.float32).reshape(-1)
    head = w.heads.get("confidence")
    out.confidence = (ProbeHead(head.probes, head.projection, np.asarray(head.bias).reshape(-1))
                      if head is not None else None)
    return out


class Needle2Weights:
    """Seeded Needle 2 weights: every matrix per-row-scaled int8, or with
    cq_bits (2, 3, 4, or 5 for ternary) the shipped archive's Cactus-Quant
    form (model/cact.ts:398-562) of that width with groups of cq_group, or
    with cq_bits "mixed" each matrix in its own width and group
    (cact.mixed_form)."""

    def __init__(self, g: Needle2Geometry, run_seed: int = 2026, cq_bits=0,
                 cq_group: int = 32):
        self.geometry = g
        L, d, hd = g.layers, g.dim, g.head_dim
        if cq_bits:
            from .cact import CqMatrix, mixed_form

            cb = synth.cq_codebook()
            books = {2: cb[0:4], 3: cb[4:12], 4: cb[12:28]}

        def mat(name, n, k, role="", index=0):
            if cq_bits:
                bits, group = (mixed_form(role, index) if cq_bits == "mixed"
                               else (cq_bits, cq_group))
                packed, norms = synth.cq_matrix(run_seed, name, n, k, group, bits,
                                                norm_lo=0.05, norm_hi=0.25)
                return CqMatrix(packed, norms, books, n, k, group, bits)
            w, s = synth.int8_matrix(run_seed, name, n, k, k)
            return Int8Matrix(w, s, k, name)

        def u(name, shape, lo, hi):
            return synth.Stream(run_seed, name).uniform(shape, lo, hi)

        self.embedding = mat("n2.embedding", g.vocab, d, "embedding")
        self.wq = [mat(f"n2.l{l}.wq", g.heads * hd, d, "wq", l) for l in range(L)]
        self.wk = [mat(f"n2.l{l}.wk", g.kv_heads * hd, d, "wk", l) for l in range(L)]
        self.wv = [mat(f"n2.l{l}.wv", g.kv_heads * hd, d, "wv", l) for l in range(L)]
        self.wgate = [mat(f"n2.l{l}.wgate", g.heads * hd, d, "wgate", l) for l in range(L)]
        self.wo = [mat(f"n2.l{l}.wo", d, g.heads * hd, "wo", l) for l in range(L)]
        self.norm_input = u("n2.norm_input", (L, d), -0.1, 0.1)
        self.query_norm = u("n2.query_norm", (L, hd), -0.1, 0.1)
        self.key_norm = u("n2.key_norm", (L, hd), -0.1, 0.1)
        self.post_attn_norm = u("n2.post_attn_norm", (L, d), -0.1, 0.1)
        self.attention_gate = u("n2.attention_gate", (L,), -1.0, 1.0)
        self.pre_hadamard_norm = u("n2.pre_hadamard_norm", (L, d), -0.1, 0.1)
        self.d1 = u("n2.d1", (L, d), 0.5, 1.5)
        self.d2 = u("n2.d2", (L, g.hadamard), 0.5, 1.5)
        self.d3 = u("n2.d3", (L, d), 0.5, 1.5)
        ln = g.lanes
        self.phi_pre = mat("n2.phi_pre", L * ln, ln * d, "phi_pre")
        self.phi_post = mat("n2.phi_post", L * ln, ln * d, "phi_post")
        self.phi_res = mat("n2.phi_res", L * ln * ln, ln * d, "phi_res")
        self.a_pre = u("n2.a_pre", (L,), 0.02, 0.1)
        self.a_post = u("n2.a_post", (L,), 0.02, 0.1)
        self.a_res = u("n2.a_res", (L,), 0.02, 0.1)
        self.b_pre = u("n2.b_pre", (L * ln,), -0.5, 0.5)
        self.b_post = u("n2.b_post", (L * ln,), -0.5, 0.5)
        self.b_res = u("n2.b_res", (L * ln * ln,), -0.5, 0.5)
        cat = g.engram_tables * g.engram_sub
        self.eg_tables = [mat(f"n2.e{s}.tables", g.engram_tables * g.engram_slots, g.engram_sub,
                              "eg_tables", s) for s in range(len(g.sites))]
        self.eg_key = [mat(f"n2.e{s}.key", d, cat, "eg_key", s) for s in range(len(g.sites))]
        self.eg_value = [mat(f"n2.e{s}.value", d, cat, "eg_value", s)
                         for s in range(len(g.sites))]
        self.eg_taps = u("n2.eg_taps", (len(g.sites), g.engram_taps, d), -0.5, 0.5)
        self.final_norm = u("n2.final_norm", (d,), -0.1, 0.1)
        self.confidence = ProbeHead(u("n2.conf.probes", (8, d), -0.1, 0.1),
                                    u("n2.conf.projection", (1, 8 * d), -0.003, 0.003),
                                    u("n2.conf.bias", (1,), -0.2, 0.2))
