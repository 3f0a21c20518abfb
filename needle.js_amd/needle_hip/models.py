"""Synthetic int8 decoder (weights, HBM-resident decoder, batched sessions).

The decoder is the synthetic model of the batched constrained-decode and
prefill workloads (8 layers, d_model 512, 8 heads x 64, FFN 2048, int8 weights
with per-row fp32 scales, vocab 32768), composed from the reference's own
per-token primitives -- the layer recipe is spelled out in
include/needle_hip.h (nd_decoder_desc) and restated by the oracle.

Host side only: every operation runs in libneedle_hip.so.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import lib as L
from . import synth
from .backend import HipBackend, Int8Matrix
from .errors import invariant

MASK_P = 0.02
MASK_THRESHOLD24 = int(round(MASK_P * (1 << 24)))  # allowed iff (z >> 40) < this
PREFIX_SCALE = (0.005, 0.02)  # synthetic prefix KV scale range


@dataclass(frozen=True)
class DecoderGeometry:
    layers: int = 8
    dim: int = 512
    heads: int = 8
    kv_heads: int = 8
    head_dim: int = 64
    ffn: int = 2048
    vocab: int = 32768
    rope_theta: float = 10000.0


class DecoderWeights:
    """Host copy of the synthetic decoder's weights (seeded)."""

    def __init__(self, geometry: DecoderGeometry, run_seed: int = 2026):
        g = geometry
        self.geometry = g
        self.run_seed = run_seed

        def mat(name, n, k):
            w, s = synth.int8_matrix(run_seed, name, n, k, k)
            return Int8Matrix(w, s, k, name)

        self.embedding = mat("embedding", g.vocab, g.dim)
        self.wq = [mat(f"l{l}.wq", g.heads * g.head_dim, g.dim) for l in range(g.layers)]
        self.wk = [mat(f"l{l}.wk", g.kv_heads * g.head_dim, g.dim) for l in range(g.layers)]
        self.wv = [mat(f"l{l}.wv", g.kv_heads * g.head_dim, g.dim) for l in range(g.layers)]
        self.wo = [mat(f"l{l}.wo", g.dim, g.heads * g.head_dim) for l in range(g.layers)]
        self.wup = [mat(f"l{l}.wup", g.ffn, g.dim) for l in range(g.layers)]
        self.wdown = [mat(f"l{l}.wdown", g.dim, g.ffn) for l in range(g.layers)]

        def vec(name, shape):
            return synth.Stream(run_seed, name).uniform(shape, -0.1, 0.1)

        self.attn_norm = vec("attn_norm", (g.layers, g.dim))
        self.ffn_norm = vec("ffn_norm", (g.layers, g.dim))
        self.q_norm = vec("q_norm", (g.layers, g.head_dim))
        self.k_norm = vec("k_norm", (g.layers, g.head_dim))
        self.final_norm = vec("final_norm", (g.dim,))


class HipDecoder:
    """The decoder's weights in HBM (nd_decoder)."""

    def __init__(self, backend: HipBackend, weights: DecoderWeights):
        self.backend = backend
        self.weights = weights
        g = weights.geometry
        self.geometry = g
        lib = backend.lib
        handles = {name: [backend.upload(m) for m in getattr(weights, name)]
                   for name in ("wq", "wk", "wv", "wo", "wup", "wdown")}
        arrays = {name: (C.c_void_p * g.layers)(*[h.value for h in hs])
                  for name, hs in handles.items()}
        self._keep = [arrays]
        desc = L.DecoderDesc()
        desc.layers, desc.dim, desc.heads, desc.kv_heads = g.layers, g.dim, g.heads, g.kv_heads
        desc.head_dim, desc.ffn, desc.vocab, desc.rope_theta = g.head_dim, g.ffn, g.vocab, g.rope_theta
        desc.embedding = backend.upload(weights.embedding)
        for name, arr in arrays.items():
            setattr(desc, name, C.cast(arr, L.PP))
        for name in ("attn_norm", "ffn_norm", "q_norm", "k_norm", "final_norm"):
            arr = np.ascontiguousarray(getattr(weights, name), dtype=np.float32)
            self._keep.append(arr)
            setattr(desc, name, L.ptr(arr))
        handle = C.c_void_p()
        backend._check(lib.nd_decoder_create(backend.ctx, C.byref(desc), C.byref(handle)),
                       "nd_decoder_create")
        self.handle = handle

    def free(self) -> None:
        if self.handle is not None and self.backend.ctx is not None:
            self.backend.lib.nd_decoder_free(self.backend.ctx, self.handle)
        self.handle = None


class HipBatch:
    """B sequences decoding together on the GPU (nd_batch)."""

    def __init__(self, decoder: HipDecoder, batch: int, max_length: int):
        self.decoder = decoder
        self.backend = decoder.backend
        self.lib = self.backend.lib
        self.batch = batch
        self.max_length = max_length
        handle = C.c_void_p()
        self.backend._check(self.lib.nd_batch_create(self.backend.ctx, decoder.handle, batch,
                                                     max_length, C.byref(handle)),
                            "nd_batch_create")
        self.handle = handle

    def fill_synthetic(self, seq: int, seed_k: int, seed_v: int, length: int, index_stride: int,
                       lo: float = PREFIX_SCALE[0], hi: float = PREFIX_SCALE[1]) -> None:
        self.backend._check(self.lib.nd_batch_fill_synthetic(
            self.backend.ctx, self.handle, seq, seed_k, seed_v, length, index_stride, lo, hi),
            "nd_batch_fill_synthetic")

    def set_state(self, tokens, positions, step: int = 0) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        p = np.ascontiguousarray(positions, dtype=np.uint32)
        invariant(t.size == self.batch and p.size == self.batch, "INVALID_CACT",
                  "one token and one position per sequence")
        self.backend._check(self.lib.nd_batch_set_state(self.backend.ctx, self.handle, L.ptr(t),
                                                        L.ptr(p), step), "nd_batch_set_state")

    def step(self, max_position: int, mask_seed: Optional[int] = None,
             threshold24: int = MASK_THRESHOLD24, stream=None) -> None:
        use = 0 if mask_seed is None else 1
        self.backend._check(self.lib.nd_batch_step(
            self.backend.ctx, self.handle, max_position, use, 0 if mask_seed is None else mask_seed,
            threshold24, C.c_void_p(stream) if stream else None), "nd_batch_step")

    def read(self, logits: bool = False):
        t = np.empty(self.batch, np.uint32)
        p = np.empty(self.batch, np.uint32)
        lp = np.empty(self.batch, np.float64)
        lg = np.empty((self.batch, self.decoder.geometry.vocab), np.float32) if logits else None
        self.backend._check(self.lib.nd_batch_read(self.backend.ctx, self.handle, L.ptr(t),
                                                   L.ptr(p), L.ptr(lp),
                                                   L.ptr(lg) if logits else None), "nd_batch_read")
        return t, p, lp, lg

    def read_projections(self):
        """The last layer's Q/K/V projections of the last step, [batch][q|k|v]."""
        g = self.decoder.geometry
        out = np.empty((self.batch, (g.heads + 2 * g.kv_heads) * g.head_dim), np.float32)
        self.backend._check(self.lib.nd_batch_read_projections(self.backend.ctx, self.handle,
                                                               L.ptr(out)),
                            "nd_batch_read_projections")
        return out

    def history(self, first_step: int, steps: int):
        """Selected ids [steps][batch] and log-probabilities recorded on device."""
        ids = np.empty((steps, self.batch), np.uint32)
        lps = np.empty((steps, self.batch), np.float64)
        self.backend._check(self.lib.nd_batch_history(self.backend.ctx, self.handle, first_step,
                                                      steps, L.ptr(ids), L.ptr(lps)),
                            "nd_batch_history")
        return ids, lps

    def kv_read(self, layer: int, seq: int, head: int):
        """(k_codes, v_codes, k_scales, v_scales) of one sequence's KV head."""
        kv = self.lib.nd_batch_kv(self.handle)
        hd = self.decoder.geometry.head_dim
        kc = np.empty((self.max_length, hd), np.int8)
        vc = np.empty((self.max_length, hd), np.int8)
        ks = np.empty(self.max_length, np.float32)
        vs = np.empty(self.max_length, np.float32)
        cache_head = seq * self.decoder.geometry.kv_heads + head
        self.backend._check(self.lib.nd_kv_read(self.backend.ctx, kv, layer, cache_head, L.ptr(kc),
                                                L.ptr(vc), L.ptr(ks), L.ptr(vs)), "nd_kv_read")
        return kc, vc, ks, vs

    def free(self) -> None:
        if self.handle is not None and self.backend.ctx is not None:
            self.lib.nd_batch_free(self.backend.ctx, self.handle)
        self.handle = None


class HipPrefill:
    """One-pass prompt prefill into an int8 KV cache (nd_prefill)."""

    def __init__(self, decoder: HipDecoder, max_tokens: int, max_context: int):
        self.decoder = decoder
        self.backend = decoder.backend
        self.lib = self.backend.lib
        handle = C.c_void_p()
        self.backend._check(self.lib.nd_prefill_create(self.backend.ctx, decoder.handle,
                                                       max_tokens, max_context, C.byref(handle)),
                            "nd_prefill_create")
        self.handle = handle

    def run(self, cache, tokens, position0: int = 0, want_logits: bool = True):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.decoder.geometry.vocab, np.float32) if want_logits else None
        self.backend._check(self.lib.nd_prefill_tokens(self.backend.ctx, self.handle,
                                                       cache.handle, L.ptr(t), t.size, position0,
                                                       L.ptr(logits) if want_logits else None),
                            "nd_prefill_tokens")
        return logits

    def set_tokens(self, tokens, position0: int = 0) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        self.backend._check(self.lib.nd_prefill_set_tokens(self.backend.ctx, self.handle,
                                                           L.ptr(t), t.size, position0),
                            "nd_prefill_set_tokens")

    def launch(self, cache, stream=None) -> None:
        self.backend._check(self.lib.nd_prefill_run_d(self.backend.ctx, self.handle, cache.handle,
                                                      C.c_void_p(stream) if stream else None),
                            "nd_prefill_run_d")

    def phase_ms(self, cache):
        """One eager pass with an event after every kernel: summed ms of
        (int8 GEMMs, causal attention, everything else)."""
        ms = np.zeros(3, np.float32)
        self.backend._check(self.lib.nd_prefill_phase_ms(self.backend.ctx, self.handle,
                                                         cache.handle, L.ptr(ms)),
                            "nd_prefill_phase_ms")
        return float(ms[0]), float(ms[1]), float(ms[2])

    def logits(self):
        out = np.empty(self.decoder.geometry.vocab, np.float32)
        self.backend._check(self.lib.nd_prefill_logits(self.backend.ctx, self.handle,
                                                       L.ptr(out)), "nd_prefill_logits")
        return out

    def read_projections(self, count: int):
        """The last layer's Q/K/V projections of the last run, [count][q|k|v]."""
        g = self.decoder.geometry
        out = np.empty((count, (g.heads + 2 * g.kv_heads) * g.head_dim), np.float32)
        self.backend._check(self.lib.nd_prefill_read_projections(self.backend.ctx, self.handle,
                                                                 L.ptr(out)),
                            "nd_prefill_read_projections")
        return out

    def free(self) -> None:
        if self.handle is not None and self.backend.ctx is not None:
            self.lib.nd_prefill_free(self.backend.ctx, self.handle)
        self.handle = None


@dataclass(frozen=True)
class ConstrainedWorkload:
    """Seeded inputs of a batched constrained decode: per-sequence prefix
    lengths, prefix KV seeds, start tokens, and the mask stream seed."""

    batch: int
    steps: int
    min_context: int
    max_context: int
    vocab: int
    run_seed: int = 2026

    @property
    def lengths(self) -> np.ndarray:
        return synth.Stream(self.run_seed, "ctx-lengths").integers(
            self.batch, self.min_context, self.max_context).astype(np.uint32)

    @property
    def start_tokens(self) -> np.ndarray:
        return synth.Stream(self.run_seed, "start-tokens").integers(
            self.batch, 0, self.vocab - 1).astype(np.uint32)

    @property
    def max_length(self) -> int:
        return self.max_context + self.steps

    def kv_seeds(self, seq: int):
        base = synth.tensor_seed(self.run_seed, "prefix-kv")
        z = synth.splitmix64(base, 2, offset=2 * seq)
        return int(z[0]), int(z[1])

    @property
    def mask_seed(self) -> int:
        return synth.tensor_seed(self.run_seed, "masks")
