"""Needle 2 on the GPU: NeedleRuntime and NeedleModel.generate over nd_needle.

Mirrors the reference's incremental decoder (model/runtime.ts:107-583) and
its greedy generate loop (model/model.ts:88-153) with the same names,
argument meanings and errors:

* ``NeedleRuntime.reset(maximum_length, sink_length)`` -- CONTEXT_OVERFLOW
  outside (0, geometry.max_length] (runtime.ts:150-160);
* ``step(token, want_logits)`` -- INVALID_CACT before reset or for a token
  outside the vocabulary, CONTEXT_OVERFLOW at the runtime limit
  (runtime.ts:280-298);
* ``prefill(tokens)`` -- INVALID_CACT for an empty prompt, CONTEXT_OVERFLOW
  when it does not fit (runtime.ts:227-243);
* ``step_selected(token, allowed)`` -- the step plus selectToken
  (runtime.ts:257-278, 880-899);
* ``NeedleModel.generate(prompt_ids, max_new_tokens, sink_tokens)`` -- token
  ids instead of text (no tokenizer), temperature 0.

Every operation runs in libneedle_hip.so (nd_needle_*); nothing here
computes model arithmetic.
"""

from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

from . import lib as L
from .backend import HipBackend
from .errors import invariant
from .needle2 import Needle2Weights

EOS_TOKEN_ID = 1  # model/tokenizer.ts:4
BOS_TOKEN_ID = 2  # model/tokenizer.ts:5


class HipNeedleSession:
    """The Needle 2 weights resident in HBM plus one runtime state (nd_needle):
    the role of the reference's ResidentExecutionSession
    (backends/backend.ts:66-80) for a whole token."""

    def __init__(self, backend: HipBackend, weights: Needle2Weights,
                 collect_confidence: bool = True):
        self.backend = backend
        self.weights = weights
        g = weights.geometry
        self.geometry = g
        lib = backend.lib
        up = backend.upload
        self._keep: list = []

        def arr(mats):
            a = (C.c_void_p * max(1, len(mats)))(*[up(m).value for m in mats])
            self._keep.append(a)
            return C.cast(a, L.PP)

        def vec(x):
            a = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
            self._keep.append(a)
            return L.ptr(a)

        d = L.NeedleDesc()
        d.vocab, d.dim, d.heads, d.kv_heads = g.vocab, g.dim, g.heads, g.kv_heads
        d.layers, d.head_dim, d.max_length, d.hadamard = g.layers, g.head_dim, g.max_length, g.hadamard
        d.lanes, d.kv_window = g.lanes, g.kv_window
        d.engram_slots, d.engram_sub = g.engram_slots, g.engram_sub
        d.engram_tables, d.engram_taps = g.engram_tables, g.engram_taps
        d.n_orders = len(g.orders)
        for i, o in enumerate(g.orders):
            d.orders[i] = o
        d.n_sites = len(g.sites)
        for i, s in enumerate(g.sites):
            d.sites[i] = s
        d.rope_theta = g.rope_theta
        w = weights
        d.embedding = up(w.embedding)
        d.wq, d.wk, d.wv = arr(w.wq), arr(w.wk), arr(w.wv)
        d.wgate, d.wo = arr(w.wgate), arr(w.wo)
        d.phi_pre, d.phi_post, d.phi_res = up(w.phi_pre), up(w.phi_post), up(w.phi_res)
        d.eg_tables, d.eg_key, d.eg_value = arr(w.eg_tables), arr(w.eg_key), arr(w.eg_value)
        for name in ("norm_input", "query_norm", "key_norm", "post_attn_norm",
                     "pre_hadamard_norm", "d1", "d2", "d3", "attention_gate", "a_pre",
                     "a_post", "a_res", "b_pre", "b_post", "b_res", "eg_taps", "final_norm"):
            setattr(d, name, vec(getattr(w, name)))
        # The confidence pool runs whenever the weights carry the head, as
        # the reference's does unless collectConfidence is false
        # (model/runtime.ts:215-224).
        head = getattr(w, "confidence", None)
        self.has_confidence = bool(collect_confidence and head is not None)
        if self.has_confidence:
            d.probes = vec(head.probes)
            d.probe_count, d.probe_out = head.probe_count, head.output_size
            d.probe_projection = vec(head.projection)
            d.probe_bias = vec(head.bias)
        handle = C.c_void_p()
        backend._check(lib.nd_needle_create(backend.ctx, C.byref(d), C.byref(handle)),
                       "nd_needle_create")
        self.handle = handle
        self.lib = lib

    def _check(self, status: int, what: str) -> None:
        self.backend._check(status, what)

    def confidence(self) -> Optional[float]:
        """residentConfidence (backends/backend.ts:77): the probe head over
        every cell pooled since reset, or None without a head."""
        if not self.has_confidence:
            return None
        out = C.c_double()
        self._check(self.lib.nd_needle_confidence(self.backend.ctx, self.handle, C.byref(out)),
                    "nd_needle_confidence")
        return float(out.value)

    def reset(self, maximum_length: int, sink_length: int = 0) -> None:
        invariant(isinstance(maximum_length, (int, np.integer)) and maximum_length > 0,
                  "CONTEXT_OVERFLOW",
                  f"Runtime length {maximum_length} is outside model limit {self.geometry.max_length}")
        self._check(self.lib.nd_needle_reset(self.backend.ctx, self.handle, int(maximum_length),
                                             max(0, int(sink_length))), "nd_needle_reset")

    @property
    def position(self) -> int:
        return int(self.lib.nd_needle_position(self.handle))

    def step(self, token: int, want_logits: bool = True) -> Optional[np.ndarray]:
        logits = np.empty(self.geometry.vocab, dtype=np.float32) if want_logits else None
        self._check(self.lib.nd_needle_step(self.backend.ctx, self.handle, _token(token),
                                            L.ptr(logits) if logits is not None else None),
                    "nd_needle_step")
        return logits

    def prefill(self, tokens: Sequence[int], want_logits: bool = True) -> Optional[np.ndarray]:
        ids = _ids(tokens)
        logits = np.empty(self.geometry.vocab, dtype=np.float32) if want_logits else None
        self._check(self.lib.nd_needle_prefill(self.backend.ctx, self.handle, L.ptr(ids),
                                               ids.size,
                                               L.ptr(logits) if logits is not None else None),
                    "nd_needle_prefill")
        return logits

    def step_selected(self, token: int, allowed: Optional[np.ndarray] = None):
        out_id, out_lp = C.c_uint32(), C.c_double()
        if allowed is None:
            st = self.lib.nd_needle_step_select(self.backend.ctx, self.handle, _token(token), None,
                                                0, C.byref(out_id), C.byref(out_lp))
        else:
            a = np.ascontiguousarray(allowed, dtype=np.uint32)
            invariant(a.size > 0, "INVALID_CACT", "Allowed token set is empty")
            st = self.lib.nd_needle_step_select(self.backend.ctx, self.handle, _token(token),
                                                L.ptr(a), a.size, C.byref(out_id),
                                                C.byref(out_lp))
        self._check(st, "nd_needle_step_select")
        return int(out_id.value), float(out_lp.value)

    def generate(self, prompt: Sequence[int], max_new_tokens: int, sink: int = 0,
                 eos: Optional[int] = EOS_TOKEN_ID):
        ids = _ids(prompt)
        n = max(0, int(max_new_tokens))
        out_ids = np.zeros(max(1, n), dtype=np.uint32)
        out_lp = np.zeros(max(1, n), dtype=np.float64)
        count = C.c_uint32()
        self._check(self.lib.nd_needle_generate(
            self.backend.ctx, self.handle, L.ptr(ids), ids.size, n, max(0, int(sink)),
            0xFFFFFFFF if eos is None else int(eos), L.ptr(out_ids), L.ptr(out_lp),
            C.byref(count)), "nd_needle_generate")
        k = int(count.value)
        return out_ids[:k].copy(), out_lp[:k].copy()

    def kv_read(self, layer: int, head: int):
        """(k codes, v codes, k scales, v scales) of one (layer, KV head)."""
        kv = self.lib.nd_needle_kv(self.handle)
        invariant(kv is not None, "INVALID_CACT", "Call runtime.reset() before decoding")
        alloc = C.c_uint32()
        self._check(self.lib.nd_kv_info(kv, C.byref(alloc), None, None, None, None), "nd_kv_info")
        alloc = alloc.value
        hd = self.geometry.head_dim
        kc = np.empty((alloc, hd), np.int8)
        vc = np.empty((alloc, hd), np.int8)
        ks = np.empty(alloc, np.float32)
        vs = np.empty(alloc, np.float32)
        self._check(self.lib.nd_kv_read(self.backend.ctx, kv, layer, head, L.ptr(kc), L.ptr(vc),
                                        L.ptr(ks), L.ptr(vs)), "nd_kv_read")
        return kc, vc, ks, vs

    def free(self) -> None:
        if self.handle is not None and self.backend.ctx is not None:
            self.lib.nd_needle_free(self.backend.ctx, self.handle)
        self.handle = None


def _token(token) -> int:
    invariant(isinstance(token, (int, np.integer)) and 0 <= int(token) < 2**32, "INVALID_CACT",
              f"Token {token} is outside the vocabulary")
    return int(token)


def _ids(tokens) -> np.ndarray:
    arr = np.asarray(tokens)
    invariant(arr.ndim == 1 and arr.size > 0, "INVALID_CACT",
              "Cannot prefill an empty token sequence")
    invariant(np.issubdtype(arr.dtype, np.integer) and (arr >= 0).all(), "INVALID_CACT",
              "Token ids must be non-negative integers")
    return np.ascontiguousarray(arr, dtype=np.uint32)


class NeedleRuntime:
    """Incremental one-token Needle 2 decoder (model/runtime.ts:107-583)."""

    def __init__(self, session: HipNeedleSession):
        self.session = session
        self.weights = session.weights
        self._maximum_length = 0

    @property
    def position(self) -> int:
        return self.session.position

    @property
    def maximum_length(self) -> int:
        return self._maximum_length

    def reset(self, maximum_length: int, sink_length: int = 0) -> None:
        self.session.reset(maximum_length, sink_length)
        self._maximum_length = int(maximum_length)

    def prefill(self, tokens: Sequence[int]) -> np.ndarray:
        return self.session.prefill(tokens)

    def prefill_selected(self, tokens: Sequence[int], allowed: Optional[np.ndarray] = None):
        invariant(len(tokens) > 0, "INVALID_CACT", "Cannot prefill an empty token sequence")
        if len(tokens) > 1:
            self.session.prefill(tokens[:-1], want_logits=False)
        return self.session.step_selected(tokens[-1], allowed)

    def step(self, token: int, want_logits: bool = True) -> Optional[np.ndarray]:
        return self.session.step(token, want_logits)

    def step_selected(self, token: int, allowed: Optional[np.ndarray] = None):
        return self.session.step_selected(token, allowed)

    def resolve_confidence(self) -> Optional[float]:
        """resolveConfidence (model/runtime.ts:634-639) from the resident pool."""
        return self.session.confidence()


@dataclass
class GenerationResult:
    token_ids: List[int]
    token_log_probabilities: List[float]
    finish_reason: str  # "eos" | "length"
    prompt_tokens: int
    generated_tokens: int
    elapsed_ms: float
    tokens_per_second: float


class NeedleModel:
    """NeedleModel.generate (model/model.ts:88-153) at temperature 0 over
    token ids: prefill, then greedy argmax tokens with their logSoftmaxAt,
    stopping before EOS or after max_new_tokens."""

    def __init__(self, backend: HipBackend, weights: Needle2Weights,
                 collect_confidence: bool = True):
        self.backend = backend
        self.weights = weights
        self.session = HipNeedleSession(backend, weights, collect_confidence)

    def create_runtime(self) -> NeedleRuntime:
        return NeedleRuntime(self.session)

    def generate(self, prompt_ids: Sequence[int], max_new_tokens: int = 96,
                 sink_tokens: int = 0, eos: Optional[int] = EOS_TOKEN_ID) -> GenerationResult:
        started = time.perf_counter()
        n = max(0, int(max_new_tokens))
        ids, lps = self.session.generate(prompt_ids, n, sink_tokens, eos)
        elapsed = (time.perf_counter() - started) * 1000.0
        g = self.weights.geometry
        room = min(g.max_length, len(prompt_ids) + n) - len(prompt_ids)
        finish = "eos" if len(ids) < min(n, max(room, 0)) else "length"
        return GenerationResult([int(t) for t in ids], [float(v) for v in lps], finish,
                                len(prompt_ids), len(ids), elapsed,
                                len(ids) / max(elapsed / 1000.0, 1e-9))

    def dispose(self) -> None:
        self.session.free()
