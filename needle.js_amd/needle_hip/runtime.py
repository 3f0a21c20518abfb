"""Needle 2 on the GPU: the backend's resident session, NeedleRuntime and
NeedleModel.

* ``Needle2Resident`` -- the Needle 2 weights resident in HBM plus one
  runtime state (``nd_needle``), with the whole-step extension calls
  (``nd_needle_step`` / ``_prefill`` / ``_step_select`` / ``_generate``) and
  the session calls below.
* ``HipNeedleSession`` -- ``ResidentExecutionSession``
  (backends/backend.ts:65-80) at method granularity: ``reset(options)``,
  ``forward(request)``, ``begin_resident_token``, ``prepare_resident_engrams``,
  ``forward_resident_token`` / ``_layer``, ``finish_resident_token``,
  ``finish_resident_token_for_selection``, ``select_resident_token``,
  ``resident_layers_enabled``, ``resident_confidence``,
  ``read_resident_lanes``, ``dispose``.  ``HipBackend.create_resident_session()``
  returns one for the backend's Needle 2 weights.
* ``NeedleRuntime`` -- the reference's incremental decoder
  (model/runtime.ts:107-878) restated with its control flow unchanged: it
  drives the backend (``row``, ``matvec_batch``, ``matvec``) and the session
  exactly where runtime.ts does, and computes on the host only what
  runtime.ts computes there (the scaled embedding, the engram hashes, and --
  for a token that does not run resident -- the lane mix before ``forward``,
  the engram ring and the confidence pool).
* ``ResidentRuntime`` -- the whole-step extension (one launch sequence or HIP
  graph per token, batched prompt passes).
* ``NeedleModel`` -- ``generate`` (model/model.ts:88-153, 202-240: greedy or
  temperature / top-k sampling with xorshift32, abort signal) over
  ``NeedleRuntime``, and ``generate_resident`` over the graph-replayed steps.

Token ids stand in for text: there is no tokenizer on this path.
"""

from __future__ import annotations

import ctypes as C
import math
import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import numpy as np

from . import lib as L
from .backend import HipBackend, MatrixRowRange, MatvecRequest
from .errors import NeedleError, invariant
from .needle2 import Needle2Weights

EOS_TOKEN_ID = 1  # model/tokenizer.ts:4
BOS_TOKEN_ID = 2  # model/tokenizer.ts:5
ENGRAM_SEED = 0x9E3779B9  # model/runtime.ts:22
ENGRAM_PRIME = 0x01000193  # model/runtime.ts:23
_U32 = 0xFFFFFFFF


# ------------------------------------------------------------ nd_needle

class Needle2Resident:
    """The Needle 2 weights in HBM plus one runtime state (nd_needle)."""

    def __init__(self, backend: HipBackend, weights: Needle2Weights):
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
        head = getattr(w, "confidence", None)
        self.has_head = head is not None
        if self.has_head:
            d.probes = vec(head.probes)
            d.probe_count, d.probe_out = head.probe_count, head.output_size
            d.probe_projection = vec(head.projection)
            d.probe_bias = vec(head.bias)
        handle = C.c_void_p()
        backend._check(lib.nd_needle_create(backend.ctx, C.byref(d), C.byref(handle)),
                       "nd_needle_create")
        self.handle = handle
        self.lib = lib
        self.collect_confidence = True
        self.kv_cache = "int8"

    @property
    def ctx(self):
        return self.backend.ctx

    def _check(self, status: int, what: str) -> None:
        self.backend._check(status, what)

    @property
    def has_confidence(self) -> bool:
        return self.has_head and self.collect_confidence

    def confidence(self) -> Optional[float]:
        """The probe head over every cell pooled since reset (None without a
        head or with collectConfidence off)."""
        if not self.has_confidence:
            return None
        out = C.c_double()
        self._check(self.lib.nd_needle_confidence(self.ctx, self.handle, C.byref(out)),
                    "nd_needle_confidence")
        return float(out.value)

    def reset(self, maximum_length: int, sink_length: int = 0, kv_cache: str = "int8",
              collect_confidence: bool = True) -> bool:
        """nd_needle_reset; False when this runtime does not keep `kv_cache`."""
        invariant(isinstance(maximum_length, (int, np.integer)) and maximum_length > 0,
                  "CONTEXT_OVERFLOW",
                  f"Runtime length {maximum_length} is outside model limit {self.geometry.max_length}")
        invariant(kv_cache in ("int8", "float32"), "INVALID_CACT", f"unknown kvCache {kv_cache}")
        mode = L.ND_KV_INT8 if kv_cache == "int8" else L.ND_KV_FLOAT32
        status = self.lib.nd_needle_reset(self.ctx, self.handle, int(maximum_length),
                                          max(0, int(sink_length)), mode,
                                          1 if collect_confidence else 0)
        if status == L.ND_ERR_UNSUPPORTED:
            return False
        self._check(status, "nd_needle_reset")
        self.collect_confidence = bool(collect_confidence)
        self.kv_cache = kv_cache
        return True

    @property
    def position(self) -> int:
        return int(self.lib.nd_needle_position(self.handle))

    # -- whole-step extension -------------------------------------------
    def step(self, token: int, want_logits: bool = True) -> Optional[np.ndarray]:
        logits = np.empty(self.geometry.vocab, dtype=np.float32) if want_logits else None
        self._check(self.lib.nd_needle_step(self.ctx, self.handle, _token(token),
                                            L.ptr(logits) if logits is not None else None),
                    "nd_needle_step")
        return logits

    def prefill(self, tokens: Sequence[int], want_logits: bool = True) -> Optional[np.ndarray]:
        ids = _ids(tokens)
        logits = np.empty(self.geometry.vocab, dtype=np.float32) if want_logits else None
        self._check(self.lib.nd_needle_prefill(self.ctx, self.handle, L.ptr(ids), ids.size,
                                               L.ptr(logits) if logits is not None else None),
                    "nd_needle_prefill")
        return logits

    def step_selected(self, token: int, allowed: Optional[np.ndarray] = None):
        out_id, out_lp = C.c_uint32(), C.c_double()
        if allowed is None:
            st = self.lib.nd_needle_step_select(self.ctx, self.handle, _token(token), None, 0,
                                                C.byref(out_id), C.byref(out_lp))
        else:
            a = np.ascontiguousarray(allowed, dtype=np.uint32)
            invariant(a.size > 0, "INVALID_CACT", "Allowed token set is empty")
            st = self.lib.nd_needle_step_select(self.ctx, self.handle, _token(token), L.ptr(a),
                                                a.size, C.byref(out_id), C.byref(out_lp))
        self._check(st, "nd_needle_step_select")
        return int(out_id.value), float(out_lp.value)

    def grammar_mask(self, masker, state: np.ndarray, budget: int):
        """nd_needle_grammar_mask: the allowed mask of the grammar state
        words `state` into the model's mask buffer; returns (the number of
        allowed pieces, the undecided ids ascending)."""
        st = np.ascontiguousarray(state, dtype=np.uint32)
        words = (self.geometry.vocab + 31) // 32
        und = np.zeros(words, np.uint32)
        count = C.c_uint32()
        self._check(self.lib.nd_needle_grammar_mask(self.ctx, self.handle, masker._grammar,
                                                    masker._pieces, L.ptr(st), st.size,
                                                    max(0, int(budget)), L.ptr(und),
                                                    C.byref(count)), "nd_needle_grammar_mask")
        bits = np.unpackbits(und.view(np.uint8), bitorder="little")[: self.geometry.vocab]
        return int(count.value), np.flatnonzero(bits).astype(np.uint32)

    def step_selected_mask(self, token: int, settled: Sequence[int] = ()):
        """stepSelected over the mask buffer plus the `settled` ids."""
        ids = np.ascontiguousarray(settled, dtype=np.uint32)
        out_id, out_lp = C.c_uint32(), C.c_double()
        self._check(self.lib.nd_needle_step_select_mask(
            self.ctx, self.handle, _token(token), L.ptr(ids) if ids.size else None, ids.size,
            C.byref(out_id), C.byref(out_lp)), "nd_needle_step_select_mask")
        return int(out_id.value), float(out_lp.value)

    def generate(self, prompt: Sequence[int], max_new_tokens: int, sink: int = 0,
                 eos: Optional[int] = EOS_TOKEN_ID):
        ids = _ids(prompt)
        n = max(0, int(max_new_tokens))
        out_ids = np.zeros(max(1, n), dtype=np.uint32)
        out_lp = np.zeros(max(1, n), dtype=np.float64)
        count = C.c_uint32()
        self._check(self.lib.nd_needle_generate(
            self.ctx, self.handle, L.ptr(ids), ids.size, n, max(0, int(sink)),
            0xFFFFFFFF if eos is None else int(eos), L.ptr(out_ids), L.ptr(out_lp),
            C.byref(count)), "nd_needle_generate")
        k = int(count.value)
        return out_ids[:k].copy(), out_lp[:k].copy()

    def step_launches(self) -> int:
        """Kernel launches of the decode-step graph (nd_needle_step_launches;
        0 before the first generate step)."""
        n = C.c_uint32()
        self._check(self.lib.nd_needle_step_launches(self.ctx, self.handle, C.byref(n)),
                    "nd_needle_step_launches")
        return int(n.value)

    def test_waits(self, extra_arrivals: int, spin_rounds: int) -> None:
        """Test hook (nd_needle_test_waits): the fused layer launch's mix
        waits for `extra_arrivals` more output-projection workgroups than it
        has, every wait bounded at `spin_rounds` rounds (0: the default), so
        that a whole-step call sees a wait run out; (0, 0) restores."""
        self._check(self.lib.nd_needle_test_waits(self.ctx, self.handle, int(extra_arrivals),
                                                  int(spin_rounds)), "nd_needle_test_waits")

    # -- session calls ---------------------------------------------------
    def begin_token(self, lanes: np.ndarray) -> None:
        x = _f32(lanes, self.geometry.lanes * self.geometry.dim, "Resident lane input")
        self._check(self.lib.nd_needle_begin_token(self.ctx, self.handle, L.ptr(x)),
                    "nd_needle_begin_token")

    def prepare_engrams(self, indices, valid, position: int) -> None:
        idx = np.ascontiguousarray(indices, dtype=np.uint32)
        ok = np.ascontiguousarray(valid, dtype=np.uint32)
        invariant(idx.size == ok.size, "INVALID_CACT", "engram indices and flags differ in length")
        self._check(self.lib.nd_needle_prepare_engrams(self.ctx, self.handle, L.ptr(idx),
                                                       L.ptr(ok), idx.size, int(position)),
                    "nd_needle_prepare_engrams")

    def forward_layer(self, layer: int, position: int, key=None, value=None) -> None:
        d = self.geometry.dim
        k = None if key is None else _f32(key, d, "engram key")
        v = None if value is None else _f32(value, d, "engram value")
        self._check(self.lib.nd_needle_forward_layer(
            self.ctx, self.handle, int(layer), int(position), L.ptr(k) if k is not None else None,
            L.ptr(v) if v is not None else None), "nd_needle_forward_layer")

    def forward_token(self, position: int, keys=None, values=None) -> None:
        g = self.geometry
        n = len(g.sites) * g.dim
        k = None if keys is None else _f32(np.concatenate(keys), n, "engram keys")
        v = None if values is None else _f32(np.concatenate(values), n, "engram values")
        self._check(self.lib.nd_needle_forward_token(
            self.ctx, self.handle, int(position), L.ptr(k) if k is not None else None,
            L.ptr(v) if v is not None else None), "nd_needle_forward_token")

    def finish_token(self, want_logits: bool) -> Optional[np.ndarray]:
        logits = np.empty(self.geometry.vocab, dtype=np.float32) if want_logits else None
        self._check(self.lib.nd_needle_finish_token(self.ctx, self.handle, 1 if want_logits else 0,
                                                    L.ptr(logits) if want_logits else None),
                    "nd_needle_finish_token")
        return logits

    def finish_token_for_selection(self) -> None:
        self._check(self.lib.nd_needle_finish_token_for_selection(self.ctx, self.handle),
                    "nd_needle_finish_token_for_selection")

    def select_token(self, allowed: Optional[np.ndarray] = None):
        out_id, out_lp = C.c_uint32(), C.c_double()
        if allowed is None:
            st = self.lib.nd_needle_select_token(self.ctx, self.handle, None, 0, C.byref(out_id),
                                                 C.byref(out_lp))
        else:
            a = np.ascontiguousarray(allowed, dtype=np.uint32)
            st = self.lib.nd_needle_select_token(self.ctx, self.handle, L.ptr(a), a.size,
                                                 C.byref(out_id), C.byref(out_lp))
        self._check(st, "nd_needle_select_token")
        return int(out_id.value), float(out_lp.value)

    def select_token_mask(self, settled: Sequence[int] = ()):
        """selectResidentToken over the mask buffer plus the `settled` ids."""
        ids = np.ascontiguousarray(settled, dtype=np.uint32)
        out_id, out_lp = C.c_uint32(), C.c_double()
        self._check(self.lib.nd_needle_select_token_mask(
            self.ctx, self.handle, L.ptr(ids) if ids.size else None, ids.size, C.byref(out_id),
            C.byref(out_lp)), "nd_needle_select_token_mask")
        return int(out_id.value), float(out_lp.value)

    def read_lanes(self) -> np.ndarray:
        g = self.geometry
        out = np.empty(g.lanes * g.dim, dtype=np.float32)
        self._check(self.lib.nd_needle_read_lanes(self.ctx, self.handle, L.ptr(out)),
                    "nd_needle_read_lanes")
        return out

    def forward(self, layer: int, position: int, attention_input, block_input, update_input, x,
                phi_post, phi_residual) -> np.ndarray:
        g = self.geometry
        d, ln = g.dim, g.lanes
        a = _f32(attention_input, d, "attention input")
        b = _f32(block_input, d, "block input")
        u = _f32(update_input, d, "update input")
        xx = _f32(x, ln * d, "lanes")
        pp = _f32(phi_post, ln, "phi post")
        pr = _f32(phi_residual, ln * ln, "phi residual")
        out = np.empty(ln * d, dtype=np.float32)
        self._check(self.lib.nd_needle_forward(self.ctx, self.handle, int(layer), int(position),
                                               L.ptr(a), L.ptr(b), L.ptr(u), L.ptr(xx), L.ptr(pp),
                                               L.ptr(pr), L.ptr(out)), "nd_needle_forward")
        return out

    def kv_read(self, layer: int, head: int):
        """(k codes, v codes, k scales, v scales) of one (layer, KV head);
        float32 rows instead of codes in kvCache "float32" mode."""
        kv = self.lib.nd_needle_kv(self.handle)
        invariant(kv is not None, "INVALID_CACT", "Call runtime.reset() before decoding")
        alloc = C.c_uint32()
        self._check(self.lib.nd_kv_info(kv, C.byref(alloc), None, None, None, None), "nd_kv_info")
        alloc = alloc.value
        hd = self.geometry.head_dim
        dt = np.float32 if self.kv_cache == "float32" else np.int8
        kc = np.empty((alloc, hd), dt)
        vc = np.empty((alloc, hd), dt)
        ks = np.empty(alloc, np.float32)
        vs = np.empty(alloc, np.float32)
        self._check(self.lib.nd_kv_read(self.ctx, kv, layer, head, L.ptr(kc), L.ptr(vc),
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


def _f32(values, size: int, what: str) -> np.ndarray:
    a = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    invariant(a.size == size, "INVALID_CACT", f"{what} must contain {size} values")
    return a


# -------------------------------------------- ResidentExecutionSession

@dataclass(frozen=True)
class ResidentExecutionResetOptions:
    """backends/backend.ts:17-22."""

    maximum_length: int
    sink_length: int
    kv_cache: str = "int8"
    collect_confidence: bool = True


@dataclass(frozen=True)
class ResidentLayerFallbackRequest:
    """backends/backend.ts:29-39."""

    layer_index: int
    position: int
    input: np.ndarray
    block_input: np.ndarray
    update_input: np.ndarray
    x: np.ndarray
    phi_post: np.ndarray
    phi_residual: np.ndarray


@dataclass(frozen=True)
class ResidentLayerFallbackResult:
    """backends/backend.ts:24-27: kind "projected" | "delta" | "nextX"."""

    kind: str
    values: np.ndarray


@dataclass(frozen=True)
class SelectedToken:
    """backends/backend.ts:41-44."""

    id: int
    log_probability: float


@dataclass(frozen=True)
class DeviceMaskSelection:
    """A selection request whose allowed set is the resident model's mask
    buffer (nd_needle_grammar_mask) plus the host-settled ids."""

    settled: List[int]


@dataclass(frozen=True)
class ResidentEngramRequest:
    """backends/backend.ts:46-50."""

    indices: np.ndarray
    valid: np.ndarray
    position: int


@dataclass(frozen=True)
class ResidentTokenRequest:
    """backends/backend.ts:52-56."""

    position: int
    engram_keys: Sequence[np.ndarray] = ()
    engram_values: Sequence[np.ndarray] = ()


@dataclass(frozen=True)
class ResidentLayerRequest:
    """backends/backend.ts:58-63."""

    layer_index: int
    position: int
    engram_key: Optional[np.ndarray] = None
    engram_value: Optional[np.ndarray] = None


class HipNeedleSession:
    """ResidentExecutionSession (backends/backend.ts:65-80) over one
    nd_needle.  With resident_layers (the default) a whole token runs on the
    device; without, begin_resident_token and prepare_resident_engrams
    return False and the runtime calls forward() once per layer, which
    returns the next lanes ("nextX")."""

    def __init__(self, backend: HipBackend, weights: Needle2Weights, resident_layers: bool = True):
        self.resident = Needle2Resident(backend, weights)
        self.weights = weights
        self.geometry = weights.geometry
        self.resident_layers = bool(resident_layers)
        self._enabled = False
        self._disposed = False

    # contract ------------------------------------------------------------
    def reset(self, options: ResidentExecutionResetOptions) -> bool:
        invariant(not self._disposed, "BACKEND_UNAVAILABLE", "Resident session was disposed")
        self._enabled = self.resident.reset(options.maximum_length, options.sink_length,
                                            options.kv_cache, options.collect_confidence)
        return self._enabled

    def forward(self, request: ResidentLayerFallbackRequest) -> ResidentLayerFallbackResult:
        invariant(self._enabled and not self._disposed, "BACKEND_UNAVAILABLE",
                  "Fused attention is off")
        values = self.resident.forward(request.layer_index, request.position, request.input,
                                       request.block_input, request.update_input, request.x,
                                       request.phi_post, request.phi_residual)
        return ResidentLayerFallbackResult("nextX", values)

    def begin_resident_token(self, lanes: np.ndarray) -> bool:
        if not self.resident_layers_enabled() or self._disposed:
            return False
        self.resident.begin_token(lanes)
        return True

    def prepare_resident_engrams(self, request: ResidentEngramRequest) -> bool:
        if not self.resident_layers_enabled() or self._disposed:
            return False
        self.resident.prepare_engrams(request.indices, request.valid, request.position)
        return True

    def forward_resident_token(self, request: ResidentTokenRequest) -> None:
        self._on()
        keys = list(request.engram_keys) if request.engram_keys else None
        values = list(request.engram_values) if request.engram_values else None
        self.resident.forward_token(request.position, keys, values)

    def forward_resident_layer(self, request: ResidentLayerRequest) -> None:
        self._on()
        self.resident.forward_layer(request.layer_index, request.position, request.engram_key,
                                    request.engram_value)

    def finish_resident_token(self, want_logits: bool) -> Optional[np.ndarray]:
        self._on()
        return self.resident.finish_token(want_logits)

    def finish_resident_token_for_selection(self) -> None:
        self._on()
        self.resident.finish_token_for_selection()

    def select_resident_token(self, allowed_token_ids: Optional[np.ndarray] = None) -> SelectedToken:
        self._on()
        if isinstance(allowed_token_ids, DeviceMaskSelection):
            token, lp = self.resident.select_token_mask(allowed_token_ids.settled)
        else:
            token, lp = self.resident.select_token(allowed_token_ids)
        return SelectedToken(token, lp)

    def resident_layers_enabled(self) -> bool:
        return self._enabled and self.resident_layers

    def resident_confidence(self) -> Optional[float]:
        if not self.resident_layers_enabled() or self._disposed:
            return None
        return self.resident.confidence()

    def read_resident_lanes(self) -> np.ndarray:
        self._on()
        return self.resident.read_lanes()

    def dispose(self) -> None:
        if self._disposed:
            return
        self._disposed = True
        self.resident.free()

    # helpers -------------------------------------------------------------
    def _on(self) -> None:
        invariant(self.resident_layers_enabled() and not self._disposed, "BACKEND_UNAVAILABLE",
                  "Resident layers are off")

    def kv_read(self, layer: int, head: int):
        return self.resident.kv_read(layer, head)

    @property
    def handle(self):
        return self.resident.handle


# ---------------------------------------------- the runtime's host math
#
# What runtime.ts computes on the host itself (math.ts, JavaScript numbers:
# float64 arithmetic left to right, Float32Array stores).

def _seq_sum(v: np.ndarray) -> float:
    """Left-to-right float64 sum (a JavaScript accumulation loop)."""
    return float(np.add.accumulate(v, dtype=np.float64)[-1]) if v.size else 0.0


def _lane_mean(x: np.ndarray, lanes: int) -> np.ndarray:
    """runtime.ts:544-549, 570-575: sum over lanes in order, / lanes, f32."""
    xl = x.reshape(lanes, -1).astype(np.float64)
    acc = np.zeros(xl.shape[1])
    for lane in range(lanes):
        acc = acc + xl[lane]
    return (acc / lanes).astype(np.float32)


def sigmoid(value: float) -> float:
    """math.ts:3-10."""
    if value >= 0:
        return 1.0 / (1.0 + math.exp(-value))
    e = math.exp(value)
    return e / (1.0 + e)


def rms_unit(x: np.ndarray) -> np.ndarray:
    """math.ts:34-44."""
    v = x.astype(np.float64)
    inverse = 1.0 / math.sqrt(_seq_sum(v * v) / v.size + 1e-6)
    return (v * inverse).astype(np.float32)


def rms_norm(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """math.ts:16-32."""
    v = x.astype(np.float64)
    inverse = 1.0 / math.sqrt(_seq_sum(v * v) / v.size + 1e-6)
    return ((1.0 + scale.astype(np.float64)) * v * inverse).astype(np.float32)


def log_softmax_at(logits: np.ndarray, token: int) -> float:
    """math.ts:153-160 over the full vocabulary."""
    v = logits.astype(np.float64)
    maximum = float(np.max(v))
    return float(v[token] - maximum - math.log(_seq_sum(np.exp(v - maximum))))


def argmax(values: np.ndarray) -> int:
    """math.ts:140-151: the first maximum, scanning with `>` from index 0 --
    so a NaN at index 0 wins (nothing compares greater than it) and a NaN
    anywhere else never does."""
    v = np.asarray(values)
    if v.size == 0 or np.isnan(v[0]):
        return 0
    return int(np.argmax(np.where(np.isnan(v), -np.inf, v)))


class OnlineProbePool:
    """model/runtime.ts:48-105, the pool of a token that does not run resident."""

    def __init__(self, head, dimension: int):
        self.head = head
        self.dimension = dimension
        self.maximum = np.full(head.probe_count, -math.inf)
        self.denominator = np.zeros(head.probe_count)
        self.weighted = np.zeros((head.probe_count, dimension))

    def add(self, cell: np.ndarray) -> None:
        c = cell.astype(np.float64)
        scale = 1.0 / math.sqrt(self.dimension)
        for p in range(self.head.probe_count):
            score = _seq_sum(c * self.head.probes[p].astype(np.float64)) * scale
            previous = self.maximum[p]
            if score <= previous:
                weight = math.exp(score - previous)
                self.denominator[p] += weight
                self.weighted[p] += weight * c
            else:
                old = math.exp(previous - score) if math.isfinite(previous) else 0.0
                self.denominator[p] = self.denominator[p] * old + 1.0
                self.weighted[p] = self.weighted[p] * old + c
                self.maximum[p] = score

    def output(self) -> np.ndarray:
        pooled = (self.weighted / np.maximum(self.denominator, 1e-30)[:, None]).astype(np.float32)
        flat = pooled.reshape(-1).astype(np.float64)
        out = np.empty(self.head.output_size, np.float32)
        for o in range(self.head.output_size):  # denseMatvec (backends/cq.ts:297-318)
            out[o] = _seq_sum(flat * self.head.projection[o].astype(np.float64)) + float(self.head.bias[o])
        return out


@dataclass(frozen=True)
class RuntimeOptions:
    """model/runtime.ts:30-40."""

    kv_cache: str = "int8"
    collect_confidence: bool = True
    on_layer: Optional[Callable[[dict], None]] = None


class AbortSignal:
    """The AbortSignal a caller hands to prefill/step/generate."""

    def __init__(self):
        self.aborted = False
        self.reason = None

    def abort(self, reason=None) -> None:
        self.aborted = True
        self.reason = reason


def _check_abort(signal: Optional[AbortSignal]) -> None:
    if signal is not None and signal.aborted:
        raise NeedleError("GENERATION_ABORTED", "Needle generation was aborted",
                          signal.reason if isinstance(signal.reason, BaseException) else None)


class NeedleRuntime:
    """Incremental one-token Needle 2 decoder (model/runtime.ts:107-878),
    control flow unchanged, over an InferenceBackend and its resident
    session.  Where runtime.ts keeps its own int8 KV cache (a backend whose
    session declines the reset) this restatement stops: every option this
    backend is asked for is kept by its session."""

    def __init__(self, weights: Needle2Weights, backend: HipBackend,
                 options: RuntimeOptions = RuntimeOptions()):
        self.weights = weights
        self.backend = backend
        self.options = options
        self.geometry = weights.geometry
        self.session: Optional[HipNeedleSession] = backend.create_resident_session()
        self._maximum_length = 0
        self._sink_length = 0
        self._position = 0
        self._history: List[int] = []
        self._engram_ring = np.zeros(0, np.float32)
        self._engram_valid = np.zeros(0, np.uint8)
        self._engram_depth = 0
        self._engram_position = 0
        self._pool: Optional[OnlineProbePool] = None
        self._session_enabled = False
        self._uses_resident_confidence = False
        self._selection_request = None
        self._selection_active = False
        self._selection_result: Optional[SelectedToken] = None

    @property
    def position(self) -> int:
        return self._position

    @property
    def maximum_length(self) -> int:
        return self._maximum_length

    def reset(self, maximum_length: int, sink_length: int = 0) -> None:
        """runtime.ts:150-225."""
        g = self.geometry
        invariant(isinstance(maximum_length, (int, np.integer)) and 0 < maximum_length <= g.max_length,
                  "CONTEXT_OVERFLOW",
                  f"Runtime length {maximum_length} is outside model limit {g.max_length}")
        self._maximum_length = int(maximum_length)
        self._sink_length = min(max(int(sink_length or 0), 0), self._maximum_length)
        self._position = 0
        self._history = []
        self._selection_active = False
        self._selection_result = None
        self._session_enabled = bool(self.session and self.session.reset(
            ResidentExecutionResetOptions(self._maximum_length, self._sink_length,
                                          self.options.kv_cache,
                                          self.options.collect_confidence is not False)))
        invariant(self._session_enabled, "BACKEND_UNAVAILABLE",
                  "the HIP backend keeps every KV cache on its resident session")
        maximum_order = max([1, *g.orders])
        self._engram_depth = (g.engram_taps - 1) * maximum_order + 1
        self._engram_ring = np.zeros((len(g.sites), self._engram_depth, g.dim), np.float32)
        self._engram_valid = np.zeros((len(g.sites), self._engram_depth), np.uint8)
        self._engram_position = 0
        head = getattr(self.weights, "confidence", None)
        self._uses_resident_confidence = bool(
            self.options.collect_confidence is not False and self.session
            and self.session.resident_layers_enabled())
        self._pool = (OnlineProbePool(head, g.dim)
                      if self.options.collect_confidence is not False and head is not None
                      and not self._uses_resident_confidence else None)

    def prefill(self, tokens: Sequence[int], signal: Optional[AbortSignal] = None) -> np.ndarray:
        """runtime.ts:227-243."""
        invariant(len(tokens) > 0, "INVALID_CACT", "Cannot prefill an empty token sequence")
        invariant(self._maximum_length >= len(tokens), "CONTEXT_OVERFLOW",
                  f"Prompt has {len(tokens)} tokens but runtime holds {self._maximum_length}")
        logits = None
        for index, token in enumerate(tokens):
            logits = self.step(int(token), want_logits=index == len(tokens) - 1, signal=signal)
        invariant(logits is not None, "INVALID_CACT", "Prefill did not produce final logits")
        return logits

    def prefill_selected(self, tokens: Sequence[int], allowed_token_ids=None,
                         signal: Optional[AbortSignal] = None) -> SelectedToken:
        """runtime.ts:245-255."""
        invariant(len(tokens) > 0, "INVALID_CACT", "Cannot prefill an empty token sequence")
        for token in tokens[:-1]:
            self.step(int(token), want_logits=False, signal=signal)
        return self.step_selected(int(tokens[-1]), allowed_token_ids, signal)

    def step_selected(self, token: int, allowed_token_ids=None,
                      signal: Optional[AbortSignal] = None) -> SelectedToken:
        """runtime.ts:257-278."""
        invariant(not self._selection_active, "BACKEND_UNAVAILABLE", "Selection is already active")
        self._selection_active = True
        self._selection_request = (None if allowed_token_ids is None
                                   else np.ascontiguousarray(allowed_token_ids, np.uint32))
        self._selection_result = None
        try:
            self.step(token, signal=signal)
            result = self._selection_result
            invariant(result is not None, "BACKEND_UNAVAILABLE",
                      "Token selection did not produce a result")
            return result
        finally:
            self._selection_active = False
            self._selection_request = None
            self._selection_result = None

    def step_constrained(self, token: int, masker, grammar, output_bytes: int = 0,
                         limit: int = 65536, signal: Optional[AbortSignal] = None) -> SelectedToken:
        """One step of the constrained agent loop (tools/agent.ts:164-183):
        stepSelected over the grammar's allowed pieces.  With resident
        layers the allowed set stays on the device (the grammar mask in the
        model's mask buffer, its undecided pieces settled by clones of
        `grammar`); otherwise it is the masker's id list."""
        if not (self.session and self.session.resident_layers_enabled()):
            allowed = masker.allowed(grammar, output_bytes, limit)
            invariant(len(allowed) > 0, "GRAMMAR_DEAD_END",
                      "No token can continue the schema-constrained tool call")
            return self.step_selected(token, allowed, signal)
        count, undecided = self.session.resident.grammar_mask(masker, masker.state(grammar),
                                                              limit - output_bytes)
        masker.last_undecided = int(undecided.size)
        settled = masker.settle(grammar, undecided)
        invariant(count + len(settled) > 0, "GRAMMAR_DEAD_END",
                  "No token can continue the schema-constrained tool call")
        invariant(not self._selection_active, "BACKEND_UNAVAILABLE", "Selection is already active")
        self._selection_active = True
        self._selection_request = DeviceMaskSelection(settled)
        self._selection_result = None
        try:
            self.step(token, signal=signal)
            result = self._selection_result
            invariant(result is not None, "BACKEND_UNAVAILABLE",
                      "Token selection did not produce a result")
            return result
        finally:
            self._selection_active = False
            self._selection_request = None
            self._selection_result = None

    def step(self, token: int, want_logits: bool = True,
             signal: Optional[AbortSignal] = None) -> Optional[np.ndarray]:
        """runtime.ts:280-583."""
        _check_abort(signal)
        g = self.geometry
        invariant(self._maximum_length > 0, "INVALID_CACT", "Call runtime.reset() before decoding")
        invariant(self._position < self._maximum_length, "CONTEXT_OVERFLOW",
                  f"Position {self._position} reached runtime limit {self._maximum_length}")
        invariant(isinstance(token, (int, np.integer)) and 0 <= int(token) < g.vocab,
                  "INVALID_CACT", f"Token {token} is outside the vocabulary")
        token = int(token)
        position = self._position
        self._history.append(token)
        dimension, lanes = g.dim, g.lanes
        embedding = self.backend.row(self.weights.embedding, token)
        scaled = (embedding.astype(np.float64) * math.sqrt(dimension)).astype(np.float32)
        if self._pool is not None:
            self._pool.add(scaled)
        x = np.tile(scaled, lanes)
        lookup = self._engram_lookup()
        resident_engrams = bool(lookup is not None and self.session and
                                self.session.prepare_resident_engrams(
                                    ResidentEngramRequest(lookup[0], lookup[1],
                                                          self._engram_position)))
        keys, values = ([], []) if resident_engrams else self._engram_step(lookup)
        if resident_engrams:
            self._engram_position += 1
        resident_layers = bool(self.session and self.session.begin_resident_token(x))
        resident_logits = None
        if resident_layers:
            for layer in range(g.layers):
                _check_abort(signal)
                if self.options.on_layer:
                    self.options.on_layer({"position": position, "layer": layer,
                                           "layers": g.layers})
            self.session.forward_resident_token(ResidentTokenRequest(position, keys, values))
            if self._selection_active:
                self.session.finish_resident_token_for_selection()
            else:
                resident_logits = self.session.finish_resident_token(want_logits is not False)
        else:
            for layer in range(g.layers):
                _check_abort(signal)
                if self.options.on_layer:
                    self.options.on_layer({"position": position, "layer": layer,
                                           "layers": g.layers})
                x = self._layer(layer, position, x, keys, values)
                if self._pool is not None:
                    self._pool.add(_lane_mean(x, lanes))

        self._position += 1
        if resident_layers and self._selection_active:
            self._selection_result = self.session.select_resident_token(self._selection_request)
            return None
        if want_logits is False:
            return None
        if resident_layers:
            invariant(resident_logits is not None, "BACKEND_UNAVAILABLE",
                      "Resident logits are missing")
            return resident_logits
        final = rms_norm(_lane_mean(x, lanes), self.weights.final_norm)
        logits = self.backend.matvec(self.weights.embedding, final)
        if self._selection_active:
            token_id, lp = self.backend.select(logits, self._selection_request)
            self._selection_result = SelectedToken(token_id, lp)
            return None
        return logits

    def _layer(self, layer: int, position: int, x: np.ndarray, keys, values) -> np.ndarray:
        """One layer of a token that does not run resident (runtime.ts:382-
        551): the lane mix on the host, then the session's forward()."""
        g, w = self.geometry, self.weights
        lanes, dimension = g.lanes, g.dim
        normalized = rms_unit(x)
        phi_pre, phi_post, phi_residual = self.backend.matvec_batch([
            MatvecRequest(w.phi_pre, normalized, MatrixRowRange(layer * lanes, lanes)),
            MatvecRequest(w.phi_post, normalized, MatrixRowRange(layer * lanes, lanes)),
            MatvecRequest(w.phi_res, normalized, MatrixRowRange(layer * lanes * lanes,
                                                                lanes * lanes)),
        ])
        own = layer % lanes
        h_pre = np.array([sigmoid(float(w.a_pre[layer]) * float(phi_pre[lane])
                                  + float(w.b_pre[layer * lanes + lane])
                                  + (4.0 if lane == own else -4.0)) for lane in range(lanes)],
                         np.float32)
        xl = x.reshape(lanes, dimension).astype(np.float64)
        acc = np.zeros(dimension)
        for lane in range(lanes):
            acc = acc + float(h_pre[lane]) * xl[lane]
        update_input = acc.astype(np.float32)
        block_input = update_input
        if layer in g.sites:
            site = g.sites.index(layer)
            key, value = keys[site], values[site]
            ni, nk = rms_unit(update_input), rms_unit(key)
            dot = _seq_sum(ni.astype(np.float64) * nk.astype(np.float64))
            alpha = sigmoid(dot / math.sqrt(dimension))
            block_input = (update_input.astype(np.float64)
                           + alpha * value.astype(np.float64)).astype(np.float32)
        attention_input = rms_norm(block_input, w.norm_input[layer])
        result = self.session.forward(ResidentLayerFallbackRequest(
            layer, position, attention_input, block_input, update_input, x, phi_post,
            phi_residual))
        invariant(result.kind == "nextX", "BACKEND_UNAVAILABLE",
                  f"unexpected forward result {result.kind}")
        return result.values

    def _engram_lookup(self):
        """runtime.ts:788-818."""
        g = self.geometry
        if not g.sites:
            return None
        heads_per_order = g.engram_tables // len(g.orders)
        invariant(heads_per_order * len(g.orders) == g.engram_tables, "INVALID_CACT",
                  "Engram table count is not divisible by order count")
        indices = np.zeros(g.engram_tables, np.uint32)
        valid = np.zeros(g.engram_tables, np.uint32)
        table = 0
        for order_index, order in enumerate(g.orders):
            for head in range(heads_per_order):
                h = (ENGRAM_SEED * (order_index * heads_per_order + head + 1)) & _U32
                is_valid = True
                for offset in range(order):
                    hi = len(self._history) - 1 - offset
                    tok = self._history[hi] if hi >= 0 else 0
                    h = ((h ^ tok) * ENGRAM_PRIME) & _U32
                    if offset == order - 1:
                        is_valid = hi >= 0
                h = (h ^ (h >> 15)) & _U32
                indices[table] = h % g.engram_slots
                valid[table] = 1 if is_valid else 0
                table += 1
        return indices, valid

    def _engram_step(self, lookup):
        """runtime.ts:820-877 on the host (when the session did not prepare
        the token's engrams): rows gathered with backend.row, the key and
        value projections with one matvec_batch, the tap convolution."""
        g, w = self.geometry, self.weights
        if lookup is None:
            return [], []
        indices, valid = lookup
        requests = []
        for site in range(len(g.sites)):
            cat = np.zeros(g.engram_tables * g.engram_sub, np.float32)
            for table in range(g.engram_tables):
                if valid[table]:
                    row = table * g.engram_slots + int(indices[table])
                    cat[table * g.engram_sub:(table + 1) * g.engram_sub] = self.backend.row(
                        w.eg_tables[site], row)
            requests += [MatvecRequest(w.eg_key[site], cat), MatvecRequest(w.eg_value[site], cat)]
        projected = self.backend.matvec_batch(requests)
        maximum_order = max(g.orders)
        keys, values = [], []
        for site in range(len(g.sites)):
            keys.append(projected[2 * site])
            slot = self._engram_position % self._engram_depth
            self._engram_ring[site, slot] = projected[2 * site + 1]
            self._engram_valid[site, slot] = 1
            mixed = np.zeros(g.dim, np.float32)
            for tap in range(g.engram_taps):
                previous = self._engram_position - tap * maximum_order
                if previous < 0:
                    continue
                ps = previous % self._engram_depth
                if not self._engram_valid[site, ps]:
                    continue
                mixed = (mixed.astype(np.float64) + w.eg_taps[site, tap].astype(np.float64)
                         * self._engram_ring[site, ps].astype(np.float64)).astype(np.float32)
            values.append(mixed)
        self._engram_position += 1
        return keys, values

    def resolve_confidence(self) -> Optional[float]:
        """runtime.ts:634-639."""
        if self._uses_resident_confidence and self.session:
            return self.session.resident_confidence()
        return self.confidence()

    def confidence(self) -> Optional[float]:
        """runtime.ts:641-645."""
        if self._pool is None:
            return None
        out = self._pool.output()
        return sigmoid(float(out[0])) if out.size else None

    def dispose(self) -> None:
        if self.session:
            self.session.dispose()


class ResidentRuntime:
    """The whole-step extension of NeedleRuntime: each step (and each batch
    of prompt positions) is one launch sequence on nd_needle, with the token
    history and engram hashing on the device."""

    def __init__(self, resident: Needle2Resident, collect_confidence: bool = True,
                 kv_cache: str = "int8"):
        self.resident = resident
        self.weights = resident.weights
        self.collect_confidence = collect_confidence
        self.kv_cache = kv_cache
        self._maximum_length = 0

    @property
    def position(self) -> int:
        return self.resident.position

    @property
    def maximum_length(self) -> int:
        return self._maximum_length

    def reset(self, maximum_length: int, sink_length: int = 0) -> None:
        self.resident.reset(maximum_length, sink_length, self.kv_cache, self.collect_confidence)
        self._maximum_length = int(maximum_length)

    def prefill(self, tokens: Sequence[int]) -> np.ndarray:
        return self.resident.prefill(tokens)

    def prefill_selected(self, tokens: Sequence[int], allowed: Optional[np.ndarray] = None):
        invariant(len(tokens) > 0, "INVALID_CACT", "Cannot prefill an empty token sequence")
        if len(tokens) > 1:
            self.resident.prefill(tokens[:-1], want_logits=False)
        return self.resident.step_selected(tokens[-1], allowed)

    def step(self, token: int, want_logits: bool = True) -> Optional[np.ndarray]:
        return self.resident.step(token, want_logits)

    def step_selected(self, token: int, allowed: Optional[np.ndarray] = None):
        return self.resident.step_selected(token, allowed)

    def step_constrained(self, token: int, masker, grammar, output_bytes: int = 0,
                         limit: int = 65536):
        """One step of the constrained agent loop (tools/agent.ts:164-183)
        with the allowed set built on the device: the grammar mask over the
        model's vocabulary, its undecided pieces settled by clones of
        `grammar`, then stepSelected over that mask.  (id, log-probability);
        NeedleError INVALID_CACT "Allowed token set is empty" when nothing
        is allowed."""
        count, undecided = self.resident.grammar_mask(masker, masker.state(grammar),
                                                      limit - output_bytes)
        masker.last_undecided = int(undecided.size)
        settled = masker.settle(grammar, undecided)
        invariant(count + len(settled) > 0, "GRAMMAR_DEAD_END",
                  "No token can continue the schema-constrained tool call")
        return self.resident.step_selected_mask(token, settled)

    def resolve_confidence(self) -> Optional[float]:
        return self.resident.confidence()


@dataclass
class GenerationResult:
    """model/model.ts GenerationResult over token ids."""

    token_ids: List[int]
    token_log_probabilities: List[float]
    finish_reason: str  # "eos" | "length"
    prompt_tokens: int
    generated_tokens: int
    elapsed_ms: float
    tokens_per_second: float


def xorshift32(seed: int) -> Callable[[], float]:
    """model/model.ts:202-211: uniform [0, 1) from a 32-bit xorshift."""
    state = (seed & _U32) or 1

    def draw() -> float:
        nonlocal state
        state ^= (state << 13) & _U32
        state ^= state >> 17
        state ^= (state << 5) & _U32
        return state / 0x1_0000_0000

    return draw


def _js_max(a: float, b: float) -> float:
    """Math.max of two numbers: NaN when either is NaN."""
    if math.isnan(a) or math.isnan(b):
        return math.nan
    return a if a >= b else b


def sample(logits: np.ndarray, temperature: float, top_k: int, random: Callable[[], float]) -> int:
    """model/model.ts:213-240: argmax at temperature 0, else a draw from the
    softmax of logits / temperature over the top_k largest (all when 0).
    Edge cases as the reference evaluates them: 0 < top_k < 1 keeps no
    candidate and returns 0 (indices[-1] ?? 0); a NaN logit makes the
    maximum NaN (Math.max), so every probability is NaN, no threshold test
    passes and the last candidate is returned (the last id when top_k keeps
    every id).  With a NaN logit and fewer candidates than ids the
    reference's comparator returns NaN, which leaves its sort order to the
    engine: that case is parity unpinned."""
    if not temperature > 0:
        return argmax(logits)
    n = logits.size
    count = min(int(math.floor(top_k)), n) if top_k > 0 else n
    indices = list(range(n))
    if count < n:
        # Array.prototype.sort is stable (a NaN logit sorts as 0 here).
        indices.sort(key=lambda i: -float(logits[i]) if not math.isnan(logits[i]) else 0.0)
    indices = indices[:count]
    if count == 0:
        return 0
    scaled = logits[indices].astype(np.float64) / temperature
    maximum = -math.inf
    for v in scaled:
        maximum = _js_max(maximum, float(v))
    probabilities = np.exp(scaled - maximum)
    threshold = random() * _seq_sum(probabilities)
    for i in range(count):
        threshold -= float(probabilities[i])
        if threshold <= 0:
            return indices[i]
    return indices[count - 1]


class NeedleModel:
    """NeedleModel (model/model.ts:56-160) over token ids."""

    def __init__(self, backend: HipBackend, weights: Needle2Weights,
                 collect_confidence: bool = True):
        self.backend = backend
        self.weights = weights
        self.runtime_options = RuntimeOptions(collect_confidence=collect_confidence)
        self._resident: Optional[Needle2Resident] = None
        self._disposed = False

    @property
    def resident(self) -> Needle2Resident:
        """The nd_needle of the whole-step extension (created on first use)."""
        if self._resident is None:
            self._resident = Needle2Resident(self.backend, self.weights)
        return self._resident

    def create_runtime(self, **options) -> NeedleRuntime:
        """model/model.ts:83-86."""
        invariant(not self._disposed, "BACKEND_UNAVAILABLE", "Needle model has been disposed")
        merged = {**self.runtime_options.__dict__, **options}
        self.backend.weights = self.weights  # the backend serves this model's weights
        return NeedleRuntime(self.weights, self.backend, RuntimeOptions(**merged))

    def create_resident_runtime(self, kv_cache: str = "int8") -> ResidentRuntime:
        invariant(not self._disposed, "BACKEND_UNAVAILABLE", "Needle model has been disposed")
        return ResidentRuntime(self.resident, self.runtime_options.collect_confidence, kv_cache)

    def generate(self, prompt_ids: Sequence[int], max_new_tokens: int = 96,
                 temperature: float = 0.0, top_k: int = 0, seed: int = 0x6D2B79F5,
                 sink_tokens: int = 0, eos: Optional[int] = EOS_TOKEN_ID,
                 signal: Optional[AbortSignal] = None,
                 on_token: Optional[Callable[[dict], None]] = None) -> GenerationResult:
        """model/model.ts:88-153 with token ids for the prompt (the BOS and
        the encoded text of the reference) and without stop strings."""
        invariant(not self._disposed, "BACKEND_UNAVAILABLE", "Needle model has been disposed")
        started = time.perf_counter()
        n = max(0, int(max_new_tokens))
        ids = [int(t) for t in prompt_ids]
        g = self.weights.geometry
        maximum_length = min(g.max_length, len(ids) + n)
        if len(ids) >= maximum_length and n > 0:
            raise NeedleError("CONTEXT_OVERFLOW",
                              f"Prompt has {len(ids)} tokens and leaves no generation room in a "
                              f"{maximum_length}-token context")
        runtime = self.create_runtime(collect_confidence=False)
        try:
            runtime.reset(max(len(ids), maximum_length), sink_tokens)
            logits = runtime.prefill(ids, signal)
            random = xorshift32(seed)
            out: List[int] = []
            lps: List[float] = []
            finish = "length"
            index = 0
            while index < n and runtime.position < maximum_length:
                token = sample(logits, temperature, top_k, random)
                if eos is not None and token == eos:
                    finish = "eos"
                    break
                lp = log_softmax_at(logits, token)
                out.append(token)
                lps.append(lp)
                if on_token:
                    on_token({"id": token, "index": index, "log_probability": lp})
                if index + 1 >= n or runtime.position >= maximum_length:
                    break
                nxt = runtime.step(token, signal=signal)
                invariant(nxt is not None, "INVALID_CACT", "Decode step did not return logits")
                logits = nxt
                index += 1
        finally:
            runtime.dispose()
        elapsed = (time.perf_counter() - started) * 1000.0
        return GenerationResult(out, lps, finish, len(ids), len(out), elapsed,
                                len(out) / max(elapsed / 1000.0, 1e-9))

    def generate_resident(self, prompt_ids: Sequence[int], max_new_tokens: int = 96,
                          sink_tokens: int = 0,
                          eos: Optional[int] = EOS_TOKEN_ID) -> GenerationResult:
        """Greedy generate with every step after the prompt replayed from one
        HIP graph (nd_needle_generate): no host round trip per token."""
        invariant(not self._disposed, "BACKEND_UNAVAILABLE", "Needle model has been disposed")
        started = time.perf_counter()
        n = max(0, int(max_new_tokens))
        ids, lps = self.resident.generate(prompt_ids, n, sink_tokens, eos)
        elapsed = (time.perf_counter() - started) * 1000.0
        g = self.weights.geometry
        room = min(g.max_length, len(prompt_ids) + n) - len(prompt_ids)
        finish = "eos" if len(ids) < min(n, max(room, 0)) else "length"
        return GenerationResult([int(t) for t in ids], [float(v) for v in lps], finish,
                                len(prompt_ids), len(ids), elapsed,
                                len(ids) / max(elapsed / 1000.0, 1e-9))

    def dispose(self) -> None:
        if self._disposed:
            return
        self._disposed = True
        if self._resident is not None:
            self._resident.free()
            self._resident = None
