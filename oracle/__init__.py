"""CPU oracle for the needle.js decode hot path -- TEST INFRASTRUCTURE ONLY.

A ctypes wrapper over liboracle.so (needle_oracle.c), the C restatement of
the reference TypeScript CPU path with JavaScript number semantics.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker; the product path never does.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"

P = C.c_void_p
U32 = C.c_uint32
D = C.c_double

_SIG = {
    "or_round_ties_even": (D, [D]),
    "or_sigmoid": (D, [D]),
    "or_silu": (D, [D]),
    "or_rms_norm": (None, [P, P, U32, P]),
    "or_rms_unit": (None, [P, U32, P]),
    "or_rms_norm_slice": (None, [P, U32, U32, P]),
    "or_softmax": (None, [P, U32]),
    "or_fwht": (C.c_int, [P, U32, U32]),
    "or_sinkhorn": (None, [P, U32, U32]),
    "or_rope": (None, [P, U32, U32, U32, D]),
    "or_hadamard_mlp": (C.c_int, [P, U32, P, P, P, U32, P]),
    "or_argmax": (U32, [P, U32]),
    "or_log_softmax_at": (D, [P, U32, U32]),
    "or_select": (C.c_int, [P, U32, P, U32, C.POINTER(U32), C.POINTER(D)]),
    "or_select_mask": (C.c_int, [P, U32, P, C.POINTER(U32), C.POINTER(D)]),
    "or_matvec_i8": (C.c_int, [P, P, U32, U32, U32, P, U32, U32, U32, P]),
    "or_row_i8": (C.c_int, [P, P, U32, U32, U32, U32, P]),
    "or_f16_to_f32": (C.c_float, [C.c_uint16]),
    "or_cq_prepare": (C.c_int, [P, U32, U32, P]),
    "or_cq_matvec": (C.c_int, [P, P, P, U32, U32, U32, U32, P, U32, U32, U32, P]),
    "or_cq_row": (C.c_int, [P, P, P, U32, U32, U32, U32, U32, P]),
    "or_kv_quantize": (None, [P, U32, P, P]),
    "or_kv_create": (P, [U32, U32, U32, U32, U32, U32, C.c_int]),
    "or_kv_destroy": (None, [P]),
    "or_kv_alloc": (U32, [P]),
    "or_kv_slot": (U32, [P, U32]),
    "or_kv_store": (C.c_int, [P, U32, U32, P, P]),
    "or_kv_export": (None, [P, U32, U32, P, P, P, P]),
    "or_kv_capture": (C.c_int, [P, U32, U32]),
    "or_kv_export_raw": (C.c_int, [P, U32, U32, U32, U32, P, P]),
    "or_attention": (C.c_int, [P, U32, U32, P, U32, P]),
}

_LIB = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIBRARY.exists():
            build()
        handle = C.CDLL(str(LIBRARY))
        for name, (res, args) in _SIG.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return a.ctypes.data


class OracleError(ValueError):
    pass


def _ok(status):
    if status != 0:
        raise OracleError(f"oracle rejected the arguments (status {status})")


# ------------------------------------------------------------- primitives

def round_ties_even(x: float) -> float:
    return lib().or_round_ties_even(float(x))


def sigmoid(x: float) -> float:
    return lib().or_sigmoid(float(x))


def rms_norm(x, scale):
    x, scale = _f32(x), _f32(scale)
    out = np.empty_like(x)
    lib().or_rms_norm(_p(x), _p(scale), x.size, _p(out))
    return out


def rms_unit(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_rms_unit(_p(x), x.size, _p(out))
    return out


def softmax(x):
    x = _f32(x).copy()
    lib().or_softmax(_p(x), x.size)
    return x


def fwht(x):
    x = _f32(x).copy()
    _ok(lib().or_fwht(_p(x), 0, x.size))
    return x


def sinkhorn(logits, size: int, iterations: int = 20):
    x = _f32(logits).copy()
    lib().or_sinkhorn(_p(x), size, iterations)
    return x


def rope(vec, heads: int, head_dim: int, position: int, theta: float):
    x = _f32(vec).copy()
    lib().or_rope(_p(x), heads, head_dim, position, float(theta))
    return x


def hadamard_mlp(x, d1, d2, d3, hdim: int):
    x, d1, d2, d3 = _f32(x), _f32(d1), _f32(d2), _f32(d3)
    out = np.empty(x.size, dtype=np.float32)
    _ok(lib().or_hadamard_mlp(_p(x), x.size, _p(d1), _p(d2), _p(d3), hdim, _p(out)))
    return out


def argmax(values) -> int:
    v = _f32(values)
    return int(lib().or_argmax(_p(v), v.size))


def log_softmax_at(logits, token: int) -> float:
    v = _f32(logits)
    return float(lib().or_log_softmax_at(_p(v), v.size, token))


def select(logits, allowed=None):
    """selectToken: (id, log_probability); raises OracleError like invariant()."""
    v = _f32(logits)
    out_id, out_lp = U32(), D()
    if allowed is None:
        st = lib().or_select(_p(v), v.size, None, 0, C.byref(out_id), C.byref(out_lp))
    else:
        a = np.ascontiguousarray(allowed, dtype=np.uint32)
        if a.size == 0:
            raise OracleError("Allowed token set is empty")
        st = lib().or_select(_p(v), v.size, _p(a), a.size, C.byref(out_id), C.byref(out_lp))
    _ok(st)
    return int(out_id.value), float(out_lp.value)


def select_mask(logits, mask):
    v = _f32(logits)
    m = np.ascontiguousarray(mask, dtype=np.uint32)
    out_id, out_lp = U32(), D()
    _ok(lib().or_select_mask(_p(v), v.size, _p(m), C.byref(out_id), C.byref(out_lp)))
    return int(out_id.value), float(out_lp.value)


def matvec_i8(w, scales, g: int, x, row_start: int = 0, row_count=None):
    w = np.ascontiguousarray(w, dtype=np.int8)
    scales = _f32(scales)
    x = _f32(x)
    n, k = w.shape
    batch = 1 if x.ndim == 1 else x.shape[0]
    rc = n - row_start if row_count is None else row_count
    y = np.empty((batch, rc), dtype=np.float32)
    _ok(lib().or_matvec_i8(_p(w), _p(scales), n, k, g, _p(x), batch, row_start, rc, _p(y)))
    return y[0] if x.ndim == 1 else y


def f16_to_f32(bits: int) -> float:
    """float16ToNumber (fp16.ts:5-32) of one binary16 bit pattern."""
    return float(lib().or_f16_to_f32(int(bits) & 0xFFFF))


def cq_prepare(x, g: int):
    """prepareCqActivation (cq.ts:30-46): padded, per-group FWHT / sqrt(g)."""
    x = _f32(x).reshape(-1)
    kpad = (x.size + g - 1) // g * g
    out = np.empty(kpad, dtype=np.float32)
    _ok(lib().or_cq_prepare(_p(x), x.size, g, _p(out)))
    return out


def _cq_args(packed, norms, codebook):
    return (np.ascontiguousarray(packed, dtype=np.uint8),
            np.ascontiguousarray(norms, dtype=np.uint16), _f32(codebook))


def cq_matvec(packed, norms, codebook, k: int, g: int, bits: int, x, row_start: int = 0,
              row_count=None):
    """cqMatvec (cq.ts:107-240) over a packed CQ matrix [n][row_bytes] with
    binary16 norms [n][groups] and the archive's 28-float codebook."""
    packed, norms, codebook = _cq_args(packed, norms, codebook)
    x = _f32(x)
    n = packed.shape[0]
    batch = 1 if x.ndim == 1 else x.shape[0]
    rc = n - row_start if row_count is None else row_count
    y = np.empty((batch, rc), dtype=np.float32)
    _ok(lib().or_cq_matvec(_p(packed), _p(norms), _p(codebook), n, k, g, bits, _p(x), batch,
                           row_start, rc, _p(y)))
    return y[0] if x.ndim == 1 else y


def cq_row(packed, norms, codebook, k: int, g: int, bits: int, row: int):
    """dequantizeCqRow (cq.ts:243-295)."""
    packed, norms, codebook = _cq_args(packed, norms, codebook)
    out = np.empty(k, dtype=np.float32)
    _ok(lib().or_cq_row(_p(packed), _p(norms), _p(codebook), packed.shape[0], k, g, bits, row,
                        _p(out)))
    return out


def row_i8(w, scales, g: int, row: int):
    w = np.ascontiguousarray(w, dtype=np.int8)
    scales = _f32(scales)
    out = np.empty(w.shape[1], dtype=np.float32)
    _ok(lib().or_row_i8(_p(w), _p(scales), w.shape[0], w.shape[1], g, row, _p(out)))
    return out


def kv_quantize(x):
    x = _f32(x)
    codes = np.empty(x.size, dtype=np.int8)
    scale = np.empty(1, dtype=np.float32)
    lib().or_kv_quantize(_p(x), x.size, _p(codes), _p(scale))
    return codes, float(scale[0])


class KvCache:
    """NeedleRuntime's KV cache (int8 or float32) and #attention."""

    def __init__(self, layers, kv_heads, max_length, sink=0, window=0, kv_cache="int8",
                 head_dim=64):
        self.layers, self.kv_heads, self.head_dim = layers, kv_heads, head_dim
        self.float_mode = kv_cache == "float32"
        self.max_length = max_length
        self.h = lib().or_kv_create(layers, kv_heads, head_dim, max_length, sink, window,
                                    1 if self.float_mode else 0)
        self.alloc = int(lib().or_kv_alloc(self.h))

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_kv_destroy(self.h)
            self.h = None

    def slot(self, position: int) -> int:
        return int(lib().or_kv_slot(self.h, position))

    def store(self, layer, position, k, v):
        k, v = _f32(k).reshape(-1), _f32(v).reshape(-1)
        per = self.kv_heads * self.head_dim
        for i in range(k.size // per):
            kk = np.ascontiguousarray(k[i * per:(i + 1) * per])
            vv = np.ascontiguousarray(v[i * per:(i + 1) * per])
            _ok(lib().or_kv_store(self.h, layer, position + i, _p(kk), _p(vv)))

    def capture(self, from_position: int = 0, count: int | None = None) -> None:
        """Keep the K/V vectors stored from now on at positions [from_position,
        +count) (their values before quantization; count defaults to the rest
        of the cache)."""
        n = int(self.max_length) - from_position if count is None else count
        _ok(lib().or_kv_capture(self.h, from_position, n))

    def read_raw(self, layer, head, from_position, count):
        """Captured (k, v) vectors of positions [from_position, +count), each
        [count][head_dim] float32."""
        k = np.empty((count, self.head_dim), np.float32)
        v = np.empty((count, self.head_dim), np.float32)
        _ok(lib().or_kv_export_raw(self.h, layer, head, from_position, count, _p(k), _p(v)))
        return k, v

    def read(self, layer, head):
        """(k, v, k scales, v scales): int8 codes, or float32 rows in float mode."""
        dt = np.float32 if self.float_mode else np.int8
        kc = np.zeros((self.alloc, self.head_dim), dtype=dt)
        vc = np.zeros((self.alloc, self.head_dim), dtype=dt)
        ks = np.empty(self.alloc, dtype=np.float32)
        vs = np.empty(self.alloc, dtype=np.float32)
        lib().or_kv_export(self.h, layer, head, _p(kc), _p(vc), _p(ks), _p(vs))
        return kc, vc, ks, vs

    def attention(self, layer, position, q):
        q = _f32(q).reshape(-1)
        out = np.empty_like(q)
        _ok(lib().or_attention(self.h, layer, position, _p(q), q.size // self.head_dim, _p(out)))
        return out


# ------------------------------------------------------ synthetic decoder

_SIG_MODEL = {
    "or_splitmix64_at": (C.c_uint64, [C.c_uint64, C.c_uint64]),
    "or_gen_mask": (None, [C.c_uint64, U32, U32, P]),
    "or_gen_kv_row": (None, [C.c_uint64, C.c_uint64, U32, C.c_float, C.c_float, P, P]),
    "or_kv_fill_synthetic": (None, [P, C.c_uint64, C.c_uint64, U32, C.c_float, C.c_float]),
    "or_synth_step": (C.c_int, [P, P, U32, U32, P, P]),
    "or_synth_decode_batch": (C.c_int, [P, P, P, P, U32, U32, C.c_uint64, U32, P, P, U32, P,
                                        U32, P]),
    "or_synth_prefill": (C.c_int, [P, P, P, U32, U32, P, U32]),
}


def _model_lib():
    h = lib()
    if not getattr(h, "_model_bound", False):
        for name, (res, args) in _SIG_MODEL.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        h._model_bound = True
    return h


class _OrMat(C.Structure):
    _fields_ = [("w", P), ("s", P), ("n", U32), ("k", U32)]


class _OrSynth(C.Structure):
    _fields_ = [("layers", U32), ("dim", U32), ("heads", U32), ("kv_heads", U32),
                ("head_dim", U32), ("ffn", U32), ("vocab", U32), ("rope_theta", D),
                ("embedding", _OrMat), ("wq", C.POINTER(_OrMat)), ("wk", C.POINTER(_OrMat)),
                ("wv", C.POINTER(_OrMat)), ("wo", C.POINTER(_OrMat)), ("wup", C.POINTER(_OrMat)),
                ("wdown", C.POINTER(_OrMat)), ("attn_norm", P), ("ffn_norm", P), ("q_norm", P),
                ("k_norm", P), ("final_norm", P)]


def splitmix64_at(seed: int, index: int) -> int:
    return int(_model_lib().or_splitmix64_at(seed, index))


def gen_mask(seed: int, vocab: int, threshold24: int):
    mask = np.zeros((vocab + 31) // 32, dtype=np.uint32)
    _model_lib().or_gen_mask(seed, vocab, threshold24, _p(mask))
    return mask


def gen_kv_row(seed: int, index: int, n: int, lo: float, hi: float):
    codes = np.empty(n, np.int8)
    scale = np.empty(1, np.float32)
    _model_lib().or_gen_kv_row(seed, index, n, lo, hi, _p(codes), _p(scale))
    return codes, float(scale[0])


def kv_fill_synthetic(cache: "KvCache", seed_k: int, seed_v: int, length: int, lo: float,
                      hi: float) -> None:
    _model_lib().or_kv_fill_synthetic(cache.h, seed_k, seed_v, length, lo, hi)


class SynthDecoder:
    """The oracle's synthetic decoder over a DecoderWeights-like object."""

    def __init__(self, weights):
        g = weights.geometry
        self.geometry = g
        self._keep = []

        def om(m):
            c = np.ascontiguousarray(m.codes, np.int8)
            s = np.ascontiguousarray(m.scales, np.float32)
            self._keep += [c, s]
            return _OrMat(_p(c), _p(s), c.shape[0], c.shape[1])

        def arr(ms):
            a = (_OrMat * len(ms))(*[om(m) for m in ms])
            self._keep.append(a)
            return a

        def vec(v):
            v = np.ascontiguousarray(v, np.float32)
            self._keep.append(v)
            return _p(v)

        st = _OrSynth()
        st.layers, st.dim, st.heads, st.kv_heads = g.layers, g.dim, g.heads, g.kv_heads
        st.head_dim, st.ffn, st.vocab, st.rope_theta = g.head_dim, g.ffn, g.vocab, float(np.float32(g.rope_theta))
        st.embedding = om(weights.embedding)
        for name in ("wq", "wk", "wv", "wo", "wup", "wdown"):
            setattr(st, name, C.cast(arr(getattr(weights, name)), C.POINTER(_OrMat)))
        for name in ("attn_norm", "ffn_norm", "q_norm", "k_norm", "final_norm"):
            setattr(st, name, vec(getattr(weights, name)))
        self.struct = st
        _model_lib()

    def new_cache(self, max_length: int) -> KvCache:
        g = self.geometry
        return KvCache(g.layers, g.kv_heads, max_length)

    def step(self, cache: KvCache, token: int, position: int, want_hidden: bool = False):
        logits = np.empty(self.geometry.vocab, np.float32)
        hidden = np.empty(self.geometry.dim, np.float32) if want_hidden else None
        _ok(_model_lib().or_synth_step(C.byref(self.struct), cache.h, token, position, _p(logits),
                                       _p(hidden) if want_hidden else None))
        return (logits, hidden) if want_hidden else logits

    def prefill(self, cache: KvCache, tokens, position0: int = 0, threads: int = 1):
        """NeedleRuntime.prefill: the logits of the last of `tokens` run at
        positions [position0, +len(tokens)), bit-identical to that many
        step() calls (evaluated layer by layer on `threads` threads)."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.geometry.vocab, np.float32)
        _ok(_model_lib().or_synth_prefill(C.byref(self.struct), cache.h, _p(tokens), tokens.size,
                                          position0, _p(logits), threads))
        return logits

    def decode_batch(self, caches, tokens, start, steps: int, mask_seed: int, threshold24: int,
                     threads: int = 1, check_steps=None):
        """(ids [steps][b], log-probabilities [steps][b]), plus the logits
        [len(check_steps)][b][vocab] of the listed steps when check_steps is
        given."""
        b = len(caches)
        ptrs = (P * b)(*[c.h for c in caches])
        tokens = np.ascontiguousarray(tokens, np.uint32)
        start = np.ascontiguousarray(start, np.uint32)
        ids = np.empty((steps, b), np.uint32)
        lps = np.empty((steps, b), np.float64)
        checks = np.ascontiguousarray(check_steps if check_steps is not None else [], np.uint32)
        check_logits = np.empty((checks.size, b, self.geometry.vocab), np.float32)
        _ok(_model_lib().or_synth_decode_batch(
            C.byref(self.struct), ptrs, _p(tokens), _p(start), b, steps, mask_seed, threshold24,
            _p(ids), _p(lps), threads, _p(checks) if checks.size else None, checks.size,
            _p(check_logits) if checks.size else None))
        if check_steps is None:
            return ids, lps
        return ids, lps, check_logits


# ------------------------------------------------------------------ Needle 2

class _N2Mat(C.Structure):
    _fields_ = [("w", P), ("s", P), ("n", U32), ("k", U32), ("bits", U32), ("g", U32),
                ("packed", P), ("norms", P), ("codebook", P)]


class _N2Model(C.Structure):
    _fields_ = [
        ("vocab", U32), ("dim", U32), ("heads", U32), ("kv_heads", U32), ("layers", U32),
        ("head_dim", U32), ("max_length", U32), ("hadamard", U32), ("lanes", U32),
        ("engram_slots", U32), ("engram_sub", U32), ("engram_tables", U32), ("engram_taps", U32),
        ("n_orders", U32), ("n_sites", U32), ("orders", U32 * 4), ("sites", U32 * 4),
        ("rope_theta", D), ("kv_window", U32), ("embedding", _N2Mat),
        ("wq", C.POINTER(_N2Mat)), ("wk", C.POINTER(_N2Mat)), ("wv", C.POINTER(_N2Mat)),
        ("wgate", C.POINTER(_N2Mat)), ("wo", C.POINTER(_N2Mat)),
        ("norm_input", P), ("query_norm", P), ("key_norm", P), ("post_attn_norm", P),
        ("attention_gate", P), ("pre_hadamard_norm", P), ("d1", P), ("d2", P), ("d3", P),
        ("phi_pre", _N2Mat), ("phi_post", _N2Mat), ("phi_res", _N2Mat),
        ("a_pre", P), ("a_post", P), ("a_res", P), ("b_pre", P), ("b_post", P), ("b_res", P),
        ("eg_tables", C.POINTER(_N2Mat)), ("eg_key", C.POINTER(_N2Mat)),
        ("eg_value", C.POINTER(_N2Mat)), ("eg_taps", P), ("final_norm", P),
        ("probes", P), ("probe_count", U32), ("probe_out", U32), ("probe_projection", P),
        ("probe_bias", P),
    ]


_SIG_N2 = {
    "or_n2_create": (P, [P, U32, U32]),
    "or_n2_create_kv": (P, [P, U32, U32, C.c_int]),
    "or_n2_destroy": (None, [P]),
    "or_n2_kv": (P, [P]),
    "or_n2_step": (C.c_int, [P, U32, P]),
    "or_n2_confidence": (C.c_int, [P, C.POINTER(D)]),
    "or_n2_record_cells": (None, [P, P, U32]),
    "or_n2_recorded_cells": (U32, [P]),
}


def _n2_lib():
    h = lib()
    if not getattr(h, "_n2_bound", False):
        for name, (res, args) in _SIG_N2.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        h._n2_bound = True
    return h


class Needle2:
    """The oracle's Needle 2 model (NeedleRuntime.step on the CPU path)."""

    def __init__(self, weights):
        g = weights.geometry
        self.geometry = g
        self._keep = []

        def om(m):
            if getattr(m, "kind", None) == "cq":  # the archive's Cactus-Quant matrix
                cb = np.zeros(28, np.float32)  # CQ2 [0, 4), CQ3 [4, 12), CQ4 [12, 28)
                for bits, off in ((2, 0), (3, 4), (4, 12)):
                    if bits in m.codebooks:
                        cb[off:off + (1 << bits)] = m.codebooks[bits]
                packed = np.ascontiguousarray(m.packed, np.uint8)
                norms = np.ascontiguousarray(m.norms, np.uint16)
                self._keep += [cb, packed, norms]
                return _N2Mat(None, None, m.output_size, m.input_size, m.bits, m.group_size,
                              _p(packed), _p(norms), _p(cb))
            c = np.ascontiguousarray(m.codes, np.int8)
            s = np.ascontiguousarray(m.scales, np.float32)
            self._keep += [c, s]
            return _N2Mat(_p(c), _p(s), c.shape[0], c.shape[1], 0, 0, None, None, None)

        def arr(ms):
            a = (_N2Mat * max(1, len(ms)))(*[om(m) for m in ms])
            self._keep.append(a)
            return C.cast(a, C.POINTER(_N2Mat))

        def vec(v):
            v = np.ascontiguousarray(v, np.float32)
            self._keep.append(v)
            return _p(v)

        st = _N2Model()
        for f in ("vocab", "dim", "heads", "kv_heads", "layers", "head_dim", "max_length",
                  "hadamard", "lanes", "engram_slots", "engram_sub", "engram_tables",
                  "engram_taps", "kv_window"):
            setattr(st, f, getattr(g, f))
        st.n_orders, st.n_sites = len(g.orders), len(g.sites)
        for i, o in enumerate(g.orders):
            st.orders[i] = o
        for i, s in enumerate(g.sites):
            st.sites[i] = s
        st.rope_theta = float(np.float32(g.rope_theta))
        st.embedding = om(weights.embedding)
        for name in ("wq", "wk", "wv", "wgate", "wo", "eg_tables", "eg_key", "eg_value"):
            setattr(st, name, arr(getattr(weights, name)))
        for name in ("phi_pre", "phi_post", "phi_res"):
            setattr(st, name, om(getattr(weights, name)))
        for name in ("norm_input", "query_norm", "key_norm", "post_attn_norm", "attention_gate",
                     "pre_hadamard_norm", "d1", "d2", "d3", "a_pre", "a_post", "a_res", "b_pre",
                     "b_post", "b_res", "eg_taps", "final_norm"):
            setattr(st, name, vec(getattr(weights, name)))
        head = getattr(weights, "confidence", None)
        if head is not None:
            st.probes = vec(head.probes)
            st.probe_count = head.probe_count
            st.probe_out = head.output_size
            st.probe_projection = vec(head.projection)
            st.probe_bias = vec(head.bias)
        self.struct = st
        _n2_lib()

    def runtime(self, max_length: int, sink: int = 0, kv_cache: str = "int8") -> "Needle2Runtime":
        return Needle2Runtime(self, max_length, sink, kv_cache)


class Needle2Runtime:
    """One sequence: reset(maximumLength, sinkLength) then step()."""

    def __init__(self, model: Needle2, max_length: int, sink: int = 0, kv_cache: str = "int8"):
        self.model = model
        self.float_kv = kv_cache == "float32"
        self.h = _n2_lib().or_n2_create_kv(C.byref(model.struct), max_length, sink,
                                           1 if self.float_kv else 0)
        if not self.h:
            raise OracleError("bad runtime length")

    def __del__(self):
        if getattr(self, "h", None):
            _n2_lib().or_n2_destroy(self.h)
            self.h = None

    def step(self, token: int, want_logits: bool = True):
        logits = np.empty(self.model.geometry.vocab, np.float32) if want_logits else None
        _ok(_n2_lib().or_n2_step(self.h, token, _p(logits) if want_logits else None))
        return logits

    def confidence(self) -> float:
        """resolveConfidence on the CPU path (runtime.ts:634-645)."""
        out = D()
        _ok(_n2_lib().or_n2_confidence(self.h, C.byref(out)))
        return out.value

    def record_cells(self, cap: int) -> np.ndarray:
        """Buffer that receives the next `cap` pooled cells ([cap][dim])."""
        self._cells = np.zeros((cap, self.model.geometry.dim), np.float32)
        _n2_lib().or_n2_record_cells(self.h, _p(self._cells), cap)
        return self._cells

    def recorded_cells(self) -> int:
        return int(_n2_lib().or_n2_recorded_cells(self.h))

    def _cache(self, fn):
        cache = KvCache.__new__(KvCache)
        g = self.model.geometry
        cache.layers, cache.kv_heads, cache.head_dim = g.layers, g.kv_heads, g.head_dim
        cache.float_mode = self.float_kv
        cache.h = _n2_lib().or_n2_kv(self.h)
        cache.alloc = int(lib().or_kv_alloc(cache.h))
        try:
            return fn(cache)
        finally:
            cache.h = None  # owned by the runtime

    def kv_read(self, layer: int, head: int):
        return self._cache(lambda c: c.read(layer, head))

    def capture_kv(self, from_position: int, count: int) -> None:
        """Keep the K/V vectors of positions [from_position, +count) before
        quantization (see KvCache.capture)."""
        self._cache(lambda c: c.capture(from_position, count))

    def kv_read_raw(self, layer: int, head: int, from_position: int, count: int):
        return self._cache(lambda c: c.read_raw(layer, head, from_position, count))
