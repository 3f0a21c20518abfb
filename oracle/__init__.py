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
    "or_kv_quantize": (None, [P, U32, P, P]),
    "or_kv_create": (P, [U32, U32, U32, U32, U32, U32, C.c_int]),
    "or_kv_destroy": (None, [P]),
    "or_kv_alloc": (U32, [P]),
    "or_kv_slot": (U32, [P, U32]),
    "or_kv_store": (C.c_int, [P, U32, U32, P, P]),
    "or_kv_export": (None, [P, U32, U32, P, P, P, P]),
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

    def read(self, layer, head):
        kc = np.zeros((self.alloc, self.head_dim), dtype=np.int8)
        vc = np.zeros((self.alloc, self.head_dim), dtype=np.int8)
        ks = np.empty(self.alloc, dtype=np.float32)
        vs = np.empty(self.alloc, dtype=np.float32)
        lib().or_kv_export(self.h, layer, head, _p(kc), _p(vc), _p(ks), _p(vs))
        return kc, vc, ks, vs

    def attention(self, layer, position, q):
        q = _f32(q).reshape(-1)
        out = np.empty_like(q)
        _ok(lib().or_attention(self.h, layer, position, _p(q), q.size // self.head_dim, _p(out)))
        return out
