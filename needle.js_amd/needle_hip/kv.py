"""Device-resident int8 KV cache and decode attention (host wrapper).

The cache is NeedleRuntime's int8 KV cache (model/runtime.ts:150-205,
659-786) living in HBM: codes [layers][kv_heads][alloc][64] and one fp32
scale per (layer, head, slot).  `store` is #storeKV, `attention` is
#attention; both run as HIP kernels in libneedle_hip.so.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import lib as L
from .errors import invariant


class HipKvCache:
    def __init__(self, backend, layers: int, kv_heads: int, max_length: int, sink: int = 0,
                 window: int = 0, kv_cache: str = "int8", head_dim: int = 64):
        invariant(kv_cache in ("int8", "float32"), "INVALID_CACT", f"unknown kvCache {kv_cache}")
        self.backend = backend
        self.lib = backend.lib
        self.layers = layers
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self.max_length = max_length
        self.mode = L.ND_KV_INT8 if kv_cache == "int8" else L.ND_KV_FLOAT32
        handle = C.c_void_p()
        backend._check(self.lib.nd_kv_create(backend.ctx, layers, kv_heads, head_dim, max_length,
                                             sink, window, self.mode, C.byref(handle)),
                       "nd_kv_create")
        self.handle = handle
        alloc = C.c_uint32()
        self.lib.nd_kv_info(handle, C.byref(alloc), None, None, None, None)
        self.alloc = int(alloc.value)
        self.sink = min(sink, max_length)
        self.window = window

    def store(self, layer: int, position: int, k: np.ndarray, v: np.ndarray) -> None:
        """Quantize and append k, v ([count][kv_heads][64] or [kv_heads*64])."""
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        per = self.kv_heads * self.head_dim
        invariant(k.size % per == 0 and k.size == v.size, "INVALID_CACT",
                  "key/value vectors do not match the KV geometry")
        count = k.size // per
        self.backend._check(self.lib.nd_kv_store(self.backend.ctx, self.handle, layer, position,
                                                 count, L.ptr(k), L.ptr(v)), "nd_kv_store")

    def attention(self, layer: int, position: int, q: np.ndarray) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
        invariant(q.size % self.head_dim == 0, "INVALID_CACT", "query size is not a head multiple")
        q_heads = q.size // self.head_dim
        out = np.empty(q.size, dtype=np.float32)
        self.backend._check(self.lib.nd_attention(self.backend.ctx, self.handle, layer, position,
                                                  L.ptr(q), q_heads, L.ptr(out)), "nd_attention")
        return out

    def read(self, layer: int, head: int):
        """(k_codes, v_codes, k_scales, v_scales) of one (layer, head)."""
        dt = np.int8 if self.mode == L.ND_KV_INT8 else np.float32
        kc = np.empty((self.alloc, self.head_dim), dtype=dt)
        vc = np.empty((self.alloc, self.head_dim), dtype=dt)
        ks = np.empty(self.alloc, dtype=np.float32)
        vs = np.empty(self.alloc, dtype=np.float32)
        self.backend._check(self.lib.nd_kv_read(self.backend.ctx, self.handle, layer, head,
                                                L.ptr(kc), L.ptr(vc), L.ptr(ks), L.ptr(vs)),
                            "nd_kv_read")
        return kc, vc, ks, vs

    def clear(self) -> None:
        self.backend._check(self.lib.nd_kv_clear(self.backend.ctx, self.handle), "nd_kv_clear")

    def free(self) -> None:
        if self.handle is not None and self.backend.ctx is not None:
            self.lib.nd_kv_free(self.backend.ctx, self.handle)
        self.handle = None
