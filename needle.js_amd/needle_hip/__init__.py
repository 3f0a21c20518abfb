"""needle_hip: MI355X (gfx950) decode backend for needle.js.

Host-side mirror of needle.js's backend contract (backends/backend.ts) over
the C ABI of libneedle_hip.so (include/needle_hip.h).  There is no CPU
fallback: constructing HipBackend without the library or a gfx950 device
raises NeedleError("BACKEND_UNAVAILABLE").
"""

from .backend import HipBackend, Int8Matrix, MatrixRowRange, MatvecRequest
from .cact import (CactArchive, CqMatrix, pack_codes, parse_cact, parse_cact_weights,
                   write_cact)
from .errors import NeedleError, invariant
from .kv import HipKvCache
from .needle2 import Needle2Geometry, Needle2Weights, weights_from_cact
from .runtime import (AbortSignal, GenerationResult, HipNeedleSession, Needle2Resident,
                      NeedleModel, NeedleRuntime, ResidentRuntime, RuntimeOptions)

__all__ = [
    "AbortSignal",
    "CactArchive",
    "CqMatrix",
    "GenerationResult",
    "HipBackend",
    "HipNeedleSession",
    "Needle2Resident",
    "Needle2Geometry",
    "Needle2Weights",
    "weights_from_cact",
    "NeedleModel",
    "NeedleRuntime",
    "ResidentRuntime",
    "RuntimeOptions",
    "HipKvCache",
    "Int8Matrix",
    "MatrixRowRange",
    "MatvecRequest",
    "NeedleError",
    "invariant",
    "pack_codes",
    "parse_cact",
    "parse_cact_weights",
    "write_cact",
]
