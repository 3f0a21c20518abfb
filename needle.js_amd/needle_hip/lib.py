"""ctypes binding of libneedle_hip.so (declarations in include/needle_hip.h).

This is the host-side equivalent of the bun:ffi `dlopen` a TypeScript host
would use: every entry point is a plain C function over pointers and sizes.
Loading fails loudly -- there is no CPU fallback behind this module.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

from .errors import NeedleError

ND_OK = 0
ND_ERR_INVALID = 1
ND_ERR_BACKEND = 2
ND_ERR_OVERFLOW = 3
ND_ERR_NOMEM = 4
ND_ERR_UNSUPPORTED = 5
ND_KV_INT8 = 0
ND_KV_FLOAT32 = 1

_STATUS_CODE = {
    ND_ERR_INVALID: "INVALID_CACT",
    ND_ERR_OVERFLOW: "CONTEXT_OVERFLOW",
    ND_ERR_BACKEND: "BACKEND_UNAVAILABLE",
    ND_ERR_NOMEM: "BACKEND_UNAVAILABLE",
    ND_ERR_UNSUPPORTED: "UNSUPPORTED_CACT",
}

PACKAGE_ROOT = Path(__file__).resolve().parent.parent
DEFAULT_LIBRARY = PACKAGE_ROOT / "libneedle_hip.so"

P = C.c_void_p
U32 = C.c_uint32
I32 = C.c_int32
PP = C.POINTER(C.c_void_p)
PU32 = C.POINTER(C.c_uint32)
PF = C.POINTER(C.c_float)


class MatvecJob(C.Structure):
    _fields_ = [
        ("mat", P),
        ("x", P),
        ("row_start", U32),
        ("row_count", U32),
        ("y", P),
    ]


# name -> (restype, argtypes).  Kept in the order of include/needle_hip.h.
SIGNATURES = {
    "nd_create": (I32, [I32, PP]),
    "nd_destroy": (I32, [P]),
    "nd_last_error": (C.c_char_p, [P]),
    "nd_sync": (I32, [P]),
    "nd_stream": (P, [P]),
    "nd_test_xcd_local": (I32, [P, I32, PU32]),
    "nd_mat_upload_i8": (I32, [P, P, P, U32, U32, U32, PP]),
    "nd_mat_upload_i8_d": (I32, [P, P, P, U32, U32, U32, PP]),
    "nd_mat_free": (I32, [P, P]),
    "nd_mat_upload_cq": (I32, [P, P, P, P, U32, U32, U32, U32, PP]),
    "nd_mat_cq_info": (I32, [P, PU32, PU32, PU32]),
    "nd_mat_info": (I32, [P, PP, PP, PU32, PU32, PU32]),
    "nd_matvec": (I32, [P, P, P, U32, U32, U32, P]),
    "nd_matvec_d": (I32, [P, P, P, U32, U32, U32, P, P]),
    "nd_matvec_batch": (I32, [P, C.POINTER(MatvecJob), U32]),
    "nd_row": (I32, [P, P, U32, P]),
    "nd_row_d": (I32, [P, P, U32, P, P]),
    "nd_stream_read_d": (I32, [P, P, C.c_uint64, U32, P, P]),
    "nd_matvec_stamped_d": (I32, [P, P, P, U32, U32, P, P, U32, PU32, P]),
    "nd_kv_create": (I32, [P, U32, U32, U32, U32, U32, U32, U32, PP]),
    "nd_kv_free": (I32, [P, P]),
    "nd_kv_clear": (I32, [P, P]),
    "nd_kv_info": (I32, [P, PU32, PP, PP, PP, PP]),
    "nd_kv_store": (I32, [P, P, U32, U32, U32, P, P]),
    "nd_kv_store_d": (I32, [P, P, U32, U32, U32, P, P, P]),
    "nd_kv_read": (I32, [P, P, U32, U32, P, P, P, P]),
    "nd_attention": (I32, [P, P, U32, U32, P, U32, P]),
    "nd_attention_d": (I32, [P, P, U32, U32, P, U32, P, P]),
    "nd_attention_stamped_d": (I32, [P, P, U32, U32, P, U32, P, P, U32, PU32, P]),
    "nd_attention_static_d": (I32, [P, P, U32, U32, P, U32, P, P]),
    "nd_select": (I32, [P, P, U32, P, U32, PU32, C.POINTER(C.c_double)]),
    "nd_select_mask_d": (I32, [P, P, U32, U32, P, P, P, P]),
    "nd_matmul": (I32, [P, P, P, U32, P]),
    "nd_matmul_d": (I32, [P, P, P, U32, P, U32, P]),
    "nd_decoder_create": (I32, [P, P, PP]),
    "nd_decoder_free": (I32, [P, P]),
    "nd_batch_create": (I32, [P, P, U32, U32, PP]),
    "nd_batch_free": (I32, [P, P]),
    "nd_batch_kv": (P, [P]),
    "nd_batch_fill_synthetic": (I32, [P, P, U32, C.c_uint64, C.c_uint64, U32, U32, C.c_float,
                                      C.c_float]),
    "nd_batch_set_state": (I32, [P, P, P, P, U32]),
    "nd_batch_step": (I32, [P, P, U32, U32, C.c_uint64, U32, P]),
    "nd_batch_read": (I32, [P, P, P, P, P, P]),
    "nd_batch_read_projections": (I32, [P, P, P]),
    "nd_batch_history": (I32, [P, P, U32, U32, P, P]),
    "nd_prefill_create": (I32, [P, P, U32, U32, PP]),
    "nd_prefill_free": (I32, [P, P]),
    "nd_prefill_tokens": (I32, [P, P, P, P, U32, U32, P]),
    "nd_prefill_set_tokens": (I32, [P, P, P, U32, U32]),
    "nd_prefill_run_d": (I32, [P, P, P, P]),
    "nd_prefill_logits": (I32, [P, P, P]),
    "nd_prefill_phase_ms": (I32, [P, P, P, P]),
    "nd_prefill_read_projections": (I32, [P, P, P]),
    "nd_needle_create": (I32, [P, P, PP]),
    "nd_needle_free": (I32, [P, P]),
    "nd_needle_reset": (I32, [P, P, U32, U32, U32, U32]),
    "nd_needle_kv": (P, [P]),
    "nd_needle_position": (U32, [P]),
    "nd_needle_confidence": (I32, [P, P, C.POINTER(C.c_double)]),
    "nd_needle_step": (I32, [P, P, U32, P]),
    "nd_needle_prefill": (I32, [P, P, P, U32, P]),
    "nd_needle_step_select": (I32, [P, P, U32, P, U32, P, P]),
    "nd_needle_step_select_mask": (I32, [P, P, U32, P, U32, P, P]),
    "nd_needle_generate": (I32, [P, P, P, U32, U32, U32, U32, P, P, P]),
    "nd_needle_test_waits": (I32, [P, P, U32, U32]),
    "nd_needle_step_launches": (I32, [P, P, PU32]),
    "nd_needle_test_stamps": (I32, [P, P, P, U32]),
    "nd_needle_begin_token": (I32, [P, P, P]),
    "nd_needle_prepare_engrams": (I32, [P, P, P, P, U32, U32]),
    "nd_needle_forward_layer": (I32, [P, P, U32, U32, P, P]),
    "nd_needle_forward_token": (I32, [P, P, U32, P, P]),
    "nd_needle_finish_token": (I32, [P, P, U32, P]),
    "nd_needle_finish_token_for_selection": (I32, [P, P]),
    "nd_needle_select_token": (I32, [P, P, P, U32, P, P]),
    "nd_needle_select_token_mask": (I32, [P, P, P, U32, P, P]),
    "nd_needle_read_lanes": (I32, [P, P, P]),
    "nd_needle_forward": (I32, [P, P, U32, U32, P, P, P, P, P, P, P]),
    "nd_pieces_upload": (I32, [P, P, P, P, U32, PP]),
    "nd_pieces_free": (I32, [P, P]),
    "nd_grammar_upload": (I32, [P, P, U32, PP]),
    "nd_grammar_free": (I32, [P, P]),
    "nd_grammar_mask": (I32, [P, P, P, U32, P, U32, P, P]),
    "nd_grammar_mask_d": (I32, [P, P, P, P, U32, P, P, P]),
    "nd_needle_grammar_mask": (I32, [P, P, P, P, P, U32, U32, P, PU32]),
}


class DecoderDesc(C.Structure):
    """nd_decoder_desc of include/needle_hip.h."""

    _fields_ = [
        ("layers", U32), ("dim", U32), ("heads", U32), ("kv_heads", U32), ("head_dim", U32),
        ("ffn", U32), ("vocab", U32), ("rope_theta", C.c_float),
        ("embedding", P),
        ("wq", PP), ("wk", PP), ("wv", PP), ("wo", PP), ("wup", PP), ("wdown", PP),
        ("attn_norm", P), ("ffn_norm", P), ("q_norm", P), ("k_norm", P), ("final_norm", P),
    ]


class NeedleDesc(C.Structure):
    """nd_needle_desc of include/needle_hip.h."""

    _fields_ = [
        ("vocab", U32), ("dim", U32), ("heads", U32), ("kv_heads", U32), ("layers", U32),
        ("head_dim", U32), ("max_length", U32), ("hadamard", U32), ("lanes", U32),
        ("kv_window", U32), ("engram_slots", U32), ("engram_sub", U32), ("engram_tables", U32),
        ("engram_taps", U32), ("n_orders", U32), ("orders", U32 * 4), ("n_sites", U32),
        ("sites", U32 * 4), ("rope_theta", C.c_float),
        ("embedding", P), ("wq", PP), ("wk", PP), ("wv", PP), ("wgate", PP), ("wo", PP),
        ("phi_pre", P), ("phi_post", P), ("phi_res", P),
        ("eg_tables", PP), ("eg_key", PP), ("eg_value", PP),
        ("norm_input", P), ("query_norm", P), ("key_norm", P), ("post_attn_norm", P),
        ("pre_hadamard_norm", P), ("d1", P), ("d2", P), ("d3", P), ("attention_gate", P),
        ("a_pre", P), ("a_post", P), ("a_res", P), ("b_pre", P), ("b_post", P), ("b_res", P),
        ("eg_taps", P), ("final_norm", P),
        ("probes", P), ("probe_count", U32), ("probe_out", U32), ("probe_projection", P),
        ("probe_bias", P),
    ]


_LIB: C.CDLL | None = None


def library_path() -> Path:
    env = os.environ.get("NEEDLE_HIP_LIB")
    return Path(env) if env else DEFAULT_LIBRARY


def load_library() -> C.CDLL:
    """Loads libneedle_hip.so once and declares every entry point."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise NeedleError(
            "BACKEND_UNAVAILABLE",
            f"{path} is missing; build it with __graft_entry__.build() or make -C needle.js_amd/csrc",
        )
    try:
        lib = C.CDLL(str(path))
    except OSError as exc:  # pragma: no cover - depends on the host
        raise NeedleError("BACKEND_UNAVAILABLE", f"cannot load {path}: {exc}", exc) from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


def last_error(lib: C.CDLL, ctx) -> str:
    msg = lib.nd_last_error(ctx)
    return msg.decode(errors="replace") if msg else ""


def check(lib: C.CDLL, ctx, status: int, what: str = "") -> None:
    """Raises the NeedleError that a nonzero nd_status maps to."""
    if status == ND_OK:
        return
    code = _STATUS_CODE.get(status, "BACKEND_UNAVAILABLE")
    message = last_error(lib, ctx) or f"{what} failed with status {status}"
    raise NeedleError(code, message)


def ptr(array) -> int:
    """Address of a numpy array's data (host pointer)."""
    return array.ctypes.data
