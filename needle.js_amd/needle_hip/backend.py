"""HipBackend: the InferenceBackend contract of needle.js over libneedle_hip.

Mirrors backends/backend.ts:82-110 (kind, name, weights, matvec, matvecBatch,
createResidentSession, row, dispose) with Python naming.  Matrices are either
the archive's own Cactus-Quant form (cact.CqMatrix, model/cact.ts:61-75:
packed 2/3/4-bit or ternary codes, binary16 group norms, a shared codebook)
or its int8 form (codes [n][k] int8 and one fp32 scale per (row, group of g
columns)), the form of the resident Needle 2 and batched decoders.  Each
matrix is uploaded to HBM once, on first use, and cached by identity as
backends/typegpu.ts:390-410 does.
Results are fresh float32 arrays (backends/cpu.ts:12-16).
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import lib as L
from .errors import NeedleError, invariant


class Int8Matrix:
    """int8 variant of CqMatrix: codes [n][k] and f32 scales [n][k/g]."""

    kind = "int8"

    def __init__(self, codes: np.ndarray, scales: np.ndarray, group_size: int, name: str = ""):
        codes = np.ascontiguousarray(codes, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        invariant(codes.ndim == 2, "INVALID_CACT", "matrix codes must be 2-D")
        n, k = codes.shape
        invariant(group_size > 0 and k % group_size == 0, "INVALID_CACT",
                  f"group size {group_size} does not divide {k}")
        invariant(scales.shape == (n, k // group_size), "INVALID_CACT",
                  f"scales shape {scales.shape} does not match {(n, k // group_size)}")
        self.codes = codes
        self.scales = scales
        self.group_size = group_size
        self.name = name

    @property
    def output_size(self) -> int:
        return self.codes.shape[0]

    @property
    def input_size(self) -> int:
        return self.codes.shape[1]

    @property
    def shape(self):
        return self.codes.shape


@dataclass(frozen=True)
class MatrixRowRange:
    row_start: Optional[int] = None
    row_count: Optional[int] = None


@dataclass(frozen=True)
class MatvecRequest:
    matrix: Int8Matrix
    input: np.ndarray
    range: Optional[MatrixRowRange] = None


class HipBackend:
    """Third needle.js backend: MI355X (gfx950) through libneedle_hip.so."""

    kind = "hip"
    name = "MI355X HIP (gfx950)"

    def __init__(self, weights=None, device: int = 0, resident_layers: bool = True):
        self.weights = weights
        self.resident_layers = resident_layers
        self.lib = L.load_library()
        ctx = C.c_void_p()
        status = self.lib.nd_create(device, C.byref(ctx))
        if status != L.ND_OK:
            raise NeedleError("BACKEND_UNAVAILABLE", L.last_error(self.lib, None) or
                              f"nd_create failed with status {status}")
        self.ctx = ctx
        self.device = device
        self._mats: dict[int, tuple[Int8Matrix, C.c_void_p]] = {}
        self._disposed = False

    # -- helpers --------------------------------------------------------
    def _check(self, status: int, what: str = "") -> None:
        L.check(self.lib, self.ctx, status, what)

    def _alive(self) -> None:
        invariant(not self._disposed, "BACKEND_UNAVAILABLE", "HIP backend has been disposed")

    def upload(self, matrix: Int8Matrix) -> C.c_void_p:
        """HBM handle of `matrix`, uploading it on first use."""
        self._alive()
        entry = self._mats.get(id(matrix))
        if entry is not None and entry[0] is matrix:
            return entry[1]
        handle = C.c_void_p()
        if getattr(matrix, "kind", None) == "cq":
            cb = matrix.codebook
            self._check(self.lib.nd_mat_upload_cq(
                self.ctx, L.ptr(matrix.packed), L.ptr(matrix.norms),
                None if cb is None else L.ptr(cb), matrix.output_size, matrix.input_size,
                matrix.group_size, matrix.bits, C.byref(handle)), "nd_mat_upload_cq")
        else:
            n, k = matrix.codes.shape
            self._check(self.lib.nd_mat_upload_i8(self.ctx, L.ptr(matrix.codes),
                                                  L.ptr(matrix.scales), n, k, matrix.group_size,
                                                  C.byref(handle)), "nd_mat_upload_i8")
        self._mats[id(matrix)] = (matrix, handle)
        return handle

    @staticmethod
    def _resolve_range(matrix: Int8Matrix, rng: Optional[MatrixRowRange]):
        rng = rng or MatrixRowRange()
        start = 0 if rng.row_start is None else rng.row_start
        count = matrix.output_size - start if rng.row_count is None else rng.row_count
        invariant(isinstance(start, (int, np.integer)) and isinstance(count, (int, np.integer))
                  and start >= 0 and count >= 0 and start + count <= matrix.output_size,
                  "INVALID_CACT", f"Invalid matrix row range {start}:{start + count}")
        return int(start), int(count)

    @staticmethod
    def _input(matrix: Int8Matrix, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        invariant(x.shape[-1] == matrix.input_size, "INVALID_CACT",
                  f"Matrix expects {matrix.input_size} inputs, received {x.shape[-1]}")
        return x

    # -- InferenceBackend -------------------------------------------------
    def matvec(self, matrix: Int8Matrix, input: np.ndarray,
               range: Optional[MatrixRowRange] = None) -> np.ndarray:
        """Selected rows of matrix @ input; input [k] or [batch][k]."""
        handle = self.upload(matrix)
        start, count = self._resolve_range(matrix, range)
        x = self._input(matrix, input)
        batch = 1 if x.ndim == 1 else x.shape[0]
        y = np.empty((batch, count), dtype=np.float32)
        self._check(self.lib.nd_matvec(self.ctx, handle, L.ptr(x), batch, start, count, L.ptr(y)),
                    "nd_matvec")
        return y[0] if x.ndim == 1 else y

    def matvec_batch(self, requests: Sequence[MatvecRequest]) -> list[np.ndarray]:
        """Independent matvecs with one host synchronisation."""
        if not requests:
            return []
        jobs = (L.MatvecJob * len(requests))()
        keep = []
        outs = []
        inputs: dict[int, np.ndarray] = {}
        for i, req in enumerate(requests):
            handle = self.upload(req.matrix)
            start, count = self._resolve_range(req.matrix, req.range)
            x = inputs.get(id(req.input))
            if x is None or x.shape[-1] != req.matrix.input_size:
                x = self._input(req.matrix, req.input)
                inputs[id(req.input)] = x
            y = np.empty(count, dtype=np.float32)
            keep.append(x)
            outs.append(y)
            jobs[i].mat = handle
            jobs[i].x = L.ptr(x)
            jobs[i].row_start = start
            jobs[i].row_count = count
            jobs[i].y = L.ptr(y)
        self._check(self.lib.nd_matvec_batch(self.ctx, jobs, len(requests)), "nd_matvec_batch")
        return outs

    def row(self, matrix: Int8Matrix, row: int, output: Optional[np.ndarray] = None) -> np.ndarray:
        handle = self.upload(matrix)
        invariant(isinstance(row, (int, np.integer)) and 0 <= row < matrix.output_size,
                  "INVALID_CACT", f"Matrix row {row} is out of range")
        result = np.empty(matrix.input_size, dtype=np.float32)
        self._check(self.lib.nd_row(self.ctx, handle, int(row), L.ptr(result)), "nd_row")
        if output is not None:
            invariant(output.shape[0] >= matrix.input_size, "INVALID_CACT",
                      "Row output buffer is too short")
            output[: matrix.input_size] = result
            return output
        return result

    def create_resident_session(self):
        """createResidentSession (backends/backend.ts:103-104): a
        ResidentExecutionSession over this backend's Needle 2 weights (their
        matrices resident in HBM with one runtime state), or None when the
        backend serves no Needle 2 weights.  Sessions run whole tokens on the
        device unless the backend was built with resident_layers=False."""
        from .needle2 import Needle2Weights
        from .runtime import HipNeedleSession

        self._alive()
        if not isinstance(self.weights, Needle2Weights):
            return None
        return HipNeedleSession(self, self.weights, self.resident_layers)

    def dispose(self) -> None:
        if self._disposed:
            return
        self._disposed = True
        self.lib.nd_destroy(self.ctx)
        self._mats.clear()
        self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()

    # -- device-level operators used by the runtime and the bench ---------
    def select(self, logits: np.ndarray, allowed: Optional[np.ndarray] = None):
        """selectToken over host logits: (id, log_probability)."""
        self._alive()
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        out_id = C.c_uint32()
        out_lp = C.c_double()
        if allowed is None:
            st = self.lib.nd_select(self.ctx, L.ptr(logits), logits.shape[0], None, 0,
                                    C.byref(out_id), C.byref(out_lp))
        else:
            allowed = np.ascontiguousarray(allowed, dtype=np.uint32)
            invariant(allowed.size > 0, "INVALID_CACT", "Allowed token set is empty")
            st = self.lib.nd_select(self.ctx, L.ptr(logits), logits.shape[0], L.ptr(allowed),
                                    allowed.size, C.byref(out_id), C.byref(out_lp))
        self._check(st, "nd_select")
        return int(out_id.value), float(out_lp.value)
