"""NeedleError and invariant, mirroring errors.ts:1-32 of needle.js."""

from __future__ import annotations

NEEDLE_ERROR_CODES = (
    "INVALID_CACT",
    "UNSUPPORTED_CACT",
    "WEIGHTS_NOT_FOUND",
    "WEIGHTS_INTEGRITY",
    "WEBGPU_UNAVAILABLE",
    "BACKEND_UNAVAILABLE",
    "CONTEXT_OVERFLOW",
    "INVALID_TOOL_SCHEMA",
    "GRAMMAR_DEAD_END",
    "GENERATION_ABORTED",
)


class NeedleError(Exception):
    """An error with a stable code suitable for application-level handling."""

    def __init__(self, code: str, message: str, cause: BaseException | None = None):
        if code not in NEEDLE_ERROR_CODES:
            raise ValueError(f"unknown NeedleError code {code}")
        super().__init__(message)
        self.code = code
        self.cause = cause

    def __repr__(self) -> str:
        return f"NeedleError({self.code!r}, {str(self)!r})"


def invariant(condition, code: str, message: str) -> None:
    if not condition:
        raise NeedleError(code, message)
