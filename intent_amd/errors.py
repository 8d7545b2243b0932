"""Exception types of the operator surface.

``CompilationStageError`` keeps the reference's shape (a stage tag plus a
message; python/intent/compiler/toolchain.py:17-26). Native status codes map
onto the exception types the reference's binders raise
(python/intent/runtime/invocation.py:42-53,90-100): ``ValueError`` for bad
shapes, strides, alignment and workspace, ``NotImplementedError`` for shapes
the kernels do not cover, ``RuntimeError`` for HIP failures.
"""
from __future__ import annotations

from pathlib import Path


class CompilationStageError(RuntimeError):
    def __init__(self, stage: str, message: str, *, cache_directory: Path | None = None,
                 candidate: str | None = None) -> None:
        super().__init__(message)
        self.stage = stage
        self.cache_directory = cache_directory
        self.candidate = candidate


class NativeLibraryError(RuntimeError):
    """The gfx950 library is missing or does not export the expected ABI."""


class LanguageUseError(RuntimeError):
    """A definition was invoked before compilation."""


# Status codes of include/intent_amd.h.
INTENT_OK = 0
INTENT_ERR_INVALID_ARGUMENT = -1
INTENT_ERR_ALIGNMENT = -2
INTENT_ERR_UNSUPPORTED = -3
INTENT_ERR_LAUNCH = -4
INTENT_ERR_WORKSPACE = -5


def status_error(status: int, entry: str, message: str) -> Exception:
    text = f"{entry}: {message or 'failed'} (status {status})"
    if status in (INTENT_ERR_INVALID_ARGUMENT, INTENT_ERR_ALIGNMENT, INTENT_ERR_WORKSPACE):
        return ValueError(text)
    if status == INTENT_ERR_UNSUPPORTED:
        return NotImplementedError(text)
    return RuntimeError(text)
