"""Errors the hip-gfx950 path raises on purpose, with the reference's stable codes.

The class names, bases and ``AOTO-xxxx`` codes follow the reference's error
catalogue (``errors.py:46-226``) for the errors this path can raise, so a
caller that catches ``CompilationError`` or ``PlanInputError`` from the
reference keeps working unchanged.
"""

from __future__ import annotations


class AotolithError(Exception):
    """Base class of every deliberate error; ``code`` is stable, ``hint`` optional."""

    code = "AOTO-0000"

    def __init__(self, message: str, *, hint: str | None = None, code: str | None = None) -> None:
        super().__init__(message)
        self.message = message
        self.hint = hint
        if code is not None:
            self.code = code

    def __str__(self) -> str:
        return self.message

    def describe(self) -> str:
        text = f"[{self.code}] {self.message}"
        return f"{text}\nhint: {self.hint}" if self.hint else text


class CompilationError(AotolithError, ValueError):
    code = "AOTO-1000"


class UnsupportedOperationError(CompilationError, NotImplementedError):
    code = "AOTO-1001"


class DynamicShapeError(CompilationError):
    code = "AOTO-1002"


class UnsupportedDTypeError(CompilationError):
    code = "AOTO-1003"


class UnsupportedModelError(CompilationError, NotImplementedError):
    code = "AOTO-1004"


class IRValidationError(AotolithError, ValueError):
    code = "AOTO-1010"


class PlanInputError(AotolithError, ValueError):
    code = "AOTO-2001"


class IndexBoundsError(AotolithError, IndexError):
    code = "AOTO-2002"


class MemoryBudgetError(AotolithError, RuntimeError):
    code = "AOTO-2004"


class BucketRangeError(PlanInputError):
    code = "AOTO-2005"


class DeviceError(AotolithError, RuntimeError):
    code = "AOTO-3001"


class ArtifactError(AotolithError, RuntimeError):
    code = "AOTO-4001"


class ArtifactCompatibilityError(ArtifactError):
    code = "AOTO-4002"
