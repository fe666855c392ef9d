"""Exception categories of the public API.

Mirrors the reference's error classes
(``packages/opake-base/src/opake/api/base/exceptions/__init__.py:8-48``) so that
call sites catching ``ValueError`` / ``TypeError`` / ``RuntimeError`` behave the
same way.
"""

from __future__ import annotations

from typing import NoReturn


class OpakeError(Exception):
    """Base class for failures reported by the public API."""

    @classmethod
    def raise_(
        cls,
        message: str,
        *,
        cause: BaseException | None = None,
        suppress_context: bool = False,
    ) -> NoReturn:
        """Raise ``cls(message)``, chained to ``cause`` or with the context
        suppressed.  Nothing in this package calls it: it is kept for API
        compatibility, because code written against the reference raises its
        errors as ``ConfigurationError.raise_(...)``
        (packages/opake-base/src/opake/api/base/exceptions/__init__.py)."""
        if suppress_context:
            raise cls(message) from None
        if cause is not None:
            raise cls(message) from cause
        raise cls(message)


class ConfigurationError(OpakeError, ValueError):
    """Invalid or incompatible configuration (a ``ValueError``)."""


class InputTypeError(OpakeError, TypeError):
    """An argument of an invalid type (a ``TypeError``)."""


class OperationError(OpakeError, RuntimeError):
    """An operation could not complete, e.g. the native library is missing."""


__all__ = ["ConfigurationError", "InputTypeError", "OpakeError", "OperationError"]
