"""The errors the ops raise.

When Ayaka itself is importable, its own classes are used, so an engine that
catches ``ayaka.core.errors.BackendError`` catches ours (reference
``python/ayaka/core/errors.py:83-124,193-196``). Otherwise this module defines
stand-ins with the same constructors and attributes.
"""

from __future__ import annotations

from collections.abc import Mapping

__all__ = ["AyakaError", "BackendError", "CapabilityError", "ConfigError"]

try:  # pragma: no cover - exercised only where the engine is installed
    from ayaka.core.errors import (  # type: ignore[import-not-found]
        AyakaError,
        BackendError,
        CapabilityError,
        ConfigError,
    )
except ImportError:

    class AyakaError(Exception):  # type: ignore[no-redef]
        """Base class of every error raised here; carries a stable ``code``."""

        code: str = "ayaka_error"
        retryable: bool = False

        def __init__(self, message: str, *, context: Mapping[str, object] | None = None) -> None:
            self.message = message
            self.context: dict[str, object] = dict(context or {})
            super().__init__(message)

    class BackendError(AyakaError, RuntimeError):  # type: ignore[no-redef]
        """An op could not run as specified; it never computes something else instead."""

        code = "backend_error"

    class CapabilityError(AyakaError, ImportError):  # type: ignore[no-redef]
        """A backend or library is unavailable on this machine."""

        code = "capability_unavailable"

        def __init__(self, capability: str, *, detail: str, remedy: str) -> None:
            self.capability = capability
            self.detail = detail
            self.remedy = remedy
            super().__init__(f"capability {capability!r} unavailable: {detail}. Remedy: {remedy}")

    class ConfigError(AyakaError, ValueError):  # type: ignore[no-redef]
        """A configuration validation failure with a stable path and code."""

        def __init__(
            self,
            path: str,
            code: str,
            message: str,
            *,
            context: Mapping[str, object] | None = None,
        ) -> None:
            self.path = path
            self.code = code
            self.message = message
            self.context = dict(context or {})
            Exception.__init__(self, f"{path}: {message} [{code}]")
