"""Exception types of the forge_amd ops, named and subclassed like the reference's (forge/core/errors.py:7-93) so
callers that catch ``ConfigError`` (a ``ValueError``) or ``HardwareUnsupported`` keep working."""
from __future__ import annotations

from typing import Any


class ForgeError(Exception):
    """Base class; ``code`` is a stable machine-readable identifier."""

    code: str = "forge_error"

    def __init__(self, message: str = "", *, details: dict[str, Any] | None = None) -> None:
        super().__init__(message)
        self.message = message
        self.details: dict[str, Any] = dict(details or {})

    def __str__(self) -> str:
        return self.message


class ConfigError(ForgeError, ValueError):
    """Invalid user/config input."""

    code = "config_error"


class NotFound(ForgeError, LookupError):
    """Unknown registry entry (e.g. a layout id)."""

    code = "not_found"


class HardwareUnsupported(ForgeError):
    """The request needs hardware this build does not run on (forge_amd: gfx950 GPUs only)."""

    code = "hardware_unsupported"


class KernelCorrectnessError(ForgeError):
    """A kernel disagreed with its reference oracle beyond tolerance."""

    code = "kernel_correctness_error"
