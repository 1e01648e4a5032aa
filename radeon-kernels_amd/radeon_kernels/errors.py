"""Exception roots shared by the runtime and the operators.

Mirrors src/radeon_kernels/errors.py:1-12 of the reference: expected user-facing failures derive
from RadeonKernelsError; configuration problems carry the offending path.
"""

from __future__ import annotations


class RadeonKernelsError(Exception):
    """Base error for expected user-facing failures."""


class ConfigError(RadeonKernelsError):
    """A manifest, contract or pack document is malformed; ``path`` names the location."""

    def __init__(self, path: str, message: str) -> None:
        self.path = path
        self.message = message
        super().__init__(f"{path}: {message}")
