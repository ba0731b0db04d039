"""Error types of the hot path, mirroring the reference's core/errors.py:1-13."""
from __future__ import annotations


class MoltStreamError(RuntimeError):
    """Base error for explicit, non-fallback failures."""


class CapabilityError(MoltStreamError):
    """The requested mechanism is unavailable on the current runtime."""


MoltError = MoltStreamError
