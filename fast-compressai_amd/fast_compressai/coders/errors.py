"""Errors raised by the coder backends.

Same classes and hierarchy as the reference
(``src/fast_compressai/coders/errors.py:4-21``), so callers that catch them
keep working.
"""


class CoderError(RuntimeError):
    """Base class for coder failures."""


class CoderInputError(CoderError, ValueError):
    """Raised when symbols, indexes, CDF metadata or a payload is invalid."""


class CoderStateError(CoderError):
    """Raised when a coder session is used in an invalid state."""


class BitstreamError(CoderError, ValueError):
    """Raised for malformed or incompatible bitstreams."""


class CoderDependencyError(CoderError, ImportError):
    """Raised when a coder dependency (the HIP library, a GPU) is unavailable."""
