"""GA-ANS (MI355X) and CompressAI RANS entropy coder backends."""

from .capabilities import CoderCapability, coder_catalog, create_coder, warp_div_capability
from .errors import (
    BitstreamError,
    CoderDependencyError,
    CoderError,
    CoderInputError,
    CoderStateError,
)
from .rans_host import CompressAIANSBackend
from .warp_div import WarpDivBackend, WarpDivPayload

__all__ = [
    "BitstreamError",
    "CoderCapability",
    "CoderDependencyError",
    "CoderError",
    "CoderInputError",
    "CoderStateError",
    "CompressAIANSBackend",
    "WarpDivBackend",
    "WarpDivPayload",
    "coder_catalog",
    "create_coder",
    "warp_div_capability",
]
