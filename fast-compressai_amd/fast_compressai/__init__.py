"""fast_compressai (MI355X): GA-ANS latent coding for CompressAI-style models.

Drop-in for the reference's coder path: ``accelerate(model, P=...,
coder="warp_div")``, ``WarpDivBackend`` / ``WarpDivPayload`` and the coder
catalog, running hand-written HIP kernels for gfx950.
"""

from .api import AccelerationReport, FastModel, accelerate, compile
from .coders import (
    Bitstream,
    BitstreamError,
    CoderCapability,
    CoderDependencyError,
    CoderError,
    CoderInputError,
    CoderStateError,
    CompressAIANSBackend,
    WarpDivBackend,
    WarpDivPayload,
    coder_catalog,
    create_coder,
    warp_div_capability,
)
from .config import AccelerationConfig, ConfigurationError

__all__ = [
    "AccelerationConfig",
    "AccelerationReport",
    "Bitstream",
    "BitstreamError",
    "CoderCapability",
    "CoderDependencyError",
    "CoderError",
    "CoderInputError",
    "CoderStateError",
    "CompressAIANSBackend",
    "ConfigurationError",
    "FastModel",
    "WarpDivBackend",
    "WarpDivPayload",
    "accelerate",
    "coder_catalog",
    "compile",
    "create_coder",
    "warp_div_capability",
]

__version__ = "0.1.0"
