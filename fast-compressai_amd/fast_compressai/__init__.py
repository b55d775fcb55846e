"""fast_compressai (MI355X): GA-ANS latent coding for CompressAI-style models.

Drop-in for the reference's coder path: ``accelerate(model, P=...,
coder="warp_div")``, ``WarpDivBackend`` / ``WarpDivPayload`` and the coder
catalog, running hand-written HIP kernels for gfx950.
"""

from .api import AccelerationReport, FastModel, accelerate, compile
from .coders import (
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
from .p_ch import (PChSelection, choose_p_ch, default_p_candidates, legal_p_candidates,
                   sweep_p_ch)
from .pipeline import CodingPipeline

__all__ = [
    "AccelerationConfig",
    "AccelerationReport",
    "BitstreamError",
    "CoderCapability",
    "CoderDependencyError",
    "CoderError",
    "CoderInputError",
    "CoderStateError",
    "CodingPipeline",
    "CompressAIANSBackend",
    "ConfigurationError",
    "FastModel",
    "PChSelection",
    "WarpDivBackend",
    "WarpDivPayload",
    "accelerate",
    "choose_p_ch",
    "coder_catalog",
    "compile",
    "create_coder",
    "default_p_candidates",
    "legal_p_candidates",
    "sweep_p_ch",
    "warp_div_capability",
]

__version__ = "0.1.0"
