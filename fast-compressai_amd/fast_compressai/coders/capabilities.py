"""Which coders this build offers and whether the GPU one can run here.

Same names as the reference's ``src/fast_compressai/coders/capabilities.py:11-49``
(``warp_div_capability``, ``coder_catalog``, ``create_coder`` and the
``CoderCapability`` record), answered for this build: the GA-ANS coder needs
a visible GPU and the built HIP library, which is only looked for on disk
here, not loaded.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native


@dataclass(frozen=True)
class CoderCapability:
    backend: str
    available: bool
    reason: str | None
    device: str | None
    persistent_payload: bool


def warp_div_capability(device: torch.device | str | None = None) -> CoderCapability:
    """Whether the MI355X GA-ANS coder can run on ``device`` (default: cuda).

    On ROCm builds of PyTorch the ``cuda`` device type is the HIP device.
    """
    requested = torch.device(device) if device is not None else None
    if not torch.cuda.is_available():
        return CoderCapability("warp_div", False, "GPU runtime/device unavailable", None, False)
    if requested is not None and requested.type != "cuda":
        return CoderCapability("warp_div", False, "warp_div requires a GPU ('cuda') device",
                               str(requested), False)
    target = str(requested or torch.device("cuda"))
    if not _native.library_available():
        return CoderCapability("warp_div", False,
                               "GA-ANS HIP library is not built (run __graft_entry__.build())",
                               target, False)
    return CoderCapability("warp_div", True, None, target, False)


def coder_catalog() -> tuple[str, ...]:
    """Names ``create_coder`` accepts: CompressAI's CPU RANS and the GA-ANS
    GPU coder."""
    return ("compressai-rans", "warp_div")


def create_coder(name: str):
    """An instance of the coder called ``name``; only that coder's module
    (and its dependency: CompressAI, or the HIP library) is loaded."""
    if name == "compressai-rans":
        from .rans_host import CompressAIANSBackend

        return CompressAIANSBackend()
    if name == "warp_div":
        from .warp_div import WarpDivBackend

        return WarpDivBackend()
    raise ValueError(f"unsupported coder {name!r}; supported coders are {coder_catalog()}")
