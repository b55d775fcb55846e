"""Coder capability discovery without loading the native library.

Mirrors ``src/fast_compressai/coders/capabilities.py:11-49`` of the reference:
``warp_div_capability`` reports whether the GA-ANS GPU coder can run, and
``coder_catalog`` / ``create_coder`` list and build the two coders.
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
    """Return exactly the supported entropy coder backend identifiers."""
    return ("compressai-rans", "warp_div")


def create_coder(name: str):
    """Construct one supported backend without loading unrelated backends."""
    if name == "compressai-rans":
        from .compressai_ans import CompressAIANSBackend

        return CompressAIANSBackend()
    if name == "warp_div":
        from .warp_div import WarpDivBackend

        return WarpDivBackend()
    raise ValueError(f"unsupported coder {name!r}; supported coders are {coder_catalog()}")
