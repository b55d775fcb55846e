"""Device-side GA-ANS engine: thin wrappers over the C ABI that allocate the
buffers with the PyTorch caching allocator and launch on the current stream.

Each encode makes exactly one host synchronisation (reading the payload size
and the device status word before the payload is allocated); each decode
makes one (reading the status word).  Reference host APIs replaced:
``encode_with_indexes_warp_v2_cuda`` (``warp_ans_kernel_v2.cu:183-306``) and
``decode_with_indexes_warp_cuda`` (``warp_ans_kernel.cu:477-544``).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native
from .errors import CoderInputError
from .tables import PreparedTables


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


@dataclass(frozen=True)
class EncodedChunks:
    packed: torch.Tensor      # uint8 [payload bytes]
    chunk_ends: torch.Tensor  # uint32 [B, K], end offset of every chunk after the header
    header_bytes: int
    chunk_len: int
    K: int


def encode(tables: PreparedTables, B: int, N: int, C: int, P: int, device: torch.device, *,
           symbols: torch.Tensor | None = None, indexes: torch.Tensor | None = None,
           y: torch.Tensor | None = None, medians: torch.Tensor | None = None) -> EncodedChunks:
    """Encode int32 ``symbols`` [B, N], or fp32 latents ``y`` with per-channel
    ``medians`` (quantize fused).  ``indexes`` None means channel-major tables."""
    L = _native.lib()
    lay = _native.layout(B, N, C, P)
    ws = torch.empty(int(lay.workspace_bytes), dtype=torch.uint8, device=device)
    stream = _stream(device)
    with torch.cuda.device(device):
        if y is not None:
            rc = L.gaans_encode_latents(stream, y.data_ptr(), medians.data_ptr(), _ptr(indexes),
                                        tables.blob.data_ptr(), tables.nbytes, tables.M, B, N, C,
                                        P, ws.data_ptr(), ws.numel())
        else:
            rc = L.gaans_encode_symbols(stream, symbols.data_ptr(), _ptr(indexes),
                                        tables.blob.data_ptr(), tables.nbytes, tables.M, B, N, C,
                                        P, ws.data_ptr(), ws.numel())
        _native.check(rc, "GA-ANS encode")
        info = ws[lay.ws_info: lay.ws_info + 16].view(torch.int64).cpu()  # the one sync
        total, status = int(info[0]), int(info[1])
        if status:
            raise CoderInputError(f"GA-ANS encode failed: {_native.describe_status(status)}")
        packed = torch.empty(total, dtype=torch.uint8, device=device)
        rc = L.gaans_encode_pack(stream, ws.data_ptr(), ws.numel(), tables.blob.data_ptr(),
                                 tables.nbytes, tables.M, B, N, C, P, packed.data_ptr(), total)
        _native.check(rc, "GA-ANS pack")
        ends = ws[lay.ws_end_off: lay.ws_end_off + 4 * lay.BK].clone()
    chunk_ends = ends.view(torch.uint32).view(B, int(lay.K))
    return EncodedChunks(packed, chunk_ends, int(lay.header_bytes), int(lay.chunk_len),
                         int(lay.K))


def decode(packed: torch.Tensor, tables: PreparedTables, B: int, N: int, C: int, P: int,
           device: torch.device, *, indexes: torch.Tensor | None = None,
           medians: torch.Tensor | None = None) -> torch.Tensor:
    """Decode to int32 symbols [B, N], or (``medians`` given) to fp32 y_hat
    [B, N] with dequantize fused."""
    L = _native.lib()
    status = torch.zeros(1, dtype=torch.int32, device=device)
    stream = _stream(device)
    with torch.cuda.device(device):
        if medians is not None:
            out = torch.empty((B, N), dtype=torch.float32, device=device)
            rc = L.gaans_decode_latents(stream, packed.data_ptr(), packed.numel(), _ptr(indexes),
                                        tables.blob.data_ptr(), tables.nbytes, tables.M,
                                        medians.data_ptr(), B, N, C, P, out.data_ptr(),
                                        status.data_ptr())
        else:
            out = torch.empty((B, N), dtype=torch.int32, device=device)
            rc = L.gaans_decode_symbols(stream, packed.data_ptr(), packed.numel(), _ptr(indexes),
                                        tables.blob.data_ptr(), tables.nbytes, tables.M, B, N, C,
                                        P, out.data_ptr(), status.data_ptr())
        _native.check(rc, "GA-ANS decode")
        st = int(status.item())  # the one sync
    if st:
        raise CoderInputError(f"warp_div decode failed: {_native.describe_status(st)}")
    return out
