"""CompressAI's RANS stream format on the host: CompressAI's own coder for
whole batches (the ``coder="rans"`` backend), and this library's host decoder
of CompressAI strings, which batches too small for the GPU are sent to.

CompressAI writes one Rans64 stream per image: its entropy models call
``compressai.ans.RansEncoder().encode_with_indexes(symbols, indexes, cdfs,
cdf_lengths, offsets)`` and ``RansDecoder().decode_with_indexes(stream, ...)``
with Python lists (the reference reaches the same two calls through its
``coder="rans"`` backend, ``src/fast_compressai/coders/compressai_ans.py:76-84``,
``:125-133``).  ``CompressAIANSBackend`` here codes a ``[B, N]`` batch row by
row with those calls: tables are converted to lists once per call, rows one
at a time, and the results come back as ``bytes`` per row and an int32
``[B, N]`` array.  CompressAI is a third-party library; when it cannot be
imported the constructor raises ``CoderDependencyError`` (nothing falls back
to another coder).

``rans64_route`` decides where a batch of CompressAI strings is decoded: on
the host (``decode_rows_host``: ``gaans_rans64_decode_host``, C++ in this
library, streams shared out over the host's threads) while that is faster,
else on the GPU (``k_rans64_decode``).  One stream is one serial chain of
symbols, so the GPU decodes a stream per lane and wins only with many streams
in flight: on one MI355X a 1x192x32x48 stream takes about 89 ms whatever the
batch up to one stream per SIMD, against 1.5 ms on one host thread (both
measured by ``bench.py``, ``rans64_decode_*``), so with 16 host threads the
host stays faster up to about 950 streams.
"""

from __future__ import annotations

import math
import os
from typing import Sequence

import numpy as np

from .errors import CoderDependencyError, CoderInputError

# one 1x192x32x48 CompressAI stream (294,912 symbols), in milliseconds: GPU
# decode of a batch of up to one stream per SIMD (88.4-89.3 ms for 1 to 256
# streams on one MI355X), and host decode on one thread of the same box (1.48
# ms; the batch of 256 on its 16 threads took 31.5 ms)
GPU_STREAM_MS = 89.0
HOST_STREAM_MS = 1.5


def host_threads() -> int:
    """Host threads this process may run on."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        return max(1, os.cpu_count() or 1)


def compressai_ans_module():
    """``compressai.ans`` or None when CompressAI is not importable."""
    try:
        from compressai import ans
    except ImportError:
        return None
    if not (hasattr(ans, "RansEncoder") and hasattr(ans, "RansDecoder")):
        return None
    return ans


def rans64_route(batch: int, threads: int | None = None) -> str:
    """``"host"`` when a batch of ``batch`` CompressAI strings decodes faster
    on the host's ``threads`` threads (default: all this process may use),
    one stream per thread at a time, than on the GPU; else ``"gpu"``."""
    threads = host_threads() if threads is None else max(1, int(threads))
    host_ms = math.ceil(batch / threads) * HOST_STREAM_MS
    return "host" if host_ms < GPU_STREAM_MS else "gpu"


def decode_rows_host(strings: Sequence[bytes], indexes, cdfs, cdf_sizes, offsets, N: int,
                     C: int, threads: int | None = None) -> np.ndarray:
    """Decode B CompressAI Rans64 strings on the host with this library's
    decoder (``gaans_rans64_decode_host``): int32 symbols ``[B, N]``;
    ``indexes`` int ``[B, N]`` or None for table = channel (C channels of
    N // C symbols); tables as CompressAI keeps them.  Raises
    CoderInputError for a corrupt stream or an index outside the tables."""
    import ctypes

    from . import _native

    if not strings or not all(isinstance(s, (bytes, bytearray)) for s in strings):
        raise CoderInputError("expected a non-empty list of CompressAI byte strings")
    B = len(strings)
    c = np.ascontiguousarray(_host_array(cdfs, "cdfs", 2), dtype=np.int32)
    sizes = np.ascontiguousarray(_host_array(cdf_sizes, "cdf_sizes", 1), dtype=np.int32)
    offs = np.ascontiguousarray(_host_array(offsets, "offsets", 1), dtype=np.int32)
    if not (len(sizes) == len(offs) == c.shape[0]):
        raise CoderInputError("cdfs, cdf_sizes and offsets describe different table counts")
    idx = None
    if indexes is not None:
        idx = np.ascontiguousarray(_host_array(indexes, "indexes", 2), dtype=np.int32)
        if idx.shape != (B, N):
            raise CoderInputError(f"indexes of shape {idx.shape}, expected {(B, N)}")
    lens = np.fromiter((len(s) for s in strings), dtype=np.int64, count=B)
    so = np.zeros(B + 1, dtype=np.int64)
    np.cumsum(lens, out=so[1:])
    buf = np.frombuffer(b"".join(bytes(s) for s in strings), dtype=np.uint8)
    out = np.empty((B, N), dtype=np.int32)
    status = ctypes.c_uint32(0)
    ptr = lambda a: None if a is None or a.size == 0 else a.ctypes.data
    L = _native.lib()
    rc = L.gaans_rans64_decode_host(ptr(buf), so.ctypes.data, ptr(idx), c.ctypes.data,
                                    sizes.ctypes.data, offs.ctypes.data, c.shape[0], c.shape[1],
                                    B, N, C, 0 if threads is None else int(threads),
                                    out.ctypes.data, ctypes.byref(status))
    _native.check(rc, "host Rans64 decode")
    if status.value:
        raise CoderInputError(f"Rans64 decode failed: {_native.describe_status(status.value)}")
    return out


def _host_array(value, name: str, ndim: int) -> np.ndarray:
    if hasattr(value, "detach"):  # a torch tensor, possibly on a GPU
        value = value.detach().to("cpu").numpy()
    arr = np.asarray(value)
    if arr.ndim != ndim or not np.issubdtype(arr.dtype, np.integer):
        raise CoderInputError(f"{name} must be a {ndim}-D integer array")
    return arr.astype(np.int64, copy=False)


class CompressAIANSBackend:
    """``coder="rans"`` on the host: CompressAI's Rans64 coder, one stream
    per batch row."""

    name = "compressai-rans"

    def __init__(self) -> None:
        ans = compressai_ans_module()
        if ans is None:
            raise CoderDependencyError(
                "CompressAI is not importable; its CPU RANS coder (compressai.ans) is needed "
                "for coder='compressai-rans'")
        self._ans = ans

    @staticmethod
    def _table_lists(cdfs, cdf_sizes, offsets):
        c = _host_array(cdfs, "cdfs", 2)
        sizes = _host_array(cdf_sizes, "cdf_sizes", 1)
        offs = _host_array(offsets, "offsets", 1)
        if not (len(sizes) == len(offs) == c.shape[0]):
            raise CoderInputError("cdfs, cdf_sizes and offsets describe different table counts")
        return c.tolist(), sizes.tolist(), offs.tolist()

    def encode_rows(self, symbols, indexes, cdfs, cdf_sizes, offsets) -> list[bytes]:
        """One CompressAI stream per row of int ``symbols`` / ``indexes``
        ``[B, N]``; tables as CompressAI keeps them (``[M, Lmax]`` padded
        quantized CDFs, lengths, offsets)."""
        sym = _host_array(symbols, "symbols", 2)
        idx = _host_array(indexes, "indexes", 2)
        if sym.shape != idx.shape:
            raise CoderInputError("symbols and indexes must have the same [B, N] shape")
        tabs = self._table_lists(cdfs, cdf_sizes, offsets)
        enc = self._ans.RansEncoder()
        return [bytes(enc.encode_with_indexes(s.tolist(), i.tolist(), *tabs))
                for s, i in zip(sym, idx)]

    def decode_rows(self, strings: Sequence[bytes], indexes, cdfs, cdf_sizes,
                    offsets) -> np.ndarray:
        """Decode one CompressAI stream per row of ``indexes`` ``[B, N]`` into
        int32 symbols ``[B, N]``."""
        idx = _host_array(indexes, "indexes", 2)
        if len(strings) != idx.shape[0]:
            raise CoderInputError(f"{len(strings)} streams for {idx.shape[0]} index rows")
        tabs = self._table_lists(cdfs, cdf_sizes, offsets)
        dec = self._ans.RansDecoder()
        out = np.empty(idx.shape, dtype=np.int32)
        for b, (data, row) in enumerate(zip(strings, idx)):
            out[b] = dec.decode_with_indexes(bytes(data), row.tolist(), *tabs)
        return out
