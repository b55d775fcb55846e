"""CompressAI's CPU RANS coder for whole batches: the ``coder="rans"`` stream
format on the host, and the decoder small batches of CompressAI strings are
sent to.

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

``rans64_route`` decides where a batch of CompressAI strings is decoded:
CompressAI's host decoder while the batch is below ``RANS64_GPU_MIN_STREAMS``
and CompressAI is importable, the GPU Rans64 decoder otherwise.  One stream is
one serial chain of symbols, so the GPU decodes a stream per lane and wins
only with many streams in flight: on one MI355X a 1x192x32x48 stream takes
about 90 ms whatever the batch up to a few hundred streams, against 3.3 ms on
one CPU thread, so the GPU overtakes one host thread at about 28 streams.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np

from .errors import CoderDependencyError, CoderInputError

# streams at and above which the GPU decodes faster than one host thread
RANS64_GPU_MIN_STREAMS = 28


def compressai_ans_module():
    """``compressai.ans`` or None when CompressAI is not importable."""
    try:
        from compressai import ans
    except ImportError:
        return None
    if not (hasattr(ans, "RansEncoder") and hasattr(ans, "RansDecoder")):
        return None
    return ans


def rans64_route(batch: int, host_available: bool | None = None) -> str:
    """``"host"`` when a batch of ``batch`` CompressAI strings decodes faster
    with CompressAI's CPU decoder (importable and fewer than
    ``RANS64_GPU_MIN_STREAMS`` streams), else ``"gpu"``."""
    if host_available is None:
        host_available = compressai_ans_module() is not None
    return "host" if host_available and batch < RANS64_GPU_MIN_STREAMS else "gpu"


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
