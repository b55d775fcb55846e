"""Table upload: CompressAI quantized CDFs laid out for the GA-ANS kernels.

CompressAI keeps ``_quantized_cdf`` as a zero-padded ``[M, Lmax]`` int32
tensor with ``_cdf_length`` and ``_offset`` (reference
``src/fast_compressai/coders/factorized.py:23-31``).  The kernels instead read
a compact blob built once per table set by ``gaans_tables_prepare``: per-table
metadata, per-symbol entries (``start | (freq - 1) << 16`` and the
encoder's division magic of ``freq``), a 256-bucket decode lookup and, for
buckets in which several symbols start, second- and third-level lookups of
16 entries (16-value sub-ranges, then single values); and the compact
search lookups (a u32 per bucket and a u16 start per symbol) that the
decoder stages instead when many wide tables (GaussianConditional) leave no
room for the sub-blocks.  The blob also carries the table digest that every
payload records, so decoding with other tables is detected on the device.
"""

from __future__ import annotations

import ctypes
import threading
from collections import OrderedDict
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _native
from .errors import CoderInputError


@dataclass(frozen=True)
class PreparedTables:
    blob: torch.Tensor  # device uint8
    nbytes: int
    M: int
    Lmax: int
    digest: int
    desc: _native.Tables  # C descriptor pointing at ``blob``
    device: torch.device = None  # the device of ``blob``
    # call plans of these tables by shape (gaans.py); they point into ``blob``
    plans: dict = field(default_factory=dict, compare=False, repr=False)

    @property
    def ref(self):
        return ctypes.byref(self.desc)

    @property
    def digest_hex(self) -> str:
        return f"{self.digest:016x}"


def prepare_tables(cdfs: torch.Tensor, cdf_sizes: torch.Tensor, offsets: torch.Tensor,
                   device: torch.device | None = None) -> PreparedTables:
    """Validate and lay out tables; the blob is placed on ``device``
    (default: the device of ``cdfs``)."""
    if cdfs.ndim != 2 or cdf_sizes.ndim != 1 or offsets.ndim != 1:
        raise CoderInputError("CDF must be [M,L] and CDF sizes/offsets must be [M]")
    M, Lmax = int(cdfs.shape[0]), int(cdfs.shape[1])
    if M <= 0 or Lmax < 2:
        raise CoderInputError("CDF table cannot be empty")
    if cdf_sizes.numel() != M or offsets.numel() != M:
        raise CoderInputError("CDF, CDF sizes, and offsets must have the same table count")
    c = np.ascontiguousarray(cdfs.detach().to("cpu").numpy().astype(np.int32, copy=False))
    s = np.ascontiguousarray(cdf_sizes.detach().to("cpu").numpy().astype(np.int32, copy=False))
    o = np.ascontiguousarray(offsets.detach().to("cpu").numpy().astype(np.int32, copy=False))
    L = _native.lib()
    nbytes = ctypes.c_int64(0)
    rc = L.gaans_tables_bytes(c.ctypes.data, s.ctypes.data, M, Lmax, ctypes.byref(nbytes))
    if rc != _native.OK:
        raise CoderInputError(f"invalid CDF tables: {_native.last_error()}")
    host = np.zeros(nbytes.value, dtype=np.uint8)
    desc = _native.Tables()
    rc = L.gaans_tables_prepare(c.ctypes.data, s.ctypes.data, o.ctypes.data, M, Lmax,
                                host.ctypes.data, nbytes.value, ctypes.byref(desc))
    if rc != _native.OK:
        raise CoderInputError(f"invalid CDF tables: {_native.last_error()}")
    dev = device if device is not None else cdfs.device
    blob = torch.from_numpy(host).to(dev)
    desc.dev = blob.data_ptr()
    return PreparedTables(blob=blob, nbytes=int(nbytes.value), M=M, Lmax=Lmax,
                          digest=int(desc.digest), desc=desc, device=blob.device)


class TableCache:
    """Small LRU of prepared tables keyed by the identity and in-place version
    of the source tensors.  Entries keep the source tensors alive, so a key
    cannot be reused by another allocation while it is cached."""

    def __init__(self, capacity: int = 8) -> None:
        self._capacity = capacity
        self._entries: OrderedDict = OrderedDict()
        self._lock = threading.Lock()
        # the last hit: the same three tensor objects, unchanged since, give
        # the same tables (checked first, without building a key)
        self._last = None

    @staticmethod
    def _key(tensors):
        # device pointers are unique across devices; dtype and device are
        # checked by the callers before tables are prepared
        return tuple((t.data_ptr(), t._version, t.shape, t.stride()) for t in tensors)

    def hit(self, cdfs, cdf_sizes, offsets) -> PreparedTables | None:
        """The tables of the last call when these are the same three tensor
        objects, unchanged since (in-place version and storage); else None."""
        last = self._last
        if (last is not None and last[0] is cdfs and last[1] is cdf_sizes and last[2] is offsets
                and last[3] == (cdfs._version, cdf_sizes._version, offsets._version,
                                cdfs.data_ptr(), cdf_sizes.data_ptr(), offsets.data_ptr())):
            return last[4]
        return None

    def get(self, cdfs: torch.Tensor, cdf_sizes: torch.Tensor,
            offsets: torch.Tensor) -> PreparedTables:
        last = self._last
        if (last is not None and last[0] is cdfs and last[1] is cdf_sizes and last[2] is offsets
                and last[3] == (cdfs._version, cdf_sizes._version, offsets._version,
                                cdfs.data_ptr(), cdf_sizes.data_ptr(), offsets.data_ptr())):
            return last[4]
        prepared = self._get(cdfs, cdf_sizes, offsets)
        self._last = (cdfs, cdf_sizes, offsets,
                      (cdfs._version, cdf_sizes._version, offsets._version, cdfs.data_ptr(),
                       cdf_sizes.data_ptr(), offsets.data_ptr()), prepared)
        return prepared

    def _get(self, cdfs: torch.Tensor, cdf_sizes: torch.Tensor,
             offsets: torch.Tensor) -> PreparedTables:
        key = self._key((cdfs, cdf_sizes, offsets))
        with self._lock:
            hit = self._entries.get(key)
            if hit is not None:
                self._entries.move_to_end(key)
                return hit[0]
        prepared = prepare_tables(cdfs, cdf_sizes, offsets)
        with self._lock:
            self._entries[key] = (prepared, (cdfs, cdf_sizes, offsets))
            while len(self._entries) > self._capacity:
                self._entries.popitem(last=False)
        return prepared
