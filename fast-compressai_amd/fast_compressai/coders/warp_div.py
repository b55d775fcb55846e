"""GA-ANS ``warp_div`` backend for MI355X: the reference's WarpDivBackend
surface on top of the wave64 HIP coder.

Same public surface as ``src/fast_compressai/coders/warp_div.py:20-215``:
``WarpDivBackend().encode(symbols, indexes, cdfs, cdf_sizes, offsets, *,
p_ch) -> WarpDivPayload`` and ``.decode(payload, indexes, cdfs, cdf_sizes,
offsets) -> int32 [B, N]``, with ``CoderInputError`` for bad inputs or
payloads and ``CoderDependencyError`` for a missing library or device.

Differences that follow from the new format:

* ``format_id`` is ``"gaans-w64-v5"``; payloads of the reference's
  ``warpans-v2`` format are rejected.
* ``segments`` (keyword of ``encode``, field of the payload) splits every
  chunk of P channels into that many independently coded units (1..256);
  None (the default) lets the coder pick enough units for the device's CUs
  within 0.6% of extra payload (``gaans.choose_segments``).
* ``WarpDivPayload.chunk_ends`` (uint32 ``[B, K S]``, exposed also under the
  reference's name ``max_rounds``) holds each coding unit's end offset in
  the payload data, not a round count.
* Index range, index content and table identity are checked on the device
  (status word) instead of with host syncs and a SHA-256 of every index.
  ``coding_fingerprint`` is a SHA-256 of the table digest and the shapes, so
  it stays cheap to recompute on every decode.
* ``channels=`` (keyword, optional) chunks over latent channels instead of
  CDF tables, for GaussianConditional-style per-element indexes.
"""

from __future__ import annotations

import functools
import hashlib
import re
import struct
from dataclasses import MISSING, dataclass, fields
import torch

from . import gaans
from .capabilities import warp_div_capability
from .errors import CoderDependencyError, CoderInputError
from .tables import PreparedTables, TableCache

FORMAT_ID = "gaans-w64-v5"
FORMAT_VERSION = 5
MAX_SEGMENTS = 256
_HEADER_MAGIC = 0x31574147
_FIXED_HEADER_BYTES = 64
_SHA256_HEX = re.compile(r"[0-9a-f]{64}")


def header_bytes_for(batch: int, units_per_row: int) -> int:
    return (_FIXED_HEADER_BYTES + 8 * batch * units_per_row + 15) // 16 * 16


@functools.lru_cache(maxsize=256)
def coding_fingerprint(table_digest: int, batch: int, symbols_per_batch: int, channels: int,
                       cdf_count: int) -> str:
    """SHA-256 over the table digest and the coding shapes."""
    text = (f"{FORMAT_ID}|tables={table_digest:016x}|B={batch}|N={symbols_per_batch}"
            f"|C={channels}|M={cdf_count}")
    return hashlib.sha256(text.encode("ascii")).hexdigest()


@dataclass(frozen=True)
class WarpDivPayload:
    packed: torch.Tensor
    chunk_ends: torch.Tensor
    header_bytes: int
    chunk_len: int
    p_ch: int
    batch: int
    symbols_per_batch: int
    cdf_count: int
    coding_fingerprint: str | None = None
    format_id: str = FORMAT_ID
    format_version: int = FORMAT_VERSION
    channels: int | None = None
    segments: int = 1

    def __post_init__(self) -> None:
        if self.format_id != FORMAT_ID or self.format_version != FORMAT_VERSION:
            raise CoderInputError("unsupported warp_div payload format")
        if type(self.segments) is not int or not 1 <= self.segments <= MAX_SEGMENTS:
            raise CoderInputError(f"warp_div segments must be in [1, {MAX_SEGMENTS}]")
        if (not isinstance(self.packed, torch.Tensor) or self.packed.device.type != "cuda"
                or self.packed.dtype != torch.uint8 or not self.packed.is_contiguous()):
            raise CoderInputError("packed payload must be contiguous GPU uint8")
        if (not isinstance(self.chunk_ends, torch.Tensor)
                or self.chunk_ends.device != self.packed.device
                or self.chunk_ends.dtype != torch.uint32 or not self.chunk_ends.is_contiguous()):
            raise CoderInputError(
                "chunk_ends must be contiguous GPU uint32 on the packed payload device")
        if self.coding_fingerprint is not None and (
            not isinstance(self.coding_fingerprint, str)
            or _SHA256_HEX.fullmatch(self.coding_fingerprint) is None
        ):
            raise CoderInputError("coding_fingerprint must be a SHA-256 hex digest")
        ints = (self.header_bytes, self.chunk_len, self.p_ch, self.batch,
                self.symbols_per_batch, self.cdf_count)
        if any(type(v) is not int for v in ints) or min(ints) <= 0:
            raise CoderInputError("warp_div metadata values must be positive integers")
        channels = self.coded_channels
        if type(channels) is not int or channels <= 0:
            raise CoderInputError("warp_div channels must be a positive integer")
        if self.p_ch > channels or self.symbols_per_batch % channels:
            raise CoderInputError("warp_div payload P_ch/channel metadata is inconsistent")
        units = (channels + self.p_ch - 1) // self.p_ch * self.segments
        if tuple(self.chunk_ends.shape) != (self.batch, units):
            raise CoderInputError("warp_div chunk table shape does not match payload metadata")
        if self.chunk_len != self.p_ch * (self.symbols_per_batch // channels):
            raise CoderInputError("warp_div chunk_len does not match P_ch and symbol dimensions")
        if self.header_bytes != header_bytes_for(self.batch, units):
            raise CoderInputError("warp_div header size does not match chunk metadata")
        if self.header_bytes > self.packed.numel():
            raise CoderInputError("warp_div header exceeds packed payload size")
        if self.packed.numel() % 4:
            raise CoderInputError("warp_div packed payload must be uint32 aligned")

    @classmethod
    def _from_encoder(cls, **values) -> "WarpDivPayload":
        """Payload built by ``WarpDivBackend.encode`` from values it has just
        produced and checked; skips the field validation of ``__init__``.
        Without ``chunk_ends`` the field is built on first use, as a view of
        the header's unit end offsets."""
        obj = object.__new__(cls)
        state = dict(_PAYLOAD_DEFAULTS)
        state.update(values)
        obj.__dict__.update(state)
        return obj

    def __getattr__(self, name: str):
        # only reached for attributes missing from the instance: the lazily
        # built fields of an encoder-made payload -- packed (the first
        # _nbytes bytes of the encoder's buffer _buf) and chunk_ends
        d = self.__dict__
        if name == "packed":
            buf = d.get("_buf")
            if buf is None:
                raise AttributeError(name)
            packed = buf[: d["_nbytes"]]
            d["packed"] = packed
            del d["_buf"]
            return packed
        if name != "chunk_ends" or ("packed" not in d and "_buf" not in d):
            raise AttributeError(name)
        channels = d["cdf_count"] if d["channels"] is None else d["channels"]
        units = (channels + d["p_ch"] - 1) // d["p_ch"] * d["segments"]
        B = d["batch"]
        ends = self.packed[64: 64 + 4 * B * units].view(torch.uint32).view(B, units)
        d["chunk_ends"] = ends
        return ends

    @property
    def coded_channels(self) -> int:
        return self.cdf_count if self.channels is None else self.channels

    @property
    def max_rounds(self) -> torch.Tensor:
        """The per-unit table ``[B, K S]`` under the reference's attribute
        name (here: coding unit end offsets, see ``chunk_ends``)."""
        return self.chunk_ends

    @property
    def chunks(self) -> int:
        """Chunks (of P channels) per batch row."""
        return int(self.chunk_ends.shape[1]) // self.segments

    def to_bytes(self) -> bytes:
        """Host copy of the payload (header + chunk streams); the format is
        self-describing, so ``from_bytes`` restores an equal payload."""
        return self.packed.cpu().numpy().tobytes()

    @classmethod
    def from_bytes(cls, data: bytes, device: torch.device | str = "cuda",
                   cdf_count: int | None = None) -> "WarpDivPayload":
        """Rebuild a payload from ``to_bytes`` output (header fields
        B, N, C, P, K, chunk_len, M, table digest, segments and unit end
        offsets)."""
        if len(data) < _FIXED_HEADER_BYTES:
            raise CoderInputError("warp_div payload header is truncated")
        words = struct.unpack_from("<16I", data, 0)
        if words[0] != _HEADER_MAGIC or words[1] != FORMAT_VERSION:
            raise CoderInputError("warp_div payload header has an unknown magic or version")
        B, N, C, P, K, chunk_len, M = words[2:9]
        S = words[12]
        if B <= 0 or K <= 0 or not 1 <= S <= MAX_SEGMENTS:
            raise CoderInputError("warp_div payload header is inconsistent")
        hb = header_bytes_for(B, K * S)
        if len(data) < hb:
            raise CoderInputError("warp_div payload header is truncated")
        if cdf_count is not None and cdf_count != M:
            raise CoderInputError("CDF count does not match payload metadata")
        digest = words[10] | (words[11] << 32)
        ends = torch.frombuffer(bytearray(data[64: 64 + 4 * B * K * S]), dtype=torch.uint8)
        dev = torch.device(device)
        packed = torch.frombuffer(bytearray(data), dtype=torch.uint8).to(dev)
        return cls(packed=packed, chunk_ends=ends.to(dev).view(torch.uint32).view(B, K * S),
                   header_bytes=hb, chunk_len=chunk_len, p_ch=P, batch=B,
                   symbols_per_batch=N, cdf_count=M,
                   coding_fingerprint=coding_fingerprint(digest, B, N, C, M),
                   channels=None if C == M else C, segments=S)


# field defaults of WarpDivPayload (for _from_encoder)
_PAYLOAD_DEFAULTS = {f.name: f.default for f in fields(WarpDivPayload) if f.default is not MISSING}


class WarpDivBackend:
    """MI355X GA-ANS coder behind the reference's ``warp_div`` surface."""

    name = "warp_div"
    format_id = FORMAT_ID
    format_version = FORMAT_VERSION

    def __init__(self) -> None:
        capability = warp_div_capability()
        if not capability.available:
            raise CoderDependencyError(f"warp_div unavailable: {capability.reason}")
        from . import _native

        _native.lib()  # raises CoderDependencyError when it cannot be loaded
        self._tables = TableCache()
        # shape -> (tables, segments, payload fields) of the last encodes
        self._shapes: dict = {}
        # payload metadata -> (tables, channels, device, index shape) of the
        # last decodes that passed every check
        self._decode_shapes: dict = {}

    def prepared_tables(self, cdfs: torch.Tensor, cdf_sizes: torch.Tensor,
                        offsets: torch.Tensor) -> PreparedTables:
        return self._tables.get(cdfs, cdf_sizes, offsets)

    def encode(
        self,
        symbols: torch.Tensor,
        indexes: torch.Tensor,
        cdfs: torch.Tensor,
        cdf_sizes: torch.Tensor,
        offsets: torch.Tensor,
        *,
        p_ch: int,
        channels: int | None = None,
        segments: int | None = None,
    ) -> WarpDivPayload:
        tables = self._tables.hit(cdfs, cdf_sizes, offsets)
        if tables is None:
            C = _validate_inputs(symbols, indexes, cdfs, cdf_sizes, offsets, p_ch, channels)
            tables = self.prepared_tables(cdfs, cdf_sizes, offsets)
        else:  # the same table tensors as the last call: their checks passed then
            C = _validate_data(symbols, indexes, p_ch, channels, tables)
        B, N = int(symbols.shape[0]), int(symbols.shape[1])
        device = symbols.device
        # per shape: the segment choice and every payload field but the bytes
        key = (B, N, C, p_ch, channels, segments, device)
        memo = self._shapes.get(key)
        if memo is None or memo[0] is not tables:
            seg = gaans.resolve_segments(segments, tables, B, N, C, p_ch, device)
            lay = gaans.layout(B, N, C, p_ch, seg)
            fields_ = dict(_PAYLOAD_DEFAULTS, header_bytes=lay.header_bytes,
                           chunk_len=lay.chunk_len, p_ch=int(p_ch), batch=B,
                           symbols_per_batch=N, cdf_count=tables.M,
                           coding_fingerprint=coding_fingerprint(tables.digest, B, N, C,
                                                                 tables.M),
                           channels=None if channels is None else int(channels), segments=seg)
            memo = (tables, seg, fields_)
            if len(self._shapes) > 64:
                self._shapes.clear()
            self._shapes[key] = memo
        buf, nbytes = gaans.encode_symbols_raw(tables, B, N, C, p_ch, device, symbols, indexes,
                                               memo[1])
        payload = object.__new__(WarpDivPayload)  # fields produced and checked here
        state = payload.__dict__
        state.update(memo[2])
        if buf.numel() - nbytes > gaans.CLONE_SLACK_BYTES:
            state["packed"] = buf[:nbytes].clone()
        else:  # packed is sliced from the buffer on first use
            state["_buf"] = buf
            state["_nbytes"] = nbytes
        return payload

    def decode(
        self,
        payload: WarpDivPayload,
        indexes: torch.Tensor,
        cdfs: torch.Tensor,
        cdf_sizes: torch.Tensor,
        offsets: torch.Tensor,
    ) -> torch.Tensor:
        if not isinstance(payload, WarpDivPayload):
            raise CoderInputError("warp_div decode expects WarpDivPayload")
        tables = self._tables.hit(cdfs, cdf_sizes, offsets)
        if tables is not None:
            # payload metadata checked before with these tables: only the
            # call's own tensors need checking (anything unusual takes the
            # full path below, which raises the right error)
            d = payload.__dict__
            key = (d["p_ch"], d["channels"], d["batch"], d["symbols_per_batch"], d["cdf_count"],
                   d["coding_fingerprint"], d["segments"])
            memo = self._decode_shapes.get(key)
            packed = d.get("packed")
            if packed is None:  # an encoder-made payload not sliced yet
                packed, nbytes = d["_buf"], d["_nbytes"]
            else:
                nbytes = packed.numel()
            if (memo is not None and memo[0] is tables and isinstance(indexes, torch.Tensor)
                    and indexes.dtype == torch.int32 and indexes.device == memo[2]
                    and packed.device == memo[2] and indexes.is_contiguous()
                    and indexes.shape == memo[3]):
                return gaans.decode_symbols_ptr(packed.data_ptr(), nbytes, tables, d["batch"],
                                                d["symbols_per_batch"], memo[1], d["p_ch"],
                                                memo[2], indexes, d["segments"])
        if tables is None:
            C = _validate_inputs(indexes, indexes, cdfs, cdf_sizes, offsets, payload.p_ch,
                                 payload.channels)
        else:
            C = _validate_data(indexes, indexes, payload.p_ch, payload.channels, tables)
        if tuple(indexes.shape) != (payload.batch, payload.symbols_per_batch):
            raise CoderInputError("indexes shape does not match payload metadata")
        if cdfs.shape[0] != payload.cdf_count or indexes.device != payload.packed.device:
            raise CoderInputError("CDF count or GPU device does not match payload metadata")
        if tables is None:
            tables = self.prepared_tables(cdfs, cdf_sizes, offsets)
        B, N = payload.batch, payload.symbols_per_batch
        if payload.coding_fingerprint is not None and payload.coding_fingerprint != \
                coding_fingerprint(tables.digest, B, N, C, payload.cdf_count):
            raise CoderInputError("coding tables or indexes do not match warp_div payload")
        device = payload.packed.device
        key = (payload.p_ch, payload.channels, B, N, payload.cdf_count,
               payload.coding_fingerprint, payload.segments)
        if len(self._decode_shapes) > 64:
            self._decode_shapes.clear()
        self._decode_shapes[key] = (tables, C, device, torch.Size((B, N)))
        return gaans.decode(payload.packed, tables, B, N, C, payload.p_ch, device,
                            indexes=indexes, segments=payload.segments)


def _validate_data(symbols: torch.Tensor, indexes: torch.Tensor, p_ch: int,
                   channels: int | None, tables: PreparedTables) -> int:
    """The checks of ``_validate_inputs`` that concern the symbols and indexes,
    for table tensors that passed them on an earlier call (same messages).
    Returns the channel count used for chunking."""
    T = torch.Tensor
    if not isinstance(symbols, T) or not isinstance(indexes, T):
        raise CoderInputError("symbols and indexes must be torch tensors")
    if type(p_ch) is not int or p_ch <= 0:
        raise CoderInputError("p_ch must be a positive integer")
    dev = symbols.device
    if dev != tables.device or indexes.device != dev:
        raise CoderInputError("all coder inputs must be GPU tensors on the same device")
    if symbols.dtype != torch.int32 or indexes.dtype != torch.int32:
        raise CoderInputError("all warp_div input tensors must use torch.int32")
    if not (symbols.is_contiguous() and indexes.is_contiguous()):
        raise CoderInputError("all warp_div input tensors must be contiguous")
    shape = symbols.shape
    if len(shape) != 2 or indexes.shape != shape:
        raise CoderInputError("symbols and indexes must have matching [B, N] shape")
    if shape[0] <= 0 or shape[1] <= 0:
        raise CoderInputError("empty symbols are not supported by this WarpANS format")
    C = tables.M if channels is None else channels
    if type(C) is not int or C <= 0:
        raise CoderInputError("channels must be a positive integer")
    if shape[1] % C != 0:
        raise CoderInputError("symbols per batch must be divisible by the channel count")
    if p_ch > C:
        raise CoderInputError("p_ch cannot exceed the number of CDF channels")
    return C


def _validate_inputs(
    symbols: torch.Tensor,
    indexes: torch.Tensor,
    cdfs: torch.Tensor,
    cdf_sizes: torch.Tensor,
    offsets: torch.Tensor,
    p_ch: int,
    channels: int | None = None,
) -> int:
    """Host-side checks of the reference (``warp_div.py:179-215``) without the
    index min/max sync (index range is checked on the device).  Returns the
    channel count used for chunking."""
    T = torch.Tensor
    if not isinstance(symbols, T) or not isinstance(indexes, T):
        raise CoderInputError("symbols and indexes must be torch tensors")
    if not (isinstance(cdfs, T) and isinstance(cdf_sizes, T) and isinstance(offsets, T)):
        raise CoderInputError("indexes, CDFs, CDF sizes, and offsets must be tensors")
    if type(p_ch) is not int or p_ch <= 0:
        raise CoderInputError("p_ch must be a positive integer")
    dev = symbols.device
    if (dev.type != "cuda" or indexes.device != dev or cdfs.device != dev
            or cdf_sizes.device != dev or offsets.device != dev):
        raise CoderInputError("all coder inputs must be GPU tensors on the same device")
    i32 = torch.int32
    if (symbols.dtype != i32 or indexes.dtype != i32 or cdfs.dtype != i32
            or cdf_sizes.dtype != i32 or offsets.dtype != i32):
        raise CoderInputError("all warp_div input tensors must use torch.int32")
    if not (symbols.is_contiguous() and indexes.is_contiguous() and cdfs.is_contiguous()
            and cdf_sizes.is_contiguous() and offsets.is_contiguous()):
        raise CoderInputError("all warp_div input tensors must be contiguous")
    if symbols.ndim != 2 or indexes.shape != symbols.shape:
        raise CoderInputError("symbols and indexes must have matching [B, N] shape")
    if cdfs.ndim != 2 or cdf_sizes.ndim != 1 or offsets.ndim != 1:
        raise CoderInputError("CDF must be [M,L] and CDF sizes/offsets must be [M]")
    if cdfs.shape[0] <= 0 or cdfs.shape[1] < 2:
        raise CoderInputError("CDF table cannot be empty")
    if cdf_sizes.numel() != cdfs.shape[0] or offsets.numel() != cdfs.shape[0]:
        raise CoderInputError("CDF, CDF sizes, and offsets must have the same table count")
    if symbols.shape[0] <= 0 or symbols.shape[1] <= 0:
        raise CoderInputError("empty symbols are not supported by this WarpANS format")
    C = int(cdfs.shape[0]) if channels is None else channels
    if type(C) is not int or C <= 0:
        raise CoderInputError("channels must be a positive integer")
    if symbols.shape[1] % C != 0:
        raise CoderInputError("symbols per batch must be divisible by the channel count")
    if p_ch > C:
        raise CoderInputError("p_ch cannot exceed the number of CDF channels")
    return C
