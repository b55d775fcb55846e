"""CompressAI RANS-backed CPU coder (the ``coder="rans"`` path and the CPU
baseline boundary).

Mirrors ``src/fast_compressai/coders/compressai_ans.py:14-161`` of the
reference: a one-shot encoder session around CompressAI's
``ans.RansEncoder.encode_with_indexes`` and a decoder around
``ans.RansDecoder.decode_with_indexes``.  CompressAI is imported lazily; when
it is absent the constructor raises ``CoderDependencyError``.
"""

from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass, field
from typing import Any, Mapping, Sequence

from .errors import BitstreamError, CoderDependencyError, CoderError, CoderInputError, CoderStateError

CDF_PRECISION = 16
CDF_TOTAL = 1 << CDF_PRECISION


@dataclass(frozen=True)
class Bitstream:
    """Host-side CompressAI RANS payload with its coding metadata."""

    backend: str
    payload: bytes
    symbol_count: int
    shape: tuple[int, ...] = ()
    metadata: Mapping[str, Any] = field(default_factory=dict)

    def __post_init__(self) -> None:
        if not isinstance(self.payload, (bytes, bytearray)):
            raise BitstreamError("payload must be bytes")
        if type(self.symbol_count) is not int or self.symbol_count < 0:
            raise BitstreamError("symbol_count must be a non-negative integer")


def normalize_coding_metadata(indexes, cdfs, offsets):
    """Validation of ``src/fast_compressai/coders/interface.py:51-84``."""
    try:
        indexes = list(indexes)
        cdfs = [list(cdf) for cdf in cdfs]
        offsets = list(offsets)
    except (TypeError, ValueError) as exc:
        raise CoderInputError("indexes, cdfs, and offsets must be integer sequences") from exc
    for name, values in (("indexes", indexes), ("offsets", offsets)):
        if any(type(v) is not int for v in values):
            raise CoderInputError(f"{name} must contain integers (bool is not accepted)")
    for row, cdf in enumerate(cdfs):
        if any(type(v) is not int for v in cdf):
            raise CoderInputError(f"CDF {row} must contain integers")
        if len(cdf) < 2:
            raise CoderInputError(f"CDF {row} must contain at least two values")
        if cdf[0] != 0 or cdf[-1] != CDF_TOTAL:
            raise CoderInputError(f"CDF {row} must start at zero and end at {CDF_TOTAL}")
        if any(a >= b for a, b in zip(cdf, cdf[1:])):
            raise CoderInputError(f"CDF {row} must be strictly increasing")
    if not cdfs and indexes:
        raise CoderInputError("cdfs must contain at least one CDF")
    if len(offsets) != len(cdfs):
        raise CoderInputError("offsets length must match the number of CDFs")
    if any(i < 0 or i >= len(cdfs) for i in indexes):
        raise CoderInputError("CDF index is out of range")
    return indexes, cdfs, offsets


def _fingerprint(indexes: Sequence[int], cdfs, offsets) -> str:
    canonical = json.dumps({"indexes": list(indexes), "cdfs": [list(c) for c in cdfs],
                            "offsets": list(offsets), "precision": CDF_PRECISION},
                           separators=(",", ":"), sort_keys=True).encode("ascii")
    return hashlib.sha256(canonical).hexdigest()


class CompressAIANSBackend:
    """CPU backend backed by CompressAI's fixed-precision RANS extension."""

    name = "compressai-rans"
    schema_version = 1

    def __init__(self) -> None:
        try:
            from compressai import ans
        except (ImportError, ModuleNotFoundError) as exc:
            raise CoderDependencyError(
                "CompressAI RANS is unavailable; install CompressAI") from exc
        self._encoder_type = getattr(ans, "RansEncoder", None)
        self._decoder_type = getattr(ans, "RansDecoder", None)
        if self._encoder_type is None or self._decoder_type is None:
            raise CoderDependencyError("the installed CompressAI package has no RANS encoder/decoder")

    def create_session(self, *, symbol_count: int, shape: Sequence[int] = (),
                       metadata: Mapping[str, Any] | None = None) -> "CompressAIANSEncoderSession":
        if type(symbol_count) is not int or symbol_count < 0:
            raise CoderInputError("symbol_count must be a non-negative integer")
        return CompressAIANSEncoderSession(self._encoder_type, self.name, symbol_count, shape,
                                           metadata)

    def decode(self, bitstream: Bitstream, *, indexes, cdfs, offsets) -> list[int]:
        if not isinstance(bitstream, Bitstream):
            raise CoderInputError("decode expects a Bitstream")
        if bitstream.backend != self.name:
            raise CoderInputError(f"bitstream backend {bitstream.backend!r} does not match {self.name!r}")
        indexes, cdfs, offsets = normalize_coding_metadata(indexes, cdfs, offsets)
        if len(indexes) != bitstream.symbol_count:
            raise CoderInputError("indexes length must equal bitstream symbol_count")
        expected = (bitstream.metadata or {}).get("coding_fingerprint")
        if expected is not None and expected != _fingerprint(indexes, cdfs, offsets):
            raise BitstreamError("coding metadata does not match bitstream fingerprint")
        if bitstream.symbol_count == 0:
            return []
        try:
            return list(self._decoder_type().decode_with_indexes(
                bitstream.payload, indexes, cdfs, [len(c) for c in cdfs], offsets))
        except Exception as exc:
            raise CoderError("CompressAI RANS decode failed") from exc


class CompressAIANSEncoderSession:
    """One-shot encoder: one full symbol sequence per session."""

    def __init__(self, encoder_type, backend: str, symbol_count: int, shape, metadata) -> None:
        self._encoder_type = encoder_type
        self._backend = backend
        self._symbol_count = symbol_count
        self._shape = tuple(shape)
        self._metadata = dict(metadata or {})
        self._payload: bytes | None = None
        self._failed = False
        self._finalized = False
        self._encode_attempted = False

    def encode(self, symbols, indexes, cdfs, offsets) -> None:
        self._ensure_open()
        if self._encode_attempted:
            raise CoderStateError("one-shot coder session accepts only one encode() call")
        self._encode_attempted = True
        try:
            symbols = list(symbols)
            if any(type(v) is not int for v in symbols):
                raise CoderInputError("symbols must contain integers (bool is not accepted)")
            indexes, cdfs, offsets = normalize_coding_metadata(indexes, cdfs, offsets)
            if len(symbols) != len(indexes):
                raise CoderInputError("symbols and indexes must have equal lengths")
            if len(symbols) != self._symbol_count:
                raise CoderInputError("encoded symbol count does not match session symbol_count")
            self._metadata["coding_fingerprint"] = _fingerprint(indexes, cdfs, offsets)
            if not symbols:
                self._payload = b""
                return
            self._payload = bytes(self._encoder_type().encode_with_indexes(
                symbols, indexes, cdfs, [len(c) for c in cdfs], offsets))
        except Exception:
            self._failed = True
            raise

    def finalize(self) -> Bitstream:
        self._ensure_open()
        if not self._encode_attempted:
            if self._symbol_count != 0:
                raise CoderStateError("cannot finalize a non-empty session before encoding its symbols")
            self._encode_attempted = True
            self._payload = b""
        if self._payload is None:
            raise CoderStateError("coder session has no finalized payload")
        self._finalized = True
        return Bitstream(self._backend, self._payload, self._symbol_count, self._shape,
                         self._metadata)

    def _ensure_open(self) -> None:
        if self._failed:
            raise CoderStateError("coder session failed and cannot be reused")
        if self._finalized:
            raise CoderStateError("coder session is already finalized")
