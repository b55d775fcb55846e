"""ctypes wrapper of the CPU oracle (oracle/gaans_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``, never by the product package.

* ``rans64_encode`` / ``rans64_decode``: CompressAI-equivalent Rans64 single
  stream (reference ``src/fast_compressai/coders/cuda/rans64_gpu.cuh:5-55``,
  ``rans64dec_gpu.cuh:8-48``, escapes ``warp_ans_kernel_v2.cu:139-169`` /
  ``warp_ans_kernel.cu:299-327``, stream order ``ans_gpu_kernel.cu:133-194``).
* ``gaans_encode`` / ``gaans_decode``: sequential emulation of the wave64
  GA-ANS payload format that the HIP kernels must reproduce byte for byte.
* ``quantize`` / ``dequantize``: CompressAI ``EntropyModel.quantize(...,
  "symbols", means)`` / ``dequantize`` closed forms (reference call sites
  ``src/fast_compressai/coders/factorized.py:46-49``, ``:99-101``).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# GAANS_ORACLE_LIB selects another build of the same source (the sanitizer
# tests load one built with -fsanitize=address,undefined)
_LIB_PATH = os.environ.get("GAANS_ORACLE_LIB") or os.path.join(_HERE, "lib", "libgaans_oracle.so")
_lib = None

ERRORS = {
    -1: "invalid arguments",
    -2: "invalid CDF table",
    -3: "table index out of range",
    -4: "escape value does not fit 32 bits",
    -5: "output buffer too small",
    -6: "payload corrupt",
    -7: "payload made with other tables or indexes",
}


class OracleError(RuntimeError):
    def __init__(self, code: int, where: str):
        super().__init__(f"{where}: {ERRORS.get(code, code)} ({code})")
        self.code = code


def build() -> str:
    """Compile the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i32, i64 = ctypes.c_int32, ctypes.c_int64
        L.rans64_ref_encode.argtypes = [p, p, i64, p, i32, i32, p, p, p, i64, p]
        L.rans64_ref_decode.argtypes = [p, i64, p, i64, p, i32, i32, p, p, p]
        L.gaans_ref_max_payload_bytes.argtypes = [i32, i32, i32, i32, i32]
        L.gaans_ref_max_payload_bytes.restype = i64
        L.gaans_ref_table_digest.argtypes = [p, i32, i32, p, p]
        L.gaans_ref_table_digest.restype = ctypes.c_uint64
        L.gaans_ref_encode.argtypes = [p, p, i32, i32, i32, i32, i32, p, i32, i32, p, p, p, i64,
                                       p]
        L.gaans_ref_decode.argtypes = [p, i64, p, i32, i32, i32, i32, i32, p, i32, i32, p, p, p]
        L.gaans_ref_index_term.argtypes = [i64, i32]
        L.gaans_ref_index_term.restype = ctypes.c_uint32
        L.gaans_ref_quantize.argtypes = [p, p, i32, i32, i64, p]
        L.gaans_ref_dequantize.argtypes = [p, p, i32, i32, i64, p]
        L.gaans_ref_build_indexes.argtypes = [p, i64, p, i32, ctypes.c_float, p]
        L.gaans_ref_quantize_elem.argtypes = [p, p, i64, p]
        L.gaans_ref_dequantize_elem.argtypes = [p, p, i64, p]
        for name in ("rans64_ref_encode", "rans64_ref_decode", "gaans_ref_encode",
                     "gaans_ref_decode"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _tables(cdfs, cdf_sizes, offsets):
    cdfs = _i32(cdfs)
    if cdfs.ndim != 2:
        raise ValueError("cdfs must be [M, Lmax]")
    return cdfs, _i32(cdf_sizes).reshape(-1), _i32(offsets).reshape(-1)


def rans64_encode(symbols, indexes, cdfs, cdf_sizes, offsets) -> bytes:
    """One CompressAI-equivalent stream; returns the little-endian bytes."""
    s, ix = _i32(symbols).reshape(-1), _i32(indexes).reshape(-1)
    cdfs, sizes, offs = _tables(cdfs, cdf_sizes, offsets)
    cap = 11 * s.size + 4
    out = np.zeros(cap, dtype=np.uint32)
    n = ctypes.c_int64(0)
    rc = lib().rans64_ref_encode(_ptr(s), _ptr(ix), s.size, _ptr(cdfs), cdfs.shape[0],
                                 cdfs.shape[1], _ptr(sizes), _ptr(offs), _ptr(out), cap,
                                 ctypes.byref(n))
    if rc:
        raise OracleError(rc, "rans64_encode")
    return out[: n.value].astype("<u4").tobytes()


def rans64_decode(data: bytes, indexes, cdfs, cdf_sizes, offsets) -> np.ndarray:
    ix = _i32(indexes).reshape(-1)
    cdfs, sizes, offs = _tables(cdfs, cdf_sizes, offsets)
    words = np.frombuffer(bytes(data), dtype="<u4").astype(np.uint32)
    out = np.zeros(ix.size, dtype=np.int32)
    rc = lib().rans64_ref_decode(_ptr(words), words.size, _ptr(ix), ix.size, _ptr(cdfs),
                                 cdfs.shape[0], cdfs.shape[1], _ptr(sizes), _ptr(offs),
                                 _ptr(out))
    if rc:
        raise OracleError(rc, "rans64_decode")
    return out


def table_digest(cdfs, cdf_sizes, offsets) -> int:
    cdfs, sizes, offs = _tables(cdfs, cdf_sizes, offsets)
    return int(lib().gaans_ref_table_digest(_ptr(cdfs), cdfs.shape[0], cdfs.shape[1],
                                            _ptr(sizes), _ptr(offs)))


def index_term(p: int, tb: int) -> int:
    """One position's term of a chunk's index hash."""
    return int(lib().gaans_ref_index_term(p, tb))


def gaans_encode(symbols, indexes, cdfs, cdf_sizes, offsets, p_ch: int,
                 channels: int | None = None, segments: int = 1) -> bytes:
    """Payload bytes of the wave64 format.  ``symbols`` is [B, N];
    ``indexes`` is [B, N] or None (channel-major: table = channel);
    ``segments`` independently coded segments per chunk."""
    s = _i32(symbols)
    if s.ndim != 2:
        raise ValueError("symbols must be [B, N]")
    B, N = s.shape
    cdfs, sizes, offs = _tables(cdfs, cdf_sizes, offsets)
    C = cdfs.shape[0] if channels is None else int(channels)
    ix = None if indexes is None else _i32(indexes).reshape(B, N)
    cap = lib().gaans_ref_max_payload_bytes(B, N, C, p_ch, segments)
    if cap < 0:
        raise OracleError(-1, "gaans_encode")
    out = np.zeros(cap, dtype=np.uint8)
    n = ctypes.c_int64(0)
    rc = lib().gaans_ref_encode(_ptr(s), None if ix is None else _ptr(ix), B, N, C, p_ch,
                                segments, _ptr(cdfs), cdfs.shape[0], cdfs.shape[1], _ptr(sizes),
                                _ptr(offs), _ptr(out), cap, ctypes.byref(n))
    if rc:
        raise OracleError(rc, "gaans_encode")
    return out[: n.value].tobytes()


def gaans_decode(payload: bytes, indexes, B: int, N: int, cdfs, cdf_sizes, offsets,
                 p_ch: int, channels: int | None = None, segments: int = 1) -> np.ndarray:
    cdfs, sizes, offs = _tables(cdfs, cdf_sizes, offsets)
    C = cdfs.shape[0] if channels is None else int(channels)
    ix = None if indexes is None else _i32(indexes).reshape(B, N)
    buf = np.frombuffer(bytes(payload), dtype=np.uint8)
    out = np.zeros((B, N), dtype=np.int32)
    rc = lib().gaans_ref_decode(_ptr(buf), buf.size, None if ix is None else _ptr(ix), B, N,
                                C, p_ch, segments, _ptr(cdfs), cdfs.shape[0], cdfs.shape[1],
                                _ptr(sizes), _ptr(offs), _ptr(out))
    if rc:
        raise OracleError(rc, "gaans_decode")
    return out


def quantize(y, medians) -> np.ndarray:
    """y: float32 [B, C, *spatial]; medians: float32 [C]."""
    y = np.ascontiguousarray(np.asarray(y, dtype=np.float32))
    med = np.ascontiguousarray(np.asarray(medians, dtype=np.float32).reshape(-1))
    B, C = y.shape[0], y.shape[1]
    HW = int(np.prod(y.shape[2:])) if y.ndim > 2 else 1
    out = np.zeros(y.shape, dtype=np.int32)
    lib().gaans_ref_quantize(_ptr(y), _ptr(med), B, C, HW, _ptr(out))
    return out


def dequantize(symbols, medians) -> np.ndarray:
    s = _i32(symbols)
    med = np.ascontiguousarray(np.asarray(medians, dtype=np.float32).reshape(-1))
    B, C = s.shape[0], s.shape[1]
    HW = int(np.prod(s.shape[2:])) if s.ndim > 2 else 1
    out = np.zeros(s.shape, dtype=np.float32)
    lib().gaans_ref_dequantize(_ptr(s), _ptr(med), B, C, HW, _ptr(out))
    return out


def build_indexes(scales, scale_table, bound: float) -> np.ndarray:
    """CompressAI GaussianConditional.build_indexes (restated): int32 indexes
    of ``scales`` (any shape) into ``scale_table``."""
    sc = np.ascontiguousarray(scales, np.float32)
    tab = np.ascontiguousarray(scale_table, np.float32)
    out = np.zeros(sc.shape, np.int32)
    lib().gaans_ref_build_indexes(_ptr(sc), sc.size, _ptr(tab), tab.size, float(bound), _ptr(out))
    return out


def quantize_elem(y, means=None) -> np.ndarray:
    """int32(rint(y - means)) elementwise (CompressAI quantize, "symbols")."""
    yy = np.ascontiguousarray(y, np.float32)
    m = None if means is None else np.ascontiguousarray(means, np.float32)
    out = np.zeros(yy.shape, np.int32)
    lib().gaans_ref_quantize_elem(_ptr(yy), None if m is None else _ptr(m), yy.size, _ptr(out))
    return out


def dequantize_elem(symbols, means=None) -> np.ndarray:
    """fp32(symbols) + means elementwise (CompressAI dequantize)."""
    s = np.ascontiguousarray(symbols, np.int32)
    m = None if means is None else np.ascontiguousarray(means, np.float32)
    out = np.zeros(s.shape, np.float32)
    lib().gaans_ref_dequantize_elem(_ptr(s), None if m is None else _ptr(m), s.size, _ptr(out))
    return out
