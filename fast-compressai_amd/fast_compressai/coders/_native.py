"""ctypes binding of the HIP GA-ANS library (``include/gaans_w64.h``).

The library is loaded lazily and only from this package's ``lib/`` folder;
there is no fallback: if it is missing, :class:`CoderDependencyError` is
raised.  Replaces the reference's pybind11 module
``fast_compressai.coders._warp_div`` (``src/fast_compressai/coders/cuda/ans_gpu.cpp:25-30``).
"""

from __future__ import annotations

import ctypes
import os
import threading

from .errors import CoderDependencyError

LIB_NAME = "libgaans_w64.so"
ABI_VERSION = 14
CTRL_BYTES = 256
PLAN_BYTES = 1536  # GAANS_PLAN_BYTES
PHASE_SLOTS = 16  # GAANS_PHASE_SLOTS
# plan modes (GAANS_MODE_*)
MODE_SYMBOLS, MODE_LATENTS, MODE_GAUSSIAN = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 16 * 1024 * 1024  # GAANS_NOALLOC_SCRATCH_BYTES

# return codes
OK, EINVAL, ETABLE, EHIP = 0, 1, 2, 3
# device status bits
ST_RANGE = 0x01
ST_INDEX = 0x02
ST_HEADER = 0x04
ST_TABLES = 0x08
ST_CORRUPT = 0x10
ST_INDEXHASH = 0x20
ST_SIZE = 0x40
ST_TIMEOUT = 0x80

STATUS_TEXT = {
    ST_RANGE: "a symbol cannot be coded (escape value >= 2^32 or non-finite latent)",
    ST_INDEX: "indexes contain a value outside the CDF table range",
    ST_HEADER: "payload header is inconsistent with the decode call",
    ST_TABLES: "coding tables do not match the payload",
    ST_CORRUPT: "payload chunk offsets or rANS stream are corrupt",
    ST_INDEXHASH: "indexes do not match the payload",
    ST_SIZE: "payload would exceed the 4 GiB format limit",
    ST_TIMEOUT: "an encode unit gave up waiting for the units before it",
}


_LAYOUT_FIELDS = ("B", "N", "C", "P", "S", "HW", "K", "chunk_len", "U", "header_bytes",
                  "max_payload_bytes", "cap_words", "workspace_bytes", "ws_chunk_words",
                  "ws_chunk_status", "ws_index_hash", "ws_end_off", "ws_info", "ws_states",
                  "ws_words", "ws_esc", "ws_esc_raw", "ws_look")


class Layout(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int64) for name in _LAYOUT_FIELDS]


class LayoutInts:
    """``gaans_layout`` as plain Python ints (read without ctypes conversions)."""

    __slots__ = _LAYOUT_FIELDS

    def __init__(self, lay: Layout) -> None:
        for name in _LAYOUT_FIELDS:
            setattr(self, name, int(getattr(lay, name)))


class Tables(ctypes.Structure):
    """``gaans_tables``: descriptor of a prepared table blob."""

    _fields_ = [("dev", ctypes.c_void_p), ("bytes", ctypes.c_int64), ("M", ctypes.c_int32),
                ("max_nsym", ctypes.c_int32), ("total_nsym", ctypes.c_int64),
                ("digest", ctypes.c_uint64), ("max_dense", ctypes.c_int32),
                ("flags", ctypes.c_int32), ("total_dense", ctypes.c_int64),
                ("mean_bits", ctypes.c_float), ("max_wide", ctypes.c_int32),
                ("total_wide", ctypes.c_int64)]


class EncodeCall(ctypes.Structure):
    """``gaans_encode_call``: gaans_run_encode's arguments (gaans_run_encode_call)."""

    _fields_ = [("plan", ctypes.c_void_p), ("stream", ctypes.c_void_p),
                ("in0", ctypes.c_void_p), ("in1", ctypes.c_void_p), ("in2", ctypes.c_void_p),
                ("in3", ctypes.c_void_p), ("workspace_dev", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_int64), ("ctrl_dev", ctypes.c_void_p),
                ("out_dev", ctypes.c_void_p), ("out_bytes", ctypes.c_int64),
                ("info_host", ctypes.c_void_p)]


class DecodeCall(ctypes.Structure):
    """``gaans_decode_call``: gaans_run_decode's arguments (gaans_run_decode_call)."""

    _fields_ = [("plan", ctypes.c_void_p), ("stream", ctypes.c_void_p),
                ("payload_dev", ctypes.c_void_p), ("payload_bytes", ctypes.c_int64),
                ("in0", ctypes.c_void_p), ("in1", ctypes.c_void_p), ("in2", ctypes.c_void_p),
                ("out_dev", ctypes.c_void_p), ("ctrl_dev", ctypes.c_void_p),
                ("status_host", ctypes.c_void_p)]


# GAANS_PHASE_TIMES=1 selects the measurement build (kernels that record phase
# timestamps; csrc/build.py --phases), for bench.py --phases only
LIB_NAME_PHASES = "libgaans_w64_phases.so"


def library_path() -> str:
    name = LIB_NAME_PHASES if os.environ.get("GAANS_PHASE_TIMES") == "1" else LIB_NAME
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", name)


def library_available() -> bool:
    return os.path.exists(library_path())


_lib = None
_lock = threading.Lock()


def _declare(L) -> None:
    p, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    T = ctypes.POINTER(Tables)
    sig = {
        "gaans_abi_version": ([], ctypes.c_int),
        "gaans_last_error": ([], ctypes.c_char_p),
        "gaans_get_layout": ([i64, i64, i64, i64, i32, ctypes.POINTER(Layout)], ctypes.c_int),
        "gaans_choose_segments": ([T, i64, i64, i64, i64, ctypes.c_double, i64,
                                   ctypes.POINTER(ctypes.c_int32)], ctypes.c_int),
        "gaans_tables_bytes": ([p, p, i32, i32, ctypes.POINTER(ctypes.c_int64)], ctypes.c_int),
        "gaans_tables_prepare": ([p, p, p, i32, i32, p, i64, T], ctypes.c_int),
        "gaans_encode_symbols": ([p, p, p, T, i64, i64, i64, i64, i32, p, i64, p, p],
                                 ctypes.c_int),
        "gaans_encode_latents": ([p, p, p, p, T, i64, i64, i64, i64, i32, p, i64, p, p],
                                 ctypes.c_int),
        "gaans_encode_pack": ([p, p, i64, T, i64, i64, i64, i64, i32, p, i64], ctypes.c_int),
        "gaans_encode_symbols_noalloc": ([p, p, p, T, i64, i64, i64, i64, i32, p, i64, p],
                                         ctypes.c_int),
        "gaans_decode_symbols": ([p, p, i64, p, T, i64, i64, i64, i64, i32, p, p, p],
                                 ctypes.c_int),
        "gaans_decode_latents": ([p, p, i64, p, T, p, i64, i64, i64, i64, i32, p, p, p],
                                 ctypes.c_int),
        "gaans_encode_gaussian": ([p, p, p, p, p, i32, f32, T, i64, i64, i64, i64, i32, p, i64, p,
                                   p], ctypes.c_int),
        "gaans_decode_gaussian": ([p, p, i64, p, p, p, i32, f32, T, i64, i64, i64, i64, i32, p, p,
                                   p], ctypes.c_int),
        "gaans_rans64_decode": ([p, p, i64, p, p, T, i64, i64, i64, p, p, p], ctypes.c_int),
        "gaans_rans64_decode_host": ([p, p, p, p, p, p, i32, i32, i64, i64, i64, i32, p, p],
                                     ctypes.c_int),
        "gaans_wait_host_word": ([p, p], ctypes.c_int),
        "gaans_debug_phases": ([p, i64, ctypes.POINTER(ctypes.c_int32)], ctypes.c_int),
        # plans are passed by address (c_void_p): no byref object per call
        "gaans_plan_encode": ([T, i32, i32, i32, f32, i64, i64, i64, i64, i32, p], ctypes.c_int),
        "gaans_plan_decode": ([T, i32, i32, i32, f32, i64, i64, i64, i64, i32, p], ctypes.c_int),
        "gaans_run_encode": ([p, p, p, p, p, p, p, i64, p, p, i64, p], ctypes.c_int),
        "gaans_run_decode": ([p, p, p, i64, p, p, p, p, p, p], ctypes.c_int),
        "gaans_enqueue_encode": ([p, p, p, p, p, p, p, i64, p, p, i64, p], ctypes.c_int),
        "gaans_enqueue_decode": ([p, p, p, i64, p, p, p, p, p, p], ctypes.c_int),
        # struct addresses (c_void_p): one argument to convert per call
        "gaans_run_encode_call": ([p], ctypes.c_int),
        "gaans_run_decode_call": ([p], ctypes.c_int),
        "gaans_host_selftest": ([], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res


def lib():
    """Load the HIP library (once).  Raises CoderDependencyError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not os.path.exists(path):
                raise CoderDependencyError(
                    f"GA-ANS HIP library is not built ({path}); run __graft_entry__.build()")
            try:
                L = ctypes.CDLL(path)
                _declare(L)
            except (OSError, AttributeError) as exc:
                raise CoderDependencyError(f"GA-ANS HIP library could not be loaded: {exc}") from exc
            if L.gaans_abi_version() != ABI_VERSION:
                raise CoderDependencyError("GA-ANS HIP library ABI version mismatch")
            _lib = L
    return _lib


def wait_host_word(stream_ptr: int, word_ptr: int, what: str) -> None:
    """Wait for a launch's completion word in pinned host memory (the one
    host synchronisation of an encode or decode call)."""
    check(_lib.gaans_wait_host_word(stream_ptr, word_ptr), what)


def last_error() -> str:
    msg = lib().gaans_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Raise for a nonzero return code: bad arguments or tables
    (GAANS_EINVAL, GAANS_ETABLE) are the caller's inputs (CoderInputError, a
    ValueError); a HIP runtime failure (GAANS_EHIP: a failed launch or
    attribute call, or a stream that reported an error) is not, and raises
    CoderError (a RuntimeError)."""
    if rc != OK:
        from .errors import CoderError, CoderInputError

        cls = CoderInputError if rc in (EINVAL, ETABLE) else CoderError
        raise cls(f"{what} failed: {last_error()} (code {rc})")


_layouts: dict = {}


def layout(B: int, N: int, C: int, P: int, S: int = 1) -> LayoutInts:
    """``gaans_layout`` of B rows of N symbols, C channels, P per chunk and S
    segments per chunk (cached)."""
    key = (B, N, C, P, S)
    out = _layouts.get(key)
    if out is None:
        raw = Layout()
        check(lib().gaans_get_layout(B, N, C, P, S, ctypes.byref(raw)), "layout")
        out = LayoutInts(raw)
        if len(_layouts) > 256:
            _layouts.clear()
        _layouts[key] = out
    return out


def describe_status(status: int) -> str:
    parts = [text for bit, text in STATUS_TEXT.items() if status & bit]
    return "; ".join(parts) if parts else f"status 0x{status:x}"
