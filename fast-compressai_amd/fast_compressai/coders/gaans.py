"""Device-side GA-ANS engine: thin wrappers over the C ABI.

Per (device, stream) the engine keeps a control block (device memory, zeroed
once; every launch leaves it zeroed), a reusable workspace (zeroed when it
is allocated: the fused encode's look-back words must start at zero, and
every launch leaves them so), and two small pinned host buffers that the
kernels write the payload size / status into, and a completion word that
carries both.  The device orders calls on one stream; the pinned words are
also shared by the host threads that call on that stream, so a lock per
(device, stream) is held from a call's launch until its words are read.

Each shape gets a call plan (``gaans_plan_encode`` / ``gaans_plan_decode``:
layout, LDS plan, kernel variant and argument block, computed once and kept
with the prepared tables), so a call is one short C call.  Encode
(``gaans_run_encode``) enqueues one kernel that codes and packs into a
worst-case-sized buffer (each unit finds its payload offset by a decoupled
look-back over the units before it), then waits for the completion word
and reads the payload size; other units may still be writing their words
when encode returns, ordered before any later work on the stream.  Decode
(``gaans_run_decode``) enqueues one kernel and waits for its completion word
to read the status word.  Reference host APIs replaced:
``encode_with_indexes_warp_v2_cuda`` (``warp_ans_kernel_v2.cu:183-306``, two
syncs and six launches) and ``decode_with_indexes_warp_cuda``
(``warp_ans_kernel.cu:477-544``, one sync and four launches).
"""

from __future__ import annotations

import ctypes
import threading

import torch

from . import _native
from .errors import CoderInputError
from .tables import PreparedTables

CLONE_SLACK_BYTES = 32 << 20  # keep a view of the worst-case buffer below this waste


class _StreamState:
    def __init__(self, device: torch.device) -> None:
        self.ctrl = torch.zeros(_native.CTRL_BYTES, dtype=torch.uint8, device=device)
        self.info = torch.zeros(4, dtype=torch.int64, pin_memory=True)
        self.status = torch.zeros(4, dtype=torch.int32, pin_memory=True)
        self.info_np = self.info.numpy()      # host views of the pinned words
        self.status_np = self.status.numpy()
        self.info_done = self.info.data_ptr() + 16    # completion words
        self.status_done = self.status.data_ptr() + 4
        self.ctrl_ptr = self.ctrl.data_ptr()
        self.info_ptr = self.info.data_ptr()
        self.status_ptr = self.status.data_ptr()
        self.workspace = torch.zeros(0, dtype=torch.uint8, device=device)
        self.device = device
        self.lock = threading.Lock()

    def ws(self, nbytes: int) -> torch.Tensor:
        """The workspace, grown (and zeroed) when a shape needs more; the
        caller holds ``lock``."""
        if self.workspace.numel() < nbytes:
            self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        return self.workspace


_states: dict = {}
_states_lock = threading.Lock()


def _state(index: int, stream_ptr: int) -> _StreamState:
    key = (index, stream_ptr)
    st = _states.get(key)
    if st is None:
        with _states_lock:
            st = _states.get(key)
            if st is None:
                device = torch.device("cuda", index)
                with torch.cuda.device(device):
                    st = _StreamState(device)
                    torch.cuda.current_stream(device).synchronize()  # ctrl zeroed before use
                _states[key] = st
    return st


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _index(device) -> int:
    d = device if type(device) is torch.device else torch.device(device)
    return torch.cuda.current_device() if d.index is None else d.index


def _enter_device(index: int):
    """Make ``index`` the current device; returns the device to restore
    afterwards, or None when it already was current.  (The caller's tensors
    are on a GPU, so torch's device runtime is initialised and the current
    device is read directly.)"""
    cur = torch._C._cuda_getDevice()
    if cur == index:
        return None
    torch.cuda.set_device(index)
    return cur


def _check_gaussian(B: int, N: int, device, scale_table: torch.Tensor,
                    **per_element: torch.Tensor | None) -> None:
    """The Gaussian kernels read every per-element operand at B*N positions
    and the scale table whole: all fp32, contiguous, on the coder's device."""
    dev = torch.device("cuda", _index(device))
    for name, t in (("scale_table", scale_table), *per_element.items()):
        if t is None and name == "means":
            continue
        if (not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or t.device != dev
                or not t.is_contiguous()):
            raise CoderInputError(f"{name} must be a contiguous float32 tensor on {dev}")
        if name == "scale_table" and (t.ndim != 1 or t.numel() < 1):
            raise CoderInputError("scale_table must be a non-empty 1-D tensor")
        if name != "scale_table" and t.numel() != B * N:
            raise CoderInputError(f"{name} holds {t.numel()} values, expected {B * N}")


# bpp budget of the automatic segment count: the states and padding of the
# added coding units may cost up to this fraction of a chunk's expected payload
SEGMENT_BUDGET = 0.006


def _cu_count(device) -> int:
    index = _index(device)
    got = _cus.get(index)
    if got is None:
        got = int(torch.cuda.get_device_properties(index).multi_processor_count)
        _cus[index] = got
    return got


_cus: dict = {}


def choose_segments(tables: PreparedTables, B: int, N: int, C: int, P: int, device=None,
                    budget: float = SEGMENT_BUDGET, target_units: int | None = None) -> int:
    """Segments per chunk for a shape (``gaans_choose_segments``): enough
    coding units to give every CU of ``device`` one (``target_units``, by
    default its CU count), within ``budget`` of extra bytes (estimated from
    the tables' entropy) and the shape's limit."""
    if target_units is None:
        target_units = _cu_count(device if device is not None else torch.cuda.current_device())
    key = (tables.digest, B, N, C, P, budget, target_units)
    got = _segments.get(key)
    if got is None:
        out = ctypes.c_int32(0)
        _native.check(_native.lib().gaans_choose_segments(tables.ref, B, N, C, P, float(budget),
                                                          int(target_units), ctypes.byref(out)),
                      "segment choice")
        got = int(out.value)
        if len(_segments) > 1024:
            _segments.clear()
        _segments[key] = got
    return got


_segments: dict = {}


def resolve_segments(segments: int | None, tables: PreparedTables, B: int, N: int, C: int,
                     P: int, device=None) -> int:
    """``segments`` as given (validated by the layout), or the automatic
    choice for None."""
    if segments is None:
        return choose_segments(tables, B, N, C, P, device)
    if type(segments) is not int or segments < 1:
        raise CoderInputError("segments must be a positive int (or None for the automatic choice)")
    return segments


class EncodedChunks:
    """One encode's payload (uint8 ``packed``, header included) and the
    layout values a payload object records."""

    __slots__ = ("packed", "header_bytes", "chunk_len", "K", "segments", "batch")

    def __init__(self, packed: torch.Tensor, header_bytes: int, chunk_len: int, K: int,
                 segments: int = 1, batch: int = 1) -> None:
        self.packed = packed
        self.header_bytes = header_bytes
        self.chunk_len = chunk_len
        self.K = K
        self.segments = segments
        self.batch = batch

    @property
    def chunk_ends(self) -> torch.Tensor:
        """uint32 [B, K S] view of the header's unit end offsets."""
        units = self.K * self.segments
        return self.packed[64: 64 + 4 * self.batch * units].view(torch.uint32).view(
            self.batch, units)


def layout(B: int, N: int, C: int, P: int, S: int) -> "_native.LayoutInts":
    """The coding layout of a shape (cached)."""
    return _native.layout(B, N, C, P, S)


def _plan(tables: PreparedTables, decode: bool, mode: int, explicit: bool, B: int, N: int,
          C: int, P: int, S: int, index: int, n_scales: int = 0, bound: float = 0.0):
    """The call plan (``gaans_plan_encode`` / ``gaans_plan_decode``) of a
    shape, cached on the tables it refers to (so it never outlives their
    blob); made with device ``index`` current.  Returns (plan buffer, its
    address, layout)."""
    key = (decode, mode, explicit, B, N, C, P, S, index, n_scales, bound)
    got = tables.plans.get(key)
    if got is None:
        L = _native.lib()
        lay = _native.layout(B, N, C, P, S)
        buf = (ctypes.c_uint64 * (_native.PLAN_BYTES // 8))()
        make = L.gaans_plan_decode if decode else L.gaans_plan_encode
        _native.check(make(tables.ref, mode, int(explicit), n_scales, bound, B, N, C, P, S,
                           ctypes.addressof(buf)), "GA-ANS plan")
        got = (buf, ctypes.addressof(buf), lay)
        if len(tables.plans) > 64:
            tables.plans.clear()
        tables.plans[key] = got
    return got


def _run_encode_raw(tables: PreparedTables, mode: int, explicit: bool, B: int, N: int, C: int,
                    P: int, S: int, device, in0: int, in1, in2, in3, what: str,
                    n_scales: int = 0, bound: float = 0.0):
    """Plan (cached), enqueue coding + pack into a worst-case buffer and wait
    for the completion word.  Returns (buffer, payload bytes, layout): the
    payload is the buffer's first bytes."""
    index = _index(device)
    prev = _enter_device(index)
    try:
        _, plan, lay = _plan(tables, False, mode, explicit, B, N, C, P, S, index, n_scales, bound)
        sp = torch._C._cuda_getCurrentRawStream(index)
        st = _state(index, sp)
        out = torch.empty(lay.max_payload_bytes, dtype=torch.uint8, device=st.device)
        with st.lock:
            ws = st.ws(lay.workspace_bytes)
            rc = _native.lib().gaans_run_encode(plan, sp, in0, in1, in2, in3, ws.data_ptr(),
                                                ws.numel(), st.ctrl_ptr, out.data_ptr(),
                                                lay.max_payload_bytes, st.info_ptr)
            word = int(st.info_np[2])  # 1 | status << 1 | payload bytes << 16
        if rc:
            _native.check(rc, what)
    finally:
        if prev is not None:
            torch.cuda.set_device(prev)
    total, status = word >> 16, (word >> 1) & 0x7FFF
    if status:
        raise CoderInputError(f"GA-ANS encode failed: {_native.describe_status(status)}")
    return out, total, lay


def _run_encode(tables: PreparedTables, mode: int, explicit: bool, B: int, N: int, C: int,
                P: int, S: int, device, in0: int, in1, in2, in3, what: str,
                n_scales: int = 0, bound: float = 0.0) -> EncodedChunks:
    """``_run_encode_raw`` with the payload sliced out of the buffer (copied
    when the buffer would waste more than CLONE_SLACK_BYTES)."""
    out, total, lay = _run_encode_raw(tables, mode, explicit, B, N, C, P, S, device, in0, in1,
                                      in2, in3, what, n_scales, bound)
    packed = out[:total]
    if lay.max_payload_bytes - total > CLONE_SLACK_BYTES:
        packed = packed.clone()
    return EncodedChunks(packed, lay.header_bytes, lay.chunk_len, lay.K, S, B)


def _run_decode(tables: PreparedTables, mode: int, explicit: bool, B: int, N: int, C: int,
                P: int, S: int, device, packed: torch.Tensor, in0, in1, in2,
                dtype: torch.dtype, what: str, n_scales: int = 0,
                bound: float = 0.0) -> torch.Tensor:
    return _run_decode_ptr(tables, mode, explicit, B, N, C, P, S, device, packed.data_ptr(),
                           packed.numel(), in0, in1, in2, dtype, what, n_scales, bound)


def _run_decode_ptr(tables: PreparedTables, mode: int, explicit: bool, B: int, N: int, C: int,
                    P: int, S: int, device, payload_ptr: int, payload_bytes: int, in0, in1,
                    in2, dtype: torch.dtype, what: str, n_scales: int = 0,
                    bound: float = 0.0) -> torch.Tensor:
    """Decode the payload of ``payload_bytes`` bytes at device address
    ``payload_ptr`` (on ``device``) with the shape's plan; waits for the
    completion word."""
    index = _index(device)
    prev = _enter_device(index)
    try:
        _, plan, _lay = _plan(tables, True, mode, explicit, B, N, C, P, S, index, n_scales, bound)
        sp = torch._C._cuda_getCurrentRawStream(index)
        st = _state(index, sp)
        out = torch.empty((B, N), dtype=dtype, device=st.device)
        with st.lock:
            rc = _native.lib().gaans_run_decode(plan, sp, payload_ptr, payload_bytes, in0,
                                                in1, in2, out.data_ptr(), st.ctrl_ptr,
                                                st.status_ptr)
            status = int(st.status_np[1]) >> 1  # 1 | status << 1
        if rc:
            _native.check(rc, what)
    finally:
        if prev is not None:
            torch.cuda.set_device(prev)
    if status:
        raise CoderInputError(f"warp_div decode failed: {_native.describe_status(status)}")
    return out


class _Call:
    """A symbols-mode call context on one stream of one device (cached on the
    tables per shape and stream): the plan, its sizes and stream state, and
    the argument struct of gaans_run_encode_call / _decode_call with the
    fields that do not change from call to call already set."""

    __slots__ = ("plan_buf", "max_bytes", "ws_bytes", "st", "args", "addr", "run", "ws")

    def __init__(self, tables: PreparedTables, decode: bool, explicit: bool, B: int, N: int,
                 C: int, P: int, S: int, index: int, sp: int) -> None:
        self.plan_buf, plan, lay = _plan(tables, decode, _native.MODE_SYMBOLS, explicit, B, N, C,
                                         P, S, index)
        self.max_bytes = lay.max_payload_bytes
        self.ws_bytes = lay.workspace_bytes
        self.st = st = _state(index, sp)
        L = _native.lib()
        if decode:
            self.args = _native.DecodeCall(plan=plan, stream=sp, ctrl_dev=st.ctrl_ptr,
                                           status_host=st.status_ptr)
            self.run = L.gaans_run_decode_call
        else:
            self.args = _native.EncodeCall(plan=plan, stream=sp, ctrl_dev=st.ctrl_ptr,
                                           out_bytes=lay.max_payload_bytes,
                                           info_host=st.info_ptr)
            self.run = L.gaans_run_encode_call
        self.addr = ctypes.addressof(self.args)
        self.ws = None  # the workspace tensor whose address the struct holds


def _symbols_call(tables: PreparedTables, decode: bool, explicit: bool, B: int, N: int, C: int,
                  P: int, S: int, index: int, sp: int) -> _Call:
    """The call context of a symbols-mode call on stream ``sp`` of device
    ``index`` (current)."""
    key = ("call", decode, explicit, B, N, C, P, S, index, sp)
    ctx = tables.plans.get(key)
    if ctx is None:
        ctx = _Call(tables, decode, explicit, B, N, C, P, S, index, sp)
        tables.plans[key] = ctx
    return ctx


def encode_symbols_raw(tables: PreparedTables, B: int, N: int, C: int, P: int, device,
                       symbols: torch.Tensor, indexes: torch.Tensor | None, segments: int):
    """``encode`` of int32 symbols, returning (worst-case buffer, payload
    bytes): the payload is the buffer's first bytes (no slice made).  With
    the device current, one cached lookup gives the plan and stream state."""
    index = device.index
    if index is None or torch._C._cuda_getDevice() != index:
        out, total, _ = _run_encode_raw(tables, _native.MODE_SYMBOLS, indexes is not None, B, N,
                                        C, P, segments, device, symbols.data_ptr(),
                                        _ptr(indexes), None, None, "GA-ANS encode")
        return out, total
    sp = torch._C._cuda_getCurrentRawStream(index)
    c = _symbols_call(tables, False, indexes is not None, B, N, C, P, segments, index, sp)
    st = c.st
    out = torch.empty(c.max_bytes, dtype=torch.uint8, device=st.device)
    with st.lock:
        a = c.args
        ws = st.ws(c.ws_bytes)
        if ws is not c.ws:
            a.workspace_dev = ws.data_ptr()
            a.workspace_bytes = ws.numel()
            c.ws = ws
        a.in0 = symbols.data_ptr()
        a.in1 = None if indexes is None else indexes.data_ptr()
        a.out_dev = out.data_ptr()
        rc = c.run(c.addr)
        word = int(st.info_np[2])  # 1 | status << 1 | payload bytes << 16
    if rc:
        _native.check(rc, "GA-ANS encode")
    status = (word >> 1) & 0x7FFF
    if status:
        raise CoderInputError(f"GA-ANS encode failed: {_native.describe_status(status)}")
    return out, word >> 16


def decode_symbols_ptr(payload_ptr: int, payload_bytes: int, tables: PreparedTables, B: int,
                       N: int, C: int, P: int, device, indexes: torch.Tensor | None,
                       segments: int) -> torch.Tensor:
    """``decode`` of int32 symbols from a payload given by device address and
    size (the cached call context of ``encode_symbols_raw``)."""
    index = device.index
    if index is None or torch._C._cuda_getDevice() != index:
        return _run_decode_ptr(tables, _native.MODE_SYMBOLS, indexes is not None, B, N, C, P,
                               segments, device, payload_ptr, payload_bytes, _ptr(indexes), None,
                               None, torch.int32, "GA-ANS decode")
    sp = torch._C._cuda_getCurrentRawStream(index)
    c = _symbols_call(tables, True, indexes is not None, B, N, C, P, segments, index, sp)
    st = c.st
    out = torch.empty((B, N), dtype=torch.int32, device=st.device)
    with st.lock:
        a = c.args
        a.payload_dev = payload_ptr
        a.payload_bytes = payload_bytes
        a.in0 = None if indexes is None else indexes.data_ptr()
        a.out_dev = out.data_ptr()
        rc = c.run(c.addr)
        status = int(st.status_np[1]) >> 1  # 1 | status << 1
    if rc:
        _native.check(rc, "GA-ANS decode")
    if status:
        raise CoderInputError(f"warp_div decode failed: {_native.describe_status(status)}")
    return out


def encode(tables: PreparedTables, B: int, N: int, C: int, P: int, device, *,
           symbols: torch.Tensor | None = None, indexes: torch.Tensor | None = None,
           y: torch.Tensor | None = None, medians: torch.Tensor | None = None,
           segments: int = 1) -> EncodedChunks:
    """Encode int32 ``symbols`` [B, N], or fp32 latents ``y`` with per-channel
    ``medians`` (quantize fused).  ``indexes`` None means channel-major
    tables; ``segments`` coding units per chunk."""
    if y is not None:
        return _run_encode(tables, _native.MODE_LATENTS, indexes is not None, B, N, C, P,
                           segments, device, y.data_ptr(), medians.data_ptr(), _ptr(indexes),
                           None, "GA-ANS encode")
    return _run_encode(tables, _native.MODE_SYMBOLS, indexes is not None, B, N, C, P, segments,
                       device, symbols.data_ptr(), _ptr(indexes), None, None, "GA-ANS encode")


def decode(packed: torch.Tensor, tables: PreparedTables, B: int, N: int, C: int, P: int,
           device, *, indexes: torch.Tensor | None = None,
           medians: torch.Tensor | None = None, segments: int = 1) -> torch.Tensor:
    """Decode to int32 symbols [B, N], or (``medians`` given) to fp32 y_hat
    [B, N] with dequantize fused; ``segments`` as recorded in the payload."""
    if medians is not None:
        return _run_decode(tables, _native.MODE_LATENTS, indexes is not None, B, N, C, P,
                           segments, device, packed, medians.data_ptr(), _ptr(indexes), None,
                           torch.float32, "GA-ANS decode")
    return _run_decode(tables, _native.MODE_SYMBOLS, indexes is not None, B, N, C, P, segments,
                       device, packed, _ptr(indexes), None, None, torch.int32, "GA-ANS decode")


def encode_gaussian(tables: PreparedTables, B: int, N: int, C: int, P: int, device, *,
                    y: torch.Tensor, scales: torch.Tensor, scale_table: torch.Tensor,
                    scale_bound: float, means: torch.Tensor | None = None,
                    segments: int = 1) -> EncodedChunks:
    """GaussianConditional encode with index building and quantize fused:
    fp32 ``y``, ``scales`` (and ``means``) [B, N] channel-major; ``scale_table``
    fp32 on the device, non-decreasing, one entry per table."""
    _check_gaussian(B, N, device, scale_table, y=y, scales=scales, means=means)
    return _run_encode(tables, _native.MODE_GAUSSIAN, True, B, N, C, P, segments, device,
                       y.data_ptr(), _ptr(means), scales.data_ptr(), scale_table.data_ptr(),
                       "GA-ANS Gaussian encode", scale_table.numel(), float(scale_bound))


def decode_gaussian(packed: torch.Tensor, tables: PreparedTables, B: int, N: int, C: int, P: int,
                    device, *, scales: torch.Tensor, scale_table: torch.Tensor,
                    scale_bound: float, means: torch.Tensor | None = None,
                    segments: int = 1) -> torch.Tensor:
    """GaussianConditional decode with index building and dequantize fused:
    fp32 y_hat [B, N] = fp32(symbol) + mean (fp32(symbol) without means)."""
    _check_gaussian(B, N, device, scale_table, scales=scales, means=means)
    return _run_decode(tables, _native.MODE_GAUSSIAN, True, B, N, C, P, segments, device, packed,
                       scales.data_ptr(), _ptr(means), scale_table.data_ptr(), torch.float32,
                       "GA-ANS Gaussian decode", scale_table.numel(), float(scale_bound))


def decode_rans64(streams: torch.Tensor, offsets: torch.Tensor, tables: PreparedTables, B: int,
                  N: int, C: int, device, *, indexes: torch.Tensor | None = None) -> torch.Tensor:
    """Decode B CompressAI Rans64 streams (uint8 ``streams`` on the device,
    stream b at bytes ``[offsets[b], offsets[b + 1])``, int64 ``offsets``)
    into int32 symbols [B, N]; ``indexes`` None means table = channel."""
    L = _native.lib()
    dev = torch.device("cuda", _index(device))
    if (streams.dtype != torch.uint8 or streams.device != dev or not streams.is_contiguous()
            or offsets.dtype != torch.int64 or offsets.device != dev
            or not offsets.is_contiguous() or offsets.numel() != B + 1):
        raise CoderInputError("streams must be uint8 and offsets int64 [B + 1], contiguous, "
                              f"on {dev}")
    if indexes is not None and (indexes.dtype != torch.int32 or indexes.device != dev
                                or not indexes.is_contiguous() or indexes.numel() != B * N):
        raise CoderInputError(f"indexes must be a contiguous int32 [B, N] tensor on {dev}")
    index = dev.index
    prev = _enter_device(index)
    try:
        sp = torch._C._cuda_getCurrentRawStream(index)
        st = _state(index, sp)
        out = torch.empty((B, N), dtype=torch.int32, device=dev)
        with st.lock:
            st.status_np[1] = 0
            rc = L.gaans_rans64_decode(sp, streams.data_ptr() if streams.numel() else None,
                                       streams.numel(), offsets.data_ptr(), _ptr(indexes),
                                       tables.ref, B, N, C, out.data_ptr(), st.ctrl_ptr,
                                       st.status_ptr)
            if rc == 0:
                rc = L.gaans_wait_host_word(sp, st.status_done)
            status = int(st.status_np[1]) >> 1
        if rc:
            _native.check(rc, "Rans64 decode")
    finally:
        if prev is not None:
            torch.cuda.set_device(prev)
    if status:
        raise CoderInputError(f"Rans64 decode failed: {_native.describe_status(status)}")
    return out


def decode_compressai_strings(strings, prepared: PreparedTables, raw_tables, B: int, N: int,
                              C: int, device, *,
                              indexes: torch.Tensor | None = None) -> torch.Tensor:
    """int32 symbols [B, N] on ``device`` of B CompressAI Rans64 strings (one
    per image), decoded where ``rans_host.rans64_route`` says is faster: this
    library's host decoder (streams over the host's threads) for batches too
    small for the GPU, else the GPU Rans64 decoder.  ``raw_tables`` are the
    CompressAI tables (cdfs, lengths, offsets) for the host decoder;
    ``indexes`` None means table = channel."""
    from .rans_host import decode_rows_host, rans64_route

    if rans64_route(len(strings)) == "host":
        idx = None if indexes is None else indexes.reshape(B, N)
        out = decode_rows_host(strings, idx, *raw_tables, N=N, C=C)
        return torch.from_numpy(out).to(device)
    buf, offs = pack_streams(strings, device)
    return decode_rans64(buf, offs, prepared, B, N, C, device, indexes=indexes)


def pack_streams(strings, device) -> tuple[torch.Tensor, torch.Tensor]:
    """CompressAI per-image byte strings -> (uint8 device buffer, int64
    offsets [B + 1]), each stream starting on a 4-byte boundary."""
    import numpy as np

    if not strings or not all(isinstance(s, (bytes, bytearray)) for s in strings):
        raise CoderInputError("expected a non-empty list of CompressAI byte strings")
    sizes = [len(s) for s in strings]
    if any(n % 4 for n in sizes):
        raise CoderInputError("a Rans64 stream is a whole number of 32-bit words")
    offs = np.zeros(len(strings) + 1, dtype=np.int64)
    np.cumsum(sizes, out=offs[1:])
    buf = np.frombuffer(b"".join(bytes(s) for s in strings), dtype=np.uint8)
    dev = torch.device(device)
    return (torch.from_numpy(buf.copy()).to(dev, non_blocking=False),
            torch.from_numpy(offs).to(dev, non_blocking=False))
