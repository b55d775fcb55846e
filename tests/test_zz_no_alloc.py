"""The no-allocation encode entry point (gaans_encode_symbols_noalloc, one
fused encode+pack kernel over a static device scratch): its payload bytes
equal those of the workspace encode and of the oracle on two calls in a row
(the second with a smaller input, so that stale scratch contents from the
first would show); shapes beyond its static scratch and payload buffers
below the shape's worst case are rejected before any device work."""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from fast_compressai import synthetic
from fast_compressai.coders import _native, gaans
from fast_compressai.coders.tables import prepare_tables


def _noalloc(L, tables, sym, idx, B, N, C, P, S, dev):
    lay = _native.layout(B, N, C, P, S)
    out = torch.zeros(lay.max_payload_bytes, dtype=torch.uint8, device=dev)
    info = torch.zeros(4, dtype=torch.int64, device=dev)
    sp = torch.cuda.current_stream(dev).cuda_stream
    rc = L.gaans_encode_symbols_noalloc(sp, sym.data_ptr(), None if idx is None else idx.data_ptr(),
                                        tables.ref, B, N, C, P, S, out.data_ptr(), out.numel(),
                                        info.data_ptr())
    _native.check(rc, "no-allocation encode")
    torch.cuda.synchronize(dev)
    total, status = int(info[0].item()), int(info[1].item())
    word = int(info[2].item())
    assert word & 1 and (word >> 16) == total and ((word >> 1) & 0x7FFF) == status
    return out[:total].cpu().numpy().tobytes(), status


@pytest.mark.gpu
def test_noalloc_matches_workspace_encode_twice(gpu_device):
    dev = gpu_device
    L = _native.lib()
    big = synthetic.coder_512x768(seed=3, p_ch=4)           # 1x192x32x48, explicit indexes
    small = synthetic.coder_512x768(seed=4, p_ch=5)          # then 12 channels of it
    cases = [
        ("1x192x32x48 P=4 explicit indexes", big, big.symbols, big.explicit_indexes(), 192, 4, 1),
        ("1x12x32x48 P=5 implicit indexes, 3 segments per chunk", small,
         small.symbols[:, :12 * 1536], None, 12, 5, 3),
    ]
    for name, w, sym_np, idx_np, C, P, S in cases:
        print("case: no-alloc encode", name, flush=True)
        M = C if idx_np is None else w.cdfs.shape[0]
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        tables = prepare_tables(t(w.cdfs[:M]), t(w.cdf_sizes[:M]), t(w.offsets[:M]))
        B, N = sym_np.shape
        sym = t(sym_np)
        idx = None if idx_np is None else t(idx_np)
        got, status = _noalloc(L, tables, sym, idx, B, N, C, P, S, dev)
        assert status == 0
        ref = gaans.encode(tables, B, N, C, P, dev, symbols=sym, indexes=idx, segments=S)
        assert got == ref.packed.cpu().numpy().tobytes()
        want = oracle.gaans_encode(sym_np, idx_np, w.cdfs[:M], w.cdf_sizes[:M], w.offsets[:M], P,
                                   channels=C, segments=S)
        assert got == want


def test_noalloc_rejects_shapes_beyond_its_scratch():
    L = _native.lib()
    B, N, C, P = 64, 192 * 1536, 192, 16  # about 113 MB of workspace
    lay = _native.layout(B, N, C, P, 1)
    assert lay.workspace_bytes + _native.CTRL_BYTES > _native.NOALLOC_SCRATCH_BYTES
    desc = _native.Tables()
    rc = L.gaans_encode_symbols_noalloc(None, None, None, ctypes.byref(desc), B, N, C, P, 1, None,
                                        0, None)
    assert rc == _native.EINVAL
    msg = _native.last_error()
    assert "scratch" in msg and str(_native.NOALLOC_SCRATCH_BYTES) in msg


def test_noalloc_rejects_a_payload_buffer_below_the_worst_case():
    """Each unit writes at the offset its look-back finds, before the
    launch's size is known: a buffer below the worst case could be
    overrun, so it is refused (GAANS_EINVAL) with no device work."""
    L = _native.lib()
    B, N, C, P = 1, 192 * 1536, 192, 4
    lay = _native.layout(B, N, C, P, 1)
    desc = _native.Tables()
    info = (ctypes.c_uint64 * 4)()
    for nbytes in (lay.header_bytes, lay.max_payload_bytes - 1):
        rc = L.gaans_encode_symbols_noalloc(None, None, None, ctypes.byref(desc), B, N, C, P, 1,
                                            ctypes.addressof(info), nbytes, ctypes.addressof(info))
        assert rc == _native.EINVAL
        assert "worst case" in _native.last_error()
