"""GPU decode of CompressAI Rans64 bitstreams (``gaans_rans64_decode``).

CompressAI is not installed, so the streams come from the oracle's
CompressAI-equivalent Rans64 encoder (``oracle.rans64_encode``, pinned by
hand-derived known answers in test_oracle.py); decoded symbols must equal the
encoded ones and ``oracle.rans64_decode``'s, bit for bit.  Covers the three
table modes of the kernel (all tables in LDS, one channel's table at a time,
global lookups), one stream per wave and several (batches larger than the
GPU's SIMD count), short rows, escape-heavy rows with extreme values, corrupt streams, and
``FastModel.decompress`` of CompressAI-format strings for the FactorizedPrior
and hyperprior stand-ins.
"""

import numpy as np
import pytest
import torch

import fast_compressai
import oracle as O
from fast_compressai import synthetic
from fast_compressai.coders import CoderInputError, gaans
from fast_compressai.coders.tables import prepare_tables
from factorized_stub import FactorizedPrior
from hyperprior_stub import make_hyperprior, reference_y_hat

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def encode_rows(symbols, indexes, cdfs, sizes, offsets):
    return [O.rans64_encode(symbols[b], indexes[b], cdfs, sizes, offsets)
            for b in range(symbols.shape[0])]


def gpu_decode(streams, cdfs, sizes, offsets, B, N, C, device, indexes=None):
    tables = prepare_tables(dev(cdfs, device), dev(sizes, device), dev(offsets, device))
    buf, offs = gaans.pack_streams(streams, device)
    idx = None if indexes is None else dev(indexes.astype(np.int32), device)
    return gaans.decode_rans64(buf, offs, tables, B, N, C, device, indexes=idx).cpu().numpy()


def factorized_rows(B, C, H, W, M_tables, seed, max_cdf=64, scale_hi=8.0):
    w = synthetic._factorized("rows", B, C, H, W, 0.1, scale_hi, max_cdf, 1, (16 * H, 16 * W),
                              seed)
    assert w.cdfs.shape[0] == M_tables
    return w


@pytest.mark.parametrize("B,C,H,W,implicit", [
    (1, 192, 32, 48, True),    # 192 tables: one channel's table at a time
    (3, 192, 32, 48, False),   # 192 tables, explicit indexes: global lookups
    (70, 12, 5, 7, True),      # 12 tables: all in LDS; two workgroups
    (65, 12, 3, 11, False),    # all in LDS, explicit indexes
    (2, 4, 1, 1, True),        # 4 symbols per row
    (1100, 4, 3, 3, True),     # more rows than SIMDs: two or more streams per wave
    (2100, 12, 2, 3, False),
])
def test_factorized_rows_match_oracle(gpu_device, B, C, H, W, implicit):
    w = factorized_rows(B, C, H, W, C, seed=B + C)
    idx = w.explicit_indexes()
    streams = encode_rows(w.symbols, idx, w.cdfs, w.cdf_sizes, w.offsets)
    say("case: rans64 factorized", (B, C, H, W), "implicit", implicit)
    got = gpu_decode(streams, w.cdfs, w.cdf_sizes, w.offsets, B, C * H * W, C, gpu_device,
                     None if implicit else idx)
    assert np.array_equal(got, w.symbols)
    ref = np.stack([O.rans64_decode(s, idx[b], w.cdfs, w.cdf_sizes, w.offsets)
                    for b, s in enumerate(streams)])
    assert np.array_equal(got, ref)


def test_hyperprior_y_rows_match_oracle(gpu_device):
    yw, _, _, _ = synthetic.hyperprior_512x768()
    idx = yw.explicit_indexes()
    streams = encode_rows(yw.symbols, idx, yw.cdfs, yw.cdf_sizes, yw.offsets)
    say("case: rans64 hyperprior y, 64 Gaussian tables")
    got = gpu_decode(streams, yw.cdfs, yw.cdf_sizes, yw.offsets, 1, yw.n, yw.channels,
                     gpu_device, idx)
    assert np.array_equal(got, yw.symbols)


def escape_case(B=3, N=200, seed=5):
    rng = np.random.default_rng(seed)
    # 3 tables of 2..4 symbols (escape bin last), offsets around 0
    cdfs = np.array([[0, 65536, 0, 0], [0, 30000, 65536, 0], [0, 20000, 40000, 65536]], np.int32)
    sizes = np.array([2, 3, 4], np.int32)
    offsets = np.array([0, -1, 5], np.int32)
    idx = rng.integers(0, 3, size=(B, N), dtype=np.int32)
    sym = rng.integers(-3, 9, size=(B, N), dtype=np.int32)
    # the one-symbol table (offset 0) codes every int32 as an escape
    extremes = np.array([2**31 - 1, -2**31, 2**31 - 7, -2**31 + 6, 123456789, -98765432, 0, 7],
                        np.int32)
    sym[0, :extremes.size] = extremes
    idx[0, :extremes.size] = 0
    sym[1, -extremes.size:] = extremes[::-1]
    idx[1, -extremes.size:] = 0
    # table 2 (offset 5, escape bin 2): the largest magnitudes it can code
    sym[B - 1, :4] = [2**31 - 1, -2**31 + 5, 2**30, -2**30]
    idx[B - 1, :4] = 2
    return cdfs, sizes, offsets, idx, sym


def test_escape_heavy_rows_with_extreme_values(gpu_device):
    cdfs, sizes, offsets, idx, sym = escape_case()
    streams = encode_rows(sym, idx, cdfs, sizes, offsets)
    say("case: rans64 escapes")
    got = gpu_decode(streams, cdfs, sizes, offsets, sym.shape[0], sym.shape[1], 1, gpu_device,
                     idx)
    assert np.array_equal(got, sym)


def test_corrupt_and_bad_inputs_rejected(gpu_device):
    cdfs, sizes, offsets, idx, sym = escape_case(B=2, N=120)
    streams = encode_rows(sym, idx, cdfs, sizes, offsets)
    B, N = sym.shape
    say("case: rans64 truncated stream")
    with pytest.raises(CoderInputError, match="corrupt|stream"):
        gpu_decode([streams[0], streams[1][:8]], cdfs, sizes, offsets, B, N, 1, gpu_device, idx)
    say("case: rans64 stream shorter than its state")
    with pytest.raises(CoderInputError):
        gpu_decode([streams[0], b"\0\0\0\0"], cdfs, sizes, offsets, B, N, 1, gpu_device, idx)
    say("case: rans64 index out of range")
    bad = idx.copy()
    bad[1, 17] = 3
    with pytest.raises(CoderInputError, match="index"):
        gpu_decode(streams, cdfs, sizes, offsets, B, N, 1, gpu_device, bad)
    with pytest.raises(CoderInputError, match="32-bit words"):
        gaans.pack_streams([streams[0][:-1]], gpu_device)
    tables = prepare_tables(dev(cdfs, gpu_device), dev(sizes, gpu_device),
                            dev(offsets, gpu_device))
    buf, offs = gaans.pack_streams(streams, gpu_device)
    with pytest.raises(CoderInputError, match="offsets"):
        gaans.decode_rans64(buf, offs[:2], tables, B, N, 1, gpu_device)
    # offsets outside the buffer are reported, not read
    wild = torch.tensor([0, len(streams[0]), 1 << 40], dtype=torch.int64, device=gpu_device)
    with pytest.raises(CoderInputError):
        gaans.decode_rans64(buf, wild, tables, B, N, 1, gpu_device,
                            indexes=dev(idx, gpu_device))


def test_factorized_decompress_of_compressai_strings(gpu_device):
    M = 12
    torch.manual_seed(7)
    w = synthetic.coder_512x768(seed=7)
    med = np.random.default_rng(7).normal(0, 0.2, M).astype(np.float32)
    model = FactorizedPrior(M, w.cdfs[:M], w.cdf_sizes[:M], w.offsets[:M], med).eval()
    fast = fast_compressai.accelerate(model, P=4, device=str(gpu_device))
    x = torch.rand(3, 3, 64, 96, device=gpu_device)
    eb = fast.model.entropy_bottleneck
    with torch.no_grad():
        y = fast.model.g_a(x)
        m4 = eb._extend_ndims(eb._get_medians().detach(), 2)
        symbols = eb.quantize(y, "symbols", m4.expand(3, -1, -1, -1))
        x_ref = fast.model.g_s(eb.dequantize(symbols, m4.expand(3, -1, -1, -1))).clamp_(0, 1)
    sym = symbols.reshape(3, -1).cpu().numpy()
    chan = np.repeat(np.arange(M, dtype=np.int32), y.shape[2] * y.shape[3])[None].repeat(3, 0)
    # what CompressAI's EntropyBottleneck.compress returns: one string per image
    strings = encode_rows(sym, chan, w.cdfs[:M], w.cdf_sizes[:M], w.offsets[:M])
    say("case: FastModel.decompress of CompressAI FactorizedPrior strings")
    out = fast.decompress([strings], tuple(y.shape[-2:]))
    assert torch.equal(out["x_hat"], x_ref)
    # and the same image through the GA-ANS payload path
    ga = fast.compress(x)
    assert torch.equal(fast.decompress(ga["strings"], ga["shape"])["x_hat"], x_ref)


@pytest.mark.parametrize("mean_scale", [True, False])
def test_hyperprior_decompress_of_compressai_strings(gpu_device, mean_scale):
    model = make_hyperprior(mean_scale).to(gpu_device)
    x = torch.rand(2, 3, 64, 64, device=gpu_device)
    y, z, z_hat, scales, means, symbols, indexes, y_hat = reference_y_hat(model, x)
    with torch.no_grad():
        x_ref = model.g_s(y_hat).clamp_(0, 1)
    eb, gc = model.entropy_bottleneck, model.gaussian_conditional
    B = x.size(0)
    med = eb._get_medians().detach().reshape(1, -1, 1, 1)
    zs = torch.round(z - med).int().reshape(B, -1).cpu().numpy()
    zc = np.repeat(np.arange(z.size(1), dtype=np.int32), z.size(2) * z.size(3))[None].repeat(B, 0)
    z_strings = encode_rows(zs, zc, eb._quantized_cdf.cpu().numpy(),
                            eb._cdf_length.cpu().numpy(), eb._offset.cpu().numpy())
    y_strings = encode_rows(symbols.reshape(B, -1).cpu().numpy(),
                            indexes.reshape(B, -1).cpu().numpy(), gc._quantized_cdf.cpu().numpy(),
                            gc._cdf_length.cpu().numpy(), gc._offset.cpu().numpy())
    fast = fast_compressai.accelerate(model, P=4, device=str(gpu_device))
    say("case: FastModel.decompress of CompressAI hyperprior strings, mean_scale", mean_scale)
    out = fast.decompress([y_strings, z_strings], tuple(z.shape[-2:]))
    assert torch.equal(out["x_hat"], x_ref)
