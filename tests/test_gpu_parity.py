"""GPU parity of the HIP GA-ANS coder against the CPU oracle, through the
C ABI (via WarpDivBackend / the engine).  Bar: payload bytes identical to
oracle/gaans_oracle.c, decoded symbols identical to the input, fused
quantize/dequantize identical to CompressAI's closed forms."""

import math
from dataclasses import replace

import numpy as np
import pytest
import torch

import oracle as O
from fast_compressai import synthetic
from fast_compressai.coders import CoderInputError, WarpDivBackend, WarpDivPayload, gaans
from fast_compressai.coders.tables import prepare_tables

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def backend(gpu_device):
    return WarpDivBackend()


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def tables_on(w, device):
    return dev(w.cdfs, device), dev(w.cdf_sizes, device), dev(w.offsets, device)


def max_segments(w, channels=None):
    """The most segments per chunk a workload's shape allows (one step each
    in a row's last chunk)."""
    C = w.channels if channels is None else channels
    N = w.symbols.shape[1]
    cl = w.p_ch * (N // C)
    K = -(-C // w.p_ch)
    return min(256, -(-(N - (K - 1) * cl) // 64))


def check_workload(backend, device, w, channels=None, bytes_check=True, segments=None):
    if segments is not None:
        segments = min(segments, max_segments(w, channels))
    say("case:", w.name, "P =", w.p_ch, "shape", w.symbols.shape, "segments", segments)
    sym = dev(w.symbols, device)
    idx = dev(w.explicit_indexes(), device)
    cdfs, sizes, offs = tables_on(w, device)
    payload = backend.encode(sym, idx, cdfs, sizes, offs, p_ch=w.p_ch, channels=channels,
                             segments=segments)
    torch.cuda.synchronize()
    if segments is not None:
        assert payload.segments == segments
    if bytes_check:
        ref = O.gaans_encode(w.symbols, w.indexes, w.cdfs, w.cdf_sizes, w.offsets, w.p_ch,
                             channels, payload.segments)
        got = payload.to_bytes()
        assert len(got) == len(ref)
        assert got == ref
    out = backend.decode(payload, idx, cdfs, sizes, offs)
    assert torch.equal(out, sym)
    return payload


# ---- reference GPU test cases (tests/gpu/test_warp_div_cuda.py:18-41) ------

REF_CDFS = [[0, 8192, 16384, 32768, 65536]] * 4


def ref_case(backend, device, symbols, p_ch):
    s = np.array([symbols], np.int32)
    idx = np.array([[0, 1, 2, 3] * (s.shape[1] // 4)], np.int32)
    w = synthetic.Workload("reference 4-table case", s, idx, np.array(REF_CDFS, np.int32),
                           np.array([5] * 4, np.int32), np.array([-2, -1, 0, 1], np.int32), 4,
                           p_ch, 0)
    payload = check_workload(backend, device, w)
    assert payload.p_ch == p_ch
    assert tuple(payload.max_rounds.shape) == (1, 4 // p_ch)


@pytest.mark.parametrize("p_ch", [1, 2, 4])
def test_reference_round_trip_multiple_p_ch(backend, gpu_device, p_ch):
    ref_case(backend, gpu_device, [0, 1, 2, 3] * 16, p_ch)


def test_reference_round_trip_escape_symbols(backend, gpu_device):
    ref_case(backend, gpu_device, [-100, 100, -101, 102] * 16, 2)


# ---- hand-derived KAT payloads (see tests/test_oracle.py) -------------------

@pytest.mark.parametrize("segments", [1, 2, 3])
def test_kat_payloads_bit_exact(backend, gpu_device, segments):
    cdf = list(range(17)) + [65536]
    s = [(5 * p + 3) % 16 for p in range(130)]
    s[3], s[70], s[129] = -1, 56, 17
    w = synthetic.Workload("KAT 130", np.array([s], np.int32), None, np.array([cdf], np.int32),
                           np.array([18], np.int32), np.array([0], np.int32), 1, 1, 0)
    check_workload(backend, gpu_device, w, segments=segments)
    w = synthetic.Workload("KAT 2", np.zeros((1, 2), np.int32), None,
                           np.array([[0, 32768, 65536]], np.int32), np.array([3], np.int32),
                           np.array([0], np.int32), 1, 1, 0)
    check_workload(backend, gpu_device, w)


# ---- random shapes, ragged chunks, escapes ---------------------------------

def random_tables(rng, M, max_size):
    cdfs = np.zeros((M, max_size), np.int32)
    sizes = np.zeros(M, np.int32)
    for t in range(M):
        S = int(rng.integers(2, max_size + 1))
        f = rng.integers(1, 1000, S - 1).astype(np.float64)
        f = np.floor(f / f.sum() * (65536 - (S - 1))).astype(np.int64) + 1
        f[np.argmax(f)] += 65536 - f.sum()
        cdfs[t, :S] = np.concatenate([[0], np.cumsum(f)])
        sizes[t] = S
    return cdfs, sizes, rng.integers(-20, 20, M).astype(np.int32)


@pytest.mark.parametrize("segments", [1, 2, 5])
def test_random_shapes_bit_exact(backend, gpu_device, segments):
    # segments: as asked, or the most the shape allows
    rng = np.random.default_rng(11 + segments)
    for trial in range(40):
        B, C = int(rng.integers(1, 4)), int(rng.integers(1, 13))
        HW = int(rng.choice([1, 3, 16, 63, 64, 65, 200, 777]))
        P = int(rng.integers(1, C + 1))
        cdfs, sizes, offs = random_tables(rng, C, int(rng.integers(2, 70)))
        s = np.rint(rng.laplace(0, rng.uniform(0.2, 30), (B, C * HW))).astype(np.int32)
        if trial % 3 == 0:
            k = int(rng.integers(s.size))
            s.flat[k] = int(rng.choice([2**30 + 7, -(2**31) + 40, 2**20, -(2**16)]))
        w = synthetic.Workload(f"random trial {trial}", s, None, cdfs, sizes, offs, C, P, 0)
        check_workload(backend, gpu_device, w, segments=segments)


@pytest.mark.parametrize("segments", [1, 2, 5])
def test_explicit_random_indexes_bit_exact(backend, gpu_device, segments):
    rng = np.random.default_rng(12 + segments)
    for trial in range(10):
        M, C, HW = int(rng.integers(1, 9)), int(rng.integers(1, 9)), int(rng.integers(1, 300))
        P = int(rng.integers(1, C + 1))
        cdfs, sizes, offs = random_tables(rng, M, 40)
        s = rng.integers(-30, 30, (2, C * HW)).astype(np.int32)
        idx = rng.integers(0, M, (2, C * HW)).astype(np.int32)
        w = synthetic.Workload(f"explicit trial {trial}", s, idx, cdfs, sizes, offs, C, P, 0)
        check_workload(backend, gpu_device, w, channels=C, segments=segments)


@pytest.mark.parametrize("segments", [1, 2])
def test_offsets_near_int32_max_bit_exact(backend, gpu_device, segments):
    # Table offsets above INT32_MAX - 65535 turn the kernels' fast record
    # paths off (symbol - offset may then leave 32 bits; the blob's flag says
    # so), so full blocks take the checked paths: escapes below the tables'
    # ranges down to offset - 2^31 (the lowest codable value, raw 2^32 - 1)
    # and above them up to INT32_MAX, next to in-range symbols, with a ragged
    # last step.
    rng = np.random.default_rng(31)
    C, HW, P = 6, 64 * 12 + 5, 3
    cdfs, sizes, _ = random_tables(rng, C, 12)
    offs = (2**31 - 100 - rng.integers(0, 60000, C)).astype(np.int64)
    sym = np.empty((1, C * HW), np.int64)
    for c in range(C):
        o, S = int(offs[c]), int(sizes[c])
        kind = rng.integers(0, 10, HW)
        inside = o + rng.integers(0, max(1, S - 2), HW)
        below = o - 2**31 + rng.integers(0, 1000, HW)
        above = 2**31 - 1 - rng.integers(0, 1000, HW)
        sym[0, c * HW:(c + 1) * HW] = np.where(kind < 7, inside, np.where(kind < 9, above, below))
    assert sym.min() >= -2**31 and sym.max() <= 2**31 - 1
    w = synthetic.Workload("offsets near INT32_MAX", sym.astype(np.int32), None, cdfs, sizes,
                           offs.astype(np.int32), C, P, 0)
    check_workload(backend, gpu_device, w, segments=segments)


def test_long_chunks_with_partial_last_block(backend, gpu_device):
    # chunks of 32,800 symbols (C=8, HW=4100, P=8): 513 steps, so with one
    # segment the encoder's 16-step blocks end with a one-step block (two and
    # five segments: units of 256/257 and 102/103 steps); explicit indexes
    # with escapes, then the fused latents path with explicit indexes
    rng = np.random.default_rng(21)
    w0 = synthetic.coder_512x768(seed=21)
    C, HW = 8, 4100
    cdfs, sizes, offs = w0.cdfs[:C], w0.cdf_sizes[:C], w0.offsets[:C]
    idx = np.repeat(np.arange(C, dtype=np.int32), HW)[None]
    s = np.rint(rng.laplace(0, 2.0, (1, C * HW))).astype(np.int32)
    s[0, ::211] = rng.integers(-90000, 90000, s[0, ::211].shape)
    for S in (1, 2, 5):
        w = synthetic.Workload("long chunks 1x8x4100", s, idx, cdfs, sizes, offs, C, C, 0)
        check_workload(backend, gpu_device, w, segments=S)
    tables = prepare_tables(dev(cdfs, gpu_device), dev(sizes, gpu_device), dev(offs, gpu_device))
    med = rng.normal(0, 0.3, C).astype(np.float32)
    y = (s.reshape(1, C, HW) + med[None, :, None]
         + rng.uniform(-0.49, 0.49, (1, C, HW))).astype(np.float32)
    sym = O.quantize(y, med).reshape(1, -1)
    for S in (1, 4):
        say("case: fused latents, explicit indexes, 1x8x4100 P=8, segments", S)
        enc = gaans.encode(tables, 1, C * HW, C, C, gpu_device, y=dev(y, gpu_device),
                           medians=dev(med, gpu_device), indexes=dev(idx, gpu_device),
                           segments=S)
        assert enc.packed.cpu().numpy().tobytes() == O.gaans_encode(sym, idx, cdfs, sizes, offs,
                                                                      C, C, S)
        y_hat = gaans.decode(enc.packed, tables, 1, C * HW, C, C, gpu_device,
                             medians=dev(med, gpu_device), indexes=dev(idx, gpu_device),
                             segments=S)
        want = O.dequantize(sym.reshape(1, C, HW), med).reshape(1, -1)
        assert np.array_equal(y_hat.cpu().numpy().view(np.uint32), want.view(np.uint32))


# ---- benchmark shapes at full size -----------------------------------------

@pytest.mark.parametrize("segments", [None, 2, 3])
def test_coder_512x768_p4_bit_exact(backend, gpu_device, segments):
    check_workload(backend, gpu_device, synthetic.coder_512x768(), segments=segments)


def test_side_stream_calls_without_device_sync(backend, gpu_device):
    # encode returns once the coding kernel's completion word is set, while
    # its pack kernel may still run: work ordered on the same stream (the
    # host copy, the decode) must see the finished payload
    w = synthetic.coder_512x768()
    say("case: side stream, back-to-back calls", w.name)
    ref = O.gaans_encode(w.symbols, w.indexes, w.cdfs, w.cdf_sizes, w.offsets, w.p_ch)
    side = torch.cuda.Stream(gpu_device)
    with torch.cuda.stream(side):
        sym = dev(w.symbols, gpu_device)
        idx = dev(w.explicit_indexes(), gpu_device)
        cdfs, sizes, offs = tables_on(w, gpu_device)
        for rep in range(4):
            payload = backend.encode(sym, idx, cdfs, sizes, offs, p_ch=w.p_ch, segments=1)
            assert payload.to_bytes() == ref, rep
            out = backend.decode(payload, idx, cdfs, sizes, offs)
            assert torch.equal(out, sym), rep
            sym_next = torch.flip(sym, dims=[1]).contiguous()
            payload2 = backend.encode(sym_next, idx.flip(1).contiguous(), cdfs, sizes, offs,
                                      p_ch=1)
            out2 = backend.decode(payload2, idx.flip(1).contiguous(), cdfs, sizes, offs)
            assert torch.equal(out2, sym_next), rep
    side.synchronize()


@pytest.mark.parametrize("p_ch", [1, 16, 192])
def test_coder_512x768_other_p(backend, gpu_device, p_ch):
    check_workload(backend, gpu_device, synthetic.coder_512x768(p_ch=p_ch))


@pytest.mark.parametrize("p_ch", [1, 4, 16, 64, 192])
def test_hyperprior_y_gaussian_tables(backend, gpu_device, p_ch):
    yw, zw, _, _ = synthetic.hyperprior_512x768(p_ch=p_ch)
    check_workload(backend, gpu_device, yw, channels=192)
    zw.p_ch = min(p_ch, 128)
    check_workload(backend, gpu_device, zw)


@pytest.mark.parametrize("segments", [None, 1, 7])
def test_highres_2160x3840_p8(backend, gpu_device, segments):
    check_workload(backend, gpu_device, synthetic.highres_2160x3840(), segments=segments)


@pytest.mark.parametrize("segments", [None, 2])
@pytest.mark.parametrize("make", [synthetic.batch_skew, synthetic.batch_uniform])
def test_batch64_p16(backend, gpu_device, make, segments):
    check_workload(backend, gpu_device, make(), segments=segments)


@pytest.mark.parametrize("segments", [1, 4])
def test_escape_heavy_chunks_bit_exact(backend, gpu_device, segments):
    # every symbol of a 1x192x32x48 image escapes: each chunk's escape section
    # holds 6,144 entries, several times the decoder's escape FIFO
    w = synthetic.coder_512x768(seed=7)
    rng = np.random.default_rng(7)
    w.symbols = (w.symbols * 40 + rng.integers(-3, 4, w.symbols.shape)
                 + np.where(rng.random(w.symbols.shape) < 0.5, 5000, -5000)).astype(np.int32)
    w.name = "all-escape 1x192x32x48"
    check_workload(backend, gpu_device, w, segments=segments)


def test_escape_heavy_batch_bit_exact(backend, gpu_device):
    # 48 images with the narrow tables of the 95%-zero workload and symbols
    # drawn wider than their support: 576 chunks, so the decoder runs three
    # workgroups per CU with 4-step blocks, and most steps carry escapes
    w = synthetic.batch_skew(batch=48)
    rng = np.random.default_rng(8)
    w.symbols = np.rint(rng.laplace(0, 2.0, w.symbols.shape)).astype(np.int32)
    w.name = "escape-heavy batch 48x192x32x48"
    check_workload(backend, gpu_device, w)


def test_non_minimal_escape_count_rejected(backend, gpu_device):
    # the oracle's case (tests/test_oracle.py): count 2 for a raw value that
    # needs one nibble, same payload length
    import struct

    cdfs, sizes, offs = (np.array([[0, 32768, 65536]], np.int32), np.array([3], np.int32),
                         np.array([0], np.int32))
    data = O.gaans_encode([[2]], None, cdfs, sizes, offs, 1)
    hb = (64 + 8 + 15) // 16 * 16
    bad = bytearray(data)
    struct.pack_into("<H", bad, hb + 6, 0x0022)
    say("case: non-minimal escape count")
    c, z, o = dev(cdfs, gpu_device), dev(sizes, gpu_device), dev(offs, gpu_device)
    idx = torch.zeros((1, 1), dtype=torch.int32, device=gpu_device)
    good = WarpDivPayload.from_bytes(data, device=gpu_device)
    assert backend.decode(good, idx, c, z, o).tolist() == [[2]]
    with pytest.raises(CoderInputError, match="corrupt"):
        backend.decode(WarpDivPayload.from_bytes(bytes(bad), device=gpu_device), idx, c, z, o)


# ---- fused quantize / dequantize -------------------------------------------

def test_fused_latents_match_quantize_then_encode(gpu_device):
    w = synthetic.coder_512x768(seed=3)
    rng = np.random.default_rng(3)
    B, N, C = w.batch, w.n, w.channels
    med = rng.normal(0, 0.3, C).astype(np.float32)
    HW = N // C
    y = (w.symbols.reshape(B, C, HW) + med[None, :, None]
         + rng.uniform(-0.5, 0.5, (B, C, HW))).astype(np.float32)
    y[0, 0, :8] = med[0] + np.array([0.5, -0.5, 1.5, -1.5, 2.5, -0.0, 1e7, -3e6], np.float32)
    sym_ref = O.quantize(y, med)
    tables = prepare_tables(*tables_on(w, gpu_device))
    say("case: fused latents 1x192x32x48 P=4")
    enc = gaans.encode(tables, B, N, C, 4, gpu_device, y=dev(y, gpu_device),
                       medians=dev(med, gpu_device))
    ref = O.gaans_encode(sym_ref.reshape(B, N), None, w.cdfs, w.cdf_sizes, w.offsets, 4)
    assert enc.packed.cpu().numpy().tobytes() == ref
    y_hat = gaans.decode(enc.packed, tables, B, N, C, 4, gpu_device,
                         medians=dev(med, gpu_device))
    ref_hat = O.dequantize(sym_ref, med).reshape(B, N)
    assert np.array_equal(y_hat.cpu().numpy().view(np.uint32), ref_hat.view(np.uint32))
    # and against torch on the GPU (CompressAI's quantize / dequantize expressions)
    yt, mt = dev(y, gpu_device), dev(med, gpu_device)[None, :, None]
    sym_t = torch.round(yt - mt).int()
    assert np.array_equal(sym_t.cpu().numpy(), sym_ref)
    assert torch.equal(y_hat.view(B, C, HW), sym_t.type_as(mt) + mt)


def test_fused_latents_many_workgroups_per_cu(gpu_device):
    """32 images at P = 16: 384 coding units, more than the device's CUs, so
    the decoder's steps skip the refill read when no lane refills (the
    256-bucket lookups of 16 tables per unit)."""
    w = synthetic.coder_512x768(seed=5, batch=32, p_ch=16)
    rng = np.random.default_rng(5)
    B, N, C = w.batch, w.n, w.channels
    med = rng.normal(0, 0.3, C).astype(np.float32)
    HW = N // C
    y = (w.symbols.reshape(B, C, HW) + med[None, :, None]
         + rng.uniform(-0.5, 0.5, (B, C, HW))).astype(np.float32)
    sym_ref = O.quantize(y, med)
    tables = prepare_tables(*tables_on(w, gpu_device))
    say("case: fused latents 32x192x32x48 P=16")
    enc = gaans.encode(tables, B, N, C, 16, gpu_device, y=dev(y, gpu_device),
                       medians=dev(med, gpu_device), segments=1)
    ref = O.gaans_encode(sym_ref.reshape(B, N), None, w.cdfs, w.cdf_sizes, w.offsets, 16)
    assert enc.packed.cpu().numpy().tobytes() == ref
    y_hat = gaans.decode(enc.packed, tables, B, N, C, 16, gpu_device,
                         medians=dev(med, gpu_device), segments=1)
    ref_hat = O.dequantize(sym_ref, med).reshape(B, N)
    assert np.array_equal(y_hat.cpu().numpy().view(np.uint32), ref_hat.view(np.uint32))


def test_fused_latents_reject_non_finite(gpu_device):
    w = synthetic.coder_512x768()
    tables = prepare_tables(*tables_on(w, gpu_device))
    y = np.zeros((1, 192, 1536), np.float32)
    y[0, 5, 7] = np.nan
    say("case: fused latents with NaN")
    with pytest.raises(CoderInputError, match="non-finite"):
        gaans.encode(tables, 1, w.n, 192, 4, gpu_device, y=dev(y, gpu_device),
                     medians=torch.zeros(192, device=gpu_device))


# ---- negative cases (tests/gpu/test_factorized_gaans.py:75-98) -------------

@pytest.fixture(scope="module")
def encoded(backend, gpu_device):
    w = synthetic.coder_512x768(seed=5)
    sym, idx = dev(w.symbols, gpu_device), dev(w.explicit_indexes(), gpu_device)
    cdfs, sizes, offs = tables_on(w, gpu_device)
    payload = backend.encode(sym, idx, cdfs, sizes, offs, p_ch=4)
    return w, sym, idx, cdfs, sizes, offs, payload


def test_flipped_header_byte_rejected(backend, encoded):
    w, sym, idx, cdfs, sizes, offs, payload = encoded
    say("case: flipped header byte")
    bad = payload.packed.clone()
    bad[0] ^= 1
    with pytest.raises(CoderInputError, match="header"):
        backend.decode(replace(payload, packed=bad), idx, cdfs, sizes, offs)


def test_corrupt_stream_rejected(backend, encoded):
    w, sym, idx, cdfs, sizes, offs, payload = encoded
    for pos in (payload.header_bytes + 3, payload.header_bytes + 5000,
                payload.packed.numel() - 7):
        say("case: corrupt stream byte", pos)
        bad = payload.packed.clone()
        bad[pos] ^= 0x21
        with pytest.raises(CoderInputError):
            backend.decode(replace(payload, packed=bad), idx, cdfs, sizes, offs)
    say("case: corrupt chunk offset")
    bad = payload.packed.clone()
    bad[64 + 4 * 3] ^= 0x04
    with pytest.raises(CoderInputError):
        backend.decode(replace(payload, packed=bad), idx, cdfs, sizes, offs)


def test_other_tables_or_indexes_rejected(backend, encoded):
    w, sym, idx, cdfs, sizes, offs, payload = encoded
    say("case: fingerprint mismatch")
    with pytest.raises(CoderInputError, match="match"):
        backend.decode(replace(payload, coding_fingerprint="0" * 64), idx, cdfs, sizes, offs)
    say("case: other tables")
    offs2 = offs.clone()
    offs2[0] += 1
    with pytest.raises(CoderInputError, match="match"):
        backend.decode(payload, idx, cdfs, sizes, offs2)
    say("case: other indexes")
    idx2 = idx.clone()
    idx2[0, 100] = 1
    with pytest.raises(CoderInputError):
        backend.decode(payload, idx2, cdfs, sizes, offs)
    with pytest.raises(CoderInputError, match="match"):
        replace(payload, p_ch=3, chunk_len=12)


def test_out_of_range_index_rejected(backend, gpu_device, encoded):
    w, sym, idx, cdfs, sizes, offs, payload = encoded
    say("case: index out of range")
    idx2 = idx.clone()
    idx2[0, 17] = 192
    with pytest.raises(CoderInputError, match="outside"):
        backend.encode(sym, idx2, cdfs, sizes, offs, p_ch=4)
    # two units (the first and the last chunk) report it in the same launch;
    # the completion counter is left clean for the next call, whose payload
    # is the one made before
    idx2[0, idx.shape[1] - 1] = -1
    with pytest.raises(CoderInputError, match="outside"):
        backend.encode(sym, idx2, cdfs, sizes, offs, p_ch=4)
    again = backend.encode(sym, idx, cdfs, sizes, offs, p_ch=4)
    assert torch.equal(again.packed, payload.packed)


def test_payload_bytes_round_trip(backend, gpu_device, encoded):
    w, sym, idx, cdfs, sizes, offs, payload = encoded
    again = WarpDivPayload.from_bytes(payload.to_bytes(), device=gpu_device)
    assert again.coding_fingerprint == payload.coding_fingerprint
    assert torch.equal(again.chunk_ends, payload.chunk_ends)
    assert torch.equal(backend.decode(again, idx, cdfs, sizes, offs), sym)


def test_bpp_against_compressai_equivalent_stream(backend, gpu_device):
    # the payload's overhead over one CompressAI-style stream per image is the
    # lane flush (64 x 32 bits per chunk) plus the header; at P=192 (one chunk)
    # it must be within 1%.
    w = synthetic.coder_512x768(p_ch=192)
    payload = check_workload(backend, gpu_device, w, bytes_check=False)
    single = len(O.rans64_encode(w.symbols[0], w.explicit_indexes()[0], w.cdfs, w.cdf_sizes,
                                 w.offsets))
    assert payload.packed.numel() <= single * 1.01


# ---- the decoder's search lookups (many wide tables, sub-blocks not in LDS) ----

def wide_gaussian_rows(B, C, HW, p_ch, seed):
    """Rows coded with the 64 GaussianConditional-style tables of the
    hyperprior workload (3 .. 3,132 symbols), per-element indexes, draws that
    reach deep into the tails and past the table ranges (escapes)."""
    yw, _, _, _ = synthetic.hyperprior_512x768()
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, 64, size=(B, C * HW), dtype=np.int32)
    scale = np.exp(np.linspace(np.log(0.11), np.log(256.0), 64))[idx]
    sym = np.rint(rng.standard_normal((B, C * HW)) * scale * 1.5).astype(np.int32)
    sym[:, ::97] = rng.integers(-5000, 5000, size=sym[:, ::97].shape, dtype=np.int32)
    return synthetic.Workload("wide Gaussian rows", sym, idx, yw.cdfs, yw.cdf_sizes, yw.offsets,
                              C, p_ch, 0)


@pytest.mark.parametrize("B,C,HW,p_ch", [(3, 24, 77, 5), (2, 64, 96, 16), (1, 8, 9, 3)])
def test_search_lookup_decoder_bit_exact(backend, gpu_device, B, C, HW, p_ch):
    w = wide_gaussian_rows(B, C, HW, p_ch, seed=B * 100 + C)
    check_workload(backend, gpu_device, w, channels=C)


def test_search_lookup_decoder_rejects_corruption(backend, gpu_device):
    w = wide_gaussian_rows(2, 24, 77, 4, seed=9)
    payload = check_workload(backend, gpu_device, w, channels=24)
    idx = dev(w.explicit_indexes(), gpu_device)
    cdfs, sizes, offs = tables_on(w, gpu_device)
    for pos in (payload.header_bytes + 11, payload.packed.numel() // 2):
        say("case: search decoder, corrupt byte", pos)
        bad = payload.packed.clone()
        bad[pos] ^= 0x5A
        with pytest.raises(CoderInputError):
            backend.decode(replace(payload, packed=bad), idx, cdfs, sizes, offs)
    say("case: search decoder, other indexes")
    idx2 = idx.clone()
    idx2[1, 7] = (idx2[1, 7] + 1) % 64
    with pytest.raises(CoderInputError):
        backend.decode(payload, idx2, cdfs, sizes, offs)
