"""CPU checks of the HIP library's host side: it loads without a GPU, exports
every symbol include/gaans_w64.h declares, computes layouts, and prepares
tables whose digest and decode lookup agree with the oracle / a brute-force
search.  No kernel is launched here."""

import ctypes
import os
import re
import struct

import numpy as np
import pytest

import oracle as O
from fast_compressai.coders import _native
from fast_compressai import synthetic

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    header = open(os.path.join(REPO, "include", "gaans_w64.h")).read()
    declared = set(re.findall(r"^\s*(?:int|const char\*)\s+(gaans_\w+)\s*\(", header, re.M))
    assert "gaans_encode_symbols" in declared and len(declared) >= 11
    lib = ctypes.CDLL(_native.library_path())
    for name in sorted(declared):
        assert hasattr(lib, name), name
    assert _native.lib().gaans_abi_version() == _native.ABI_VERSION


def test_host_selftest_division_constants():
    assert _native.lib().gaans_host_selftest() == 0, _native.last_error()


def test_layout_limits_of_the_completion_counters():
    # the encoder's completion counter is one 64-bit word: units in 24 bits,
    # the payload body in 36 bits of u32 words; larger shapes are refused
    # before any device work
    from fast_compressai.coders import CoderInputError
    assert _native.layout(2**24 - 1, 64, 1, 1).U == 2**24 - 1
    with pytest.raises(CoderInputError, match="too many coding units"):
        _native.layout(2**24, 64, 1, 1)
    assert _native.layout(16, 2**30, 2**16, 1).U == 2**20  # 7.5e10-byte worst case
    with pytest.raises(CoderInputError, match="shape too large"):
        _native.layout(64, 2**30, 2**16, 1)  # 4.8e11 bytes >= 2^38


def test_layout_matches_format():
    lay = _native.layout(1, 192 * 32 * 48, 192, 4)
    assert (lay.K, lay.chunk_len, lay.U, lay.HW, lay.S) == (48, 6144, 48, 1536, 1)
    assert lay.header_bytes == (64 + 8 * 48 + 15) // 16 * 16
    lay = _native.layout(64, 192 * 1536, 192, 16)
    assert (lay.K, lay.U, lay.chunk_len) == (12, 768, 24576)
    assert lay.workspace_bytes >= lay.U * lay.cap_words * 2
    lay = _native.layout(1, 128 * 96, 128, 5)  # C not a multiple of P
    assert lay.K == 26 and lay.chunk_len == 480
    for bad in ((0, 4, 1, 1), (1, 5, 2, 1), (1, 4, 2, 3)):
        with pytest.raises(Exception):
            _native.layout(*bad)


def test_segment_layout_and_choice():
    N = 192 * 1536
    one, three = _native.layout(1, N, 192, 4, 1), _native.layout(1, N, 192, 4, 3)
    assert (one.S, three.S, one.U, three.U) == (1, 3, 48, 144)
    # two more units of 64 states (+ pad and escape word) per chunk, 48 chunks
    assert three.max_payload_bytes - three.header_bytes - (
        one.max_payload_bytes - one.header_bytes) == 48 * 2 * (64 * 4 + 8)
    assert three.header_bytes == (64 + 8 * 144 + 15) // 16 * 16
    # a unit holds at most ceil(96 / 3) = 32 steps: its staging words (one
    # per symbol, 2 more, rounded to whole 16-byte chunks)
    assert three.cap_words == 32 * 64 + 8
    # at least one step per segment (the shortest chunk decides), at most 256
    _native.layout(1, N, 192, 4, 96)
    for bad in ((1, N, 192, 4, 97), (1, N, 192, 4, 0), (1, 64 * 300, 1, 1, 257),
                (1, 3 * 64, 3, 2, 2)):
        with pytest.raises(Exception):
            _native.layout(*bad)
    _native.layout(1, 64 * 300, 1, 1, 256)
    L = _native.lib()
    # the tables' mean entropy: 1 bit (two halves) and 1.5 bits (1/4, 1/4, 1/2)
    cdfs = np.array([[0, 32768, 65536, 0], [0, 16384, 32768, 65536]], np.int32)
    sizes, offs = np.array([3, 4], np.int32), np.zeros(2, np.int32)
    nb = ctypes.c_int64()
    assert L.gaans_tables_bytes(cdfs.ctypes.data, sizes.ctypes.data, 2, 4, ctypes.byref(nb)) == 0
    blob, desc = np.zeros(nb.value, np.uint8), _native.Tables()
    assert L.gaans_tables_prepare(cdfs.ctypes.data, sizes.ctypes.data, offs.ctypes.data, 2, 4,
                                  blob.ctypes.data, nb.value, ctypes.byref(desc)) == 0
    assert desc.mean_bits == pytest.approx(1.25, abs=1e-6)

    def choose(bits, B, N, C, P, budget=0.006, target=256):
        d = _native.Tables()
        d.mean_bits = bits
        out = ctypes.c_int32(0)
        assert L.gaans_choose_segments(ctypes.byref(d), B, N, C, P, budget, target,
                                       ctypes.byref(out)) == 0
        return out.value

    # 2160x3840 latent, P=8: 40 chunks of 261,120 symbols at 3.74 bits, about
    # 122,330 B each; an added unit costs 3.125 * 64 + 4 = 204 B (0.17%):
    # 0.6% allows 3 more (1 + floor(734 / 204))
    assert choose(3.74, 1, 320 * 32640, 320, 8) == 4
    assert choose(3.74, 1, 320 * 32640, 320, 8, budget=0.01) == 6
    assert choose(3.74, 1, 320 * 32640, 320, 8, budget=0.1) == 7  # 280 units fill 256 CUs
    # without a unit target: 1 + floor(0.1 * 122,330 / 204) = 60
    assert choose(3.74, 1, 320 * 32640, 320, 8, budget=0.1, target=0) == 60
    assert choose(3.74, 1, 320 * 32640, 320, 8, budget=0.001) == 1
    # 512x768 latent, P=4: 6,144 symbols at 2.67 bits (about 2 KB): one unit
    assert choose(2.67, 1, N, 192, 4) == 1
    # 768 chunks already fill the device
    assert choose(8.0, 64, N, 192, 16, budget=1.0) == 1
    # one step per chunk: nothing to split
    assert choose(8.0, 1, 64 * 12, 12, 1, budget=1.0) == 1


def prepare_host(cdfs, sizes, offs):
    L = _native.lib()
    cdfs = np.ascontiguousarray(cdfs, np.int32)
    sizes = np.ascontiguousarray(sizes, np.int32)
    offs = np.ascontiguousarray(offs, np.int32)
    nb = ctypes.c_int64()
    rc = L.gaans_tables_bytes(cdfs.ctypes.data, sizes.ctypes.data, cdfs.shape[0], cdfs.shape[1],
                              ctypes.byref(nb))
    if rc:
        return rc, None, None
    out = np.zeros(nb.value, np.uint8)
    desc = _native.Tables()
    rc = L.gaans_tables_prepare(cdfs.ctypes.data, sizes.ctypes.data, offs.ctypes.data,
                                cdfs.shape[0], cdfs.shape[1], out.ctypes.data, nb.value,
                                ctypes.byref(desc))
    if rc == 0:
        assert desc.bytes == nb.value and desc.M == cdfs.shape[0]
        assert desc.max_nsym == int(np.max(sizes)) - 1
        assert desc.total_nsym == int(np.sum(sizes)) - cdfs.shape[0]
    return rc, out, desc.digest


def host_lookup(blob, t, cum, levels=None):
    """Decode lookup as the kernel does it, read from the prepared blob: the
    table's entry of bucket cum >> 8, for a dense bucket entry (cum >> 4) & 15
    of its sub-block, for a dense sub-range entry cum & 15 of the next one."""
    hdr = struct.unpack_from("<16I", blob, 0)
    meta_off, lut_off, sub_off, total_sub = hdr[6], hdr[8], hdr[11], hdr[12]
    e = struct.unpack_from("<Q", blob, lut_off + 8 * (256 * t + (cum >> 8)))[0]
    depth = 1
    for shift in (4, 0):
        if e >> 48 != 0xFFFF:
            break
        blk = e & 0xFFFFFFFF
        assert blk < total_sub
        e = struct.unpack_from("<Q", blob, sub_off + 8 * (16 * blk + ((cum >> shift) & 15)))[0]
        depth += 1
    assert e >> 48 != 0xFFFF
    if levels is not None:
        levels[depth] = levels.get(depth, 0) + 1
    lo, hi = e & 0xFFFFFFFF, e >> 32
    s0, nxt = hi & 0xFFFF, hi >> 16
    st0, st1 = lo & 0xFFFF, (lo >> 16) + 1  # start(s0), start(s0 + 1)
    if cum >= st1:
        return s0 + 1, st1, nxt + 1
    return s0, st0, st1 - st0


def host_lookup_wide(blob, t, cum, levels=None):
    """The wide decode lookup as the kernel does it, read from the prepared
    blob: entry cum >> 5 of the table's 2048, for a dense bucket entry
    (cum >> 1) & 15 of its sub-block, which is never dense."""
    hdr = struct.unpack_from("<20I", blob, 0)
    wide_off, wdense_off, total_wide = hdr[16], hdr[17], hdr[19]
    e = struct.unpack_from("<Q", blob, wide_off + 8 * (2048 * t + (cum >> 5)))[0]
    depth = 1
    if e >> 48 == 0xFFFF:
        blk = e & 0xFFFFFFFF
        assert blk < total_wide
        e = struct.unpack_from("<Q", blob, wdense_off + 8 * (16 * blk + ((cum >> 1) & 15)))[0]
        depth = 2
    assert e >> 48 != 0xFFFF
    if levels is not None:
        levels[depth] = levels.get(depth, 0) + 1
    lo, hi = e & 0xFFFFFFFF, e >> 32
    s0, nxt = hi & 0xFFFF, hi >> 16
    st0, st1 = lo & 0xFFFF, (lo >> 16) + 1
    if cum >= st1:
        return s0 + 1, st1, nxt + 1
    return s0, st0, st1 - st0


def wide_bases(blob, M):
    hdr = struct.unpack_from("<20I", blob, 0)
    return struct.unpack_from(f"<{M + 1}I", blob, hdr[18])


def test_wide_lookups_exhaustive():
    # every cum value of the 512x768 tables (Laplacian tails) and of the
    # hyperprior's widest GaussianConditional tables (freq-1 tails) against
    # np.searchsorted; the per-table sub-block bases partition the sub-blocks
    w = synthetic.coder_512x768()
    yw, _, _, _ = synthetic.hyperprior_512x768()
    for cdfs, sizes, offs, tabs in ((w.cdfs[:6], w.cdf_sizes[:6], w.offsets[:6], range(6)),
                                    (yw.cdfs, yw.cdf_sizes, yw.offsets, (0, 31, 62, 63))):
        rc, blob, _ = prepare_host(cdfs, sizes, offs)
        assert rc == 0
        blob = blob.tobytes()
        hdr = struct.unpack_from("<20I", blob, 0)
        assert hdr[13] & 4  # wide lookups present
        bases = wide_bases(blob, cdfs.shape[0])
        assert bases[0] == 0 and bases[-1] == hdr[19] and list(bases) == sorted(bases)
        levels = {}
        for t in tabs:
            c = cdfs[t, : sizes[t]]
            want = np.searchsorted(c, np.arange(65536), side="right") - 1
            for cum in range(65536):
                v, start, freq = host_lookup_wide(blob, t, cum, levels)
                assert v == want[cum] and start == c[v] and freq == c[v + 1] - c[v], (t, cum)
        assert levels.get(2, 0) > 0  # dense buckets exist and resolve in one more read


def test_wide_lookups_only_for_at_most_4096_tables():
    w = synthetic.coder_512x768()
    cdfs = np.repeat(w.cdfs[:1], 4097, 0)
    sizes = np.repeat(w.cdf_sizes[:1], 4097)
    rc, blob, _ = prepare_host(cdfs, sizes, np.zeros(4097, np.int32))
    assert rc == 0 and not struct.unpack_from("<20I", blob.tobytes(), 0)[13] & 4
    rc, blob, _ = prepare_host(cdfs[:4096], sizes[:4096], np.zeros(4096, np.int32))
    assert rc == 0 and struct.unpack_from("<20I", blob.tobytes(), 0)[13] & 4


def test_prepared_tables_digest_and_lookup_exhaustive():
    w = synthetic.coder_512x768()
    cdfs, sizes, offs = w.cdfs[:6], w.cdf_sizes[:6], w.offsets[:6]
    rc, blob, dg = prepare_host(cdfs, sizes, offs)
    assert rc == 0
    assert dg == O.table_digest(cdfs, sizes, offs)
    blob = blob.tobytes()
    # entry word 1 is the encoder's division constant: q = x // freq on [0, freq << 16)
    hdr = struct.unpack_from("<16I", blob, 0)
    for t in range(6):
        ent_base, nsym = struct.unpack_from("<II", blob, hdr[6] + 16 * t)
        for v in range(nsym):
            w0, m = struct.unpack_from("<II", blob, hdr[7] + 8 * (ent_base + v))
            f = (w0 >> 16) + 1
            if f == 1:
                continue
            sh = (f - 1).bit_length() - 1
            for x in (0, f - 1, f, (f << 16) - 1, (f << 15) + 12345, 0xFFFF * f):
                tt = (x * m) >> 32
                assert (tt + ((x - tt) >> 1)) >> sh == x // f, (t, v, f, x)
    levels = {}
    for t in range(6):
        c = cdfs[t, : sizes[t]]
        want = np.searchsorted(c, np.arange(65536), side="right") - 1
        for cum in range(0, 65536, 7):
            v, start, freq = host_lookup(blob, t, cum, levels)
            assert v == want[cum] and start == c[v] and freq == c[v + 1] - c[v], (t, cum)
    assert levels.get(2, 0) > 0  # the Laplacian tails are dense buckets


def test_prepared_tables_dense_tail_lookup():
    # GaussianConditional-style table with many freq-1 tail bins
    yw, _, _, _ = synthetic.hyperprior_512x768()
    t = 63
    c = yw.cdfs[t, : yw.cdf_sizes[t]]
    rc, blob, _ = prepare_host(yw.cdfs[t:t + 1], yw.cdf_sizes[t:t + 1], yw.offsets[t:t + 1])
    assert rc == 0
    blob = blob.tobytes()
    want = np.searchsorted(c, np.arange(65536), side="right") - 1
    levels = {}
    for cum in range(65536):  # every value: all three lookup levels occur
        v, start, freq = host_lookup(blob, 0, cum, levels)
        assert v == want[cum] and start == c[v] and freq == c[v + 1] - c[v], cum
    assert levels.get(2, 0) > 0 and levels.get(3, 0) > 0


SEARCH_ENTRIES = 320  # segments per table: 64 parts of 32 values, then the 256 buckets


def host_search(blob, t):
    """The decoder's search lookup of every cum value of table t, read from
    the prepared blob.  Starts: start - 1 mod 2^16 of every symbol, each
    table followed by three 0xFFFF, so table t's symbol v is at starts index
    ent_base + 3 t + v.  Segment of cum: a 32-value part when cum < 1024 or
    cum >= 64512 (entry (cum >> 5) & 63), else its 256-value bucket (entry
    64 + (cum >> 8)).  Entry: m | n << 8 | G << 16.  n = 0: c = G + (((cum
    & 255) * m) >> 8); n > 0: c = G, and n + 1 candidates are narrowed four
    ways (three start reads a round) while more than three remain.  Then
    "start - 1 < cum" over starts c + 1 .. c + 3 counts the symbol's offset
    from c; freq from the next start mod 2^16 (2^16 for a one-symbol table).
    Returns the table's symbol, start and freq per cum and the 4-way rounds
    per cum."""
    hdr = struct.unpack_from("<16I", blob, 0)
    M, clut_off, starts_off = hdr[1], hdr[14], hdr[15]
    first = struct.unpack_from("<I", blob, hdr[6] + 16 * t)[0] + 3 * t
    clut = np.frombuffer(blob, "<u4", SEARCH_ENTRIES * M, clut_off).astype(np.int64)
    starts = np.frombuffer(blob, "<u2", hdr[2] + 3 * M + 8, starts_off).astype(np.int64)
    cum = np.arange(65536, dtype=np.int64)
    fine = ((cum + 1024) & 0xFFFF) < 2048
    e = clut[SEARCH_ENTRIES * t + np.where(fine, (cum >> 5) & 63, 64 + (cum >> 8))]
    m, nl = e & 0xFF, (e >> 8) & 0xFF
    g = (e >> 16) + (((cum & 0xFF) * m) >> 8)
    rounds = np.zeros(65536, np.int64)
    while (nl > 3).any():  # 4-way: probes q, 2q, 3q
        w = nl > 3
        q = (nl + 1) >> 2
        le = [np.where(w, starts[np.where(w, g + j * q, 0)] < cum, False) for j in (1, 2, 3)]
        g = g + np.where(w, (le[0].astype(np.int64) + le[1] + le[2]) * q, 0)
        nl = np.where(w, np.where(le[2], nl - 3 * q, q - 1), nl)
        rounds += w
    v = starts[g[:, None] + np.arange(5)]
    kk = (v[:, 1] < cum).astype(np.int64) + (v[:, 2] < cum) + (v[:, 3] < cum)
    sm = v[np.arange(65536), kk]
    nx = v[np.arange(65536), kk + 1]
    return g + kk - first, (sm + 1) & 0xFFFF, ((nx - sm - 1) & 0xFFFF) + 1, rounds


def test_search_lookups_exhaustive():
    # the 64 GaussianConditional-style tables of the hyperprior workload
    # (3 .. 3,133 symbols, long freq-1 tails), a one-symbol table, and a
    # table that no slope fits (a wide symbol, then 300 freq-1 symbols in a
    # 256-value bucket), every cum value of every table
    yw, _, _, _ = synthetic.hyperprior_512x768()
    cdfs = np.zeros((66, yw.cdfs.shape[1]), np.int32)
    cdfs[:64] = yw.cdfs
    cdfs[64, :2] = [0, 65536]
    odd = np.concatenate([[0], 40000 + np.arange(300), [65536]])
    cdfs[65, : len(odd)] = odd
    sizes = np.concatenate([yw.cdf_sizes, [2, len(odd)]]).astype(np.int32)
    offs = np.concatenate([yw.offsets, [-7, 3]]).astype(np.int32)
    rc, blob, _ = prepare_host(cdfs, sizes, offs)
    assert rc == 0
    blob = blob.tobytes()
    hdr = struct.unpack_from("<16I", blob, 0)
    assert hdr[13] & 2  # search lookups present
    assert hdr[15] - hdr[14] == 4 * SEARCH_ENTRIES * 66
    rounds_seen = np.zeros(8, np.int64)
    for t in range(66):
        c = cdfs[t, : sizes[t]]
        want = np.searchsorted(c, np.arange(65536), side="right") - 1
        v, start, freq, rounds = host_search(blob, t)
        bad = np.flatnonzero((v != want) | (start != c[want]) | (freq != c[want + 1] - c[want]))
        assert bad.size == 0, (t, bad[:5])
        rounds_seen += np.bincount(rounds, minlength=8)[:8]
    # the slopes resolve nearly every value in one read; the unfitted
    # segments (tails of the Gaussian tables, the odd table) search
    assert rounds_seen[0] > 0.98 * rounds_seen.sum()
    assert rounds_seen[1:].sum() > 0 and rounds_seen[3:].sum() > 0


def test_search_lookups_absent_when_not_addressable():
    # more symbols than 16-bit starts indexes reach, or an offset near INT32_MIN
    w = synthetic.batch_uniform(batch=1)
    reps = 300  # 300 tables of 255 symbols: 76,500 > 65,527
    cdfs = np.repeat(w.cdfs[:1], reps, 0)
    sizes = np.repeat(w.cdf_sizes[:1], reps)
    rc, blob, _ = prepare_host(cdfs, sizes, np.zeros(reps, np.int32))
    assert rc == 0 and not struct.unpack_from("<16I", blob.tobytes(), 0)[13] & 2
    rc, blob, _ = prepare_host(w.cdfs[:2], w.cdf_sizes[:2], [0, -2**31 + 5])
    assert rc == 0 and not struct.unpack_from("<16I", blob.tobytes(), 0)[13] & 2


@pytest.mark.parametrize("cdf,size", [([1, 65536], 2), ([0, 65535], 2), ([0, 100, 100, 65536], 4),
                                      ([0, 65536], 1), ([0, 65536], 3)])
def test_invalid_tables_rejected(cdf, size):
    cdfs = np.zeros((1, max(len(cdf), 3)), np.int32)
    cdfs[0, : len(cdf)] = cdf
    rc, _, _ = prepare_host(cdfs, [size], [0])
    assert rc == _native.ETABLE


def test_return_codes_map_to_error_classes():
    # input problems are CoderInputError (a ValueError); a HIP runtime failure
    # is a CoderError (a RuntimeError) but not an input error
    from fast_compressai.coders.errors import CoderError, CoderInputError

    _native.check(_native.OK, "ok")
    for rc in (_native.EINVAL, _native.ETABLE):
        with pytest.raises(CoderInputError, match=f"code {rc}"):
            _native.check(rc, "call")
    with pytest.raises(CoderError, match="code 3") as info:
        _native.check(_native.EHIP, "call")
    assert not isinstance(info.value, ValueError)
    assert isinstance(info.value, RuntimeError)


def test_plan_and_run_reject_bad_arguments_before_device_work():
    # argument errors are found on the host, before any device query (no GPU
    # here): a NULL plan, an unknown mode, a bad shape, and runs with a plan
    # that gaans_plan_* did not fill (or filled for the other direction)
    L = _native.lib()
    plan = (ctypes.c_uint64 * (_native.PLAN_BYTES // 8))()
    addr = ctypes.addressof(plan)
    desc = _native.Tables()
    assert L.gaans_plan_encode(ctypes.byref(desc), 0, 1, 0, 0.0, 1, 64, 1, 1, 1, None) \
        == _native.EINVAL
    assert L.gaans_plan_encode(ctypes.byref(desc), 7, 1, 0, 0.0, 1, 64, 1, 1, 1, addr) \
        == _native.EINVAL
    assert "mode" in _native.last_error()
    assert L.gaans_plan_decode(ctypes.byref(desc), 0, 1, 0, 0.0, 1, 65, 2, 1, 1, addr) \
        == _native.EINVAL  # N % C != 0
    assert L.gaans_plan_encode(ctypes.byref(desc), 0, 1, 0, 0.0, 1, 64, 1, 1, 1, addr) \
        == _native.EINVAL  # descriptor without a blob
    info = (ctypes.c_uint64 * 3)()
    status = (ctypes.c_uint32 * 2)()
    fake = 1 << 20  # never dereferenced: the runs stop at the plan check
    assert L.gaans_run_encode(addr, None, fake, None, None, None, fake, 1 << 20, fake, fake,
                              1 << 20, ctypes.addressof(info)) == _native.EINVAL
    assert "encode plan" in _native.last_error()
    assert L.gaans_run_decode(addr, None, fake, 1 << 20, None, None, None, fake, fake,
                              ctypes.addressof(status)) == _native.EINVAL
    assert "decode plan" in _native.last_error()
    assert L.gaans_run_encode(None, None, fake, None, None, None, fake, 1 << 20, fake, fake,
                              1 << 20, ctypes.addressof(info)) == _native.EINVAL
    assert ctypes.sizeof(plan) == _native.PLAN_BYTES


def test_call_structs_match_the_header(tmp_path):
    # the ctypes mirrors of gaans_encode_call / gaans_decode_call against the
    # C compiler's offsets and sizes for the header's structs
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    probes = []
    for cname, cls in (("gaans_encode_call", _native.EncodeCall),
                       ("gaans_decode_call", _native.DecodeCall)):
        probes.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            member = {"in0": "in[0]", "in1": "in[1]", "in2": "in[2]",
                      "in3": "in[3]"}.get(fname, fname)
            probes.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {member}));')
    src = tmp_path / "probe.c"
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"gaans_w64.h\"\n"
                   "int main(void) {\n" + "\n".join(probes) + "\nreturn 0;\n}\n")
    exe = tmp_path / "probe"
    subprocess.run([cc, "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True,
                               text=True).stdout.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, cls in (("gaans_encode_call", _native.EncodeCall),
                       ("gaans_decode_call", _native.DecodeCall)):
        assert got[(cname, "size")] == ctypes.sizeof(cls)
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, (cname, fname)


def test_call_struct_entries_reject_bad_arguments():
    L = _native.lib()
    assert L.gaans_run_encode_call(None) == _native.EINVAL
    assert L.gaans_run_decode_call(None) == _native.EINVAL
    plan = (ctypes.c_uint64 * (_native.PLAN_BYTES // 8))()  # not filled by gaans_plan_*
    info = (ctypes.c_uint64 * 3)()
    status = (ctypes.c_uint32 * 2)()
    fake = 1 << 20  # never dereferenced: the runs stop at the plan check
    e = _native.EncodeCall(plan=ctypes.addressof(plan), in0=fake, workspace_dev=fake,
                           workspace_bytes=1 << 20, ctrl_dev=fake, out_dev=fake,
                           out_bytes=1 << 20, info_host=ctypes.addressof(info))
    assert L.gaans_run_encode_call(ctypes.addressof(e)) == _native.EINVAL
    assert "encode plan" in _native.last_error()
    d = _native.DecodeCall(plan=ctypes.addressof(plan), payload_dev=fake, payload_bytes=1 << 20,
                           out_dev=fake, ctrl_dev=fake, status_host=ctypes.addressof(status))
    assert L.gaans_run_decode_call(ctypes.addressof(d)) == _native.EINVAL
    assert "decode plan" in _native.last_error()
