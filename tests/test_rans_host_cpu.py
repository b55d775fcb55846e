"""CompressAI RANS on the host (no GPU): the CompressAI harness, this
library's host Rans64 decoder (gaans_rans64_decode_host) against the oracle,
and the routing of CompressAI strings.

CompressAI is not installed here, so its ``compressai.ans`` module is stood in
for by one whose RansEncoder / RansDecoder call the oracle's Rans64
restatement: that checks the harness's row handling and list conversion, not
CompressAI itself.  The host decoder is checked against streams the oracle
writes (the oracle's Rans64 restatement is pinned by hand-derived known
answers in test_oracle.py)."""

import math

import sys
import types

import numpy as np
import pytest
import torch

import oracle
from fast_compressai import synthetic
from fast_compressai.coders import (CompressAIANSBackend, CoderDependencyError, CoderInputError,
                                    gaans)
from fast_compressai.coders import _native
from fast_compressai.coders.rans_host import (GPU_STREAM_MS, HOST_STREAM_MS, decode_rows_host,
                                               rans64_route)


def _lengthed(cdfs, sizes):
    return np.array([list(r) for r in cdfs], dtype=np.int32), np.asarray(sizes, np.int32)


class _Enc:
    def encode_with_indexes(self, symbols, indexes, cdfs, sizes, offsets):
        assert all(type(v) is int for v in symbols[:4] + indexes[:4])  # lists of ints
        c, s = _lengthed(cdfs, sizes)
        return oracle.rans64_encode(symbols, indexes, c, s, offsets)


class _Dec:
    def decode_with_indexes(self, data, indexes, cdfs, sizes, offsets):
        assert isinstance(data, bytes) and type(indexes[0]) is int
        c, s = _lengthed(cdfs, sizes)
        return oracle.rans64_decode(data, indexes, c, s, offsets).tolist()


@pytest.fixture
def stand_in_compressai(monkeypatch):
    ans = types.ModuleType("compressai.ans")
    ans.RansEncoder, ans.RansDecoder = _Enc, _Dec
    pkg = types.ModuleType("compressai")
    pkg.ans = ans
    monkeypatch.setitem(sys.modules, "compressai", pkg)
    monkeypatch.setitem(sys.modules, "compressai.ans", ans)
    return ans


def test_route_by_estimated_time():
    # the host takes ceil(B / threads) stream times; the GPU one stream time
    per = math.ceil(GPU_STREAM_MS / HOST_STREAM_MS)  # streams a thread decodes in one GPU time
    for threads in (1, 4, 16):
        assert rans64_route(1, threads) == "host"
        assert rans64_route(threads * (per - 1), threads) == "host"
        assert rans64_route(threads * per + 1, threads) == "gpu"


def test_backend_needs_compressai(monkeypatch):
    monkeypatch.setitem(sys.modules, "compressai", None)
    assert rans64_route(1) == "host"  # this library's host decoder needs no CompressAI
    with pytest.raises(CoderDependencyError, match="CompressAI"):
        CompressAIANSBackend()


def test_rows_round_trip_through_the_harness(stand_in_compressai):
    w = synthetic.coder_512x768(seed=5, batch=2)
    B, C = 2, 12
    HW = w.n // 192
    sym = w.symbols[:, : C * HW]
    idx = np.repeat(np.arange(C, dtype=np.int32), HW)[None].repeat(B, 0)
    be = CompressAIANSBackend()
    strings = be.encode_rows(torch.from_numpy(sym), idx, w.cdfs[:C], w.cdf_sizes[:C],
                             w.offsets[:C])
    assert [s for s in strings] == [oracle.rans64_encode(sym[b], idx[b], w.cdfs[:C],
                                                         w.cdf_sizes[:C], w.offsets[:C])
                                    for b in range(B)]
    out = be.decode_rows(strings, idx, w.cdfs[:C], w.cdf_sizes[:C], w.offsets[:C])
    assert out.dtype == np.int32 and np.array_equal(out, sym)
    # small batches of CompressAI strings take the host route (table = channel)
    raw = tuple(torch.from_numpy(np.ascontiguousarray(a))
                for a in (w.cdfs[:C], w.cdf_sizes[:C], w.offsets[:C]))
    got = gaans.decode_compressai_strings(strings, None, raw, B, C * HW, C, "cpu")
    assert torch.equal(got, torch.from_numpy(sym))
    with pytest.raises(Exception, match="streams for"):
        be.decode_rows(strings[:1], idx, w.cdfs[:C], w.cdf_sizes[:C], w.offsets[:C])


def _streams(sym, idx, cdfs, sizes, offs):
    return [oracle.rans64_encode(sym[b], idx[b], cdfs, sizes, offs) for b in range(len(sym))]


@pytest.mark.parametrize("threads", [1, 3, 0])
def test_host_decoder_matches_the_oracle(threads):
    """Factorized rows (table = channel and the same as explicit indexes),
    one to several threads; rows with escapes on both sides."""
    w = synthetic.coder_512x768(seed=11, batch=5)
    C = 24
    HW = w.n // 192
    N = C * HW
    sym = np.ascontiguousarray(w.symbols[:, :N])
    sym[0, :50] = 300     # escapes above the tables' range
    sym[1, 100:140] = -77  # and below
    idx = np.repeat(np.arange(C, dtype=np.int32), HW)[None].repeat(len(sym), 0)
    cd, sz, of = w.cdfs[:C], w.cdf_sizes[:C], w.offsets[:C]
    strings = _streams(sym, idx, cd, sz, of)
    for b, s_ in enumerate(strings):  # the oracle's own decode agrees
        assert np.array_equal(oracle.rans64_decode(s_, idx[b], cd, sz, of), sym[b])
    got = decode_rows_host(strings, None, cd, sz, of, N=N, C=C, threads=threads)
    assert got.dtype == np.int32 and np.array_equal(got, sym)
    got = decode_rows_host(strings, idx, cd, sz, of, N=N, C=C, threads=threads)
    assert np.array_equal(got, sym)


def test_host_decoder_per_element_indexes_and_wide_tables():
    """Per-element indexes into 64 Gaussian tables of up to 3,133 entries
    (the mean-scale hyperprior's y), and values far outside every table."""
    yw, _, _, _ = synthetic.hyperprior_512x768()
    n = 20000
    sym = np.ascontiguousarray(yw.symbols[:, :n]).copy()
    idx = np.ascontiguousarray(yw.explicit_indexes()[:, :n])
    sym[0, ::997] = 2_000_000_000
    sym[0, 5::1013] = -2_000_000_000
    strings = _streams(sym, idx, yw.cdfs, yw.cdf_sizes, yw.offsets)
    got = decode_rows_host(strings, idx, yw.cdfs, yw.cdf_sizes, yw.offsets, N=n, C=1)
    assert np.array_equal(got, sym)


def test_host_decoder_rejects_bad_streams_and_indexes():
    w = synthetic.coder_512x768(seed=12, batch=2)
    C, HW = 6, w.n // 192
    N = C * HW
    sym = np.ascontiguousarray(w.symbols[:, :N])
    idx = np.repeat(np.arange(C, dtype=np.int32), HW)[None].repeat(2, 0)
    cd, sz, of = w.cdfs[:C], w.cdf_sizes[:C], w.offsets[:C]
    strings = _streams(sym, idx, cd, sz, of)
    with pytest.raises(CoderInputError, match="corrupt"):
        decode_rows_host([strings[0], strings[1][: len(strings[1]) // 2]], None, cd, sz, of,
                         N=N, C=C)
    with pytest.raises(CoderInputError, match="corrupt"):
        decode_rows_host([strings[0], strings[1][:-2]], None, cd, sz, of, N=N, C=C)  # not words
    bad = idx.copy()
    bad[1, 7] = C
    with pytest.raises(CoderInputError, match="outside"):
        decode_rows_host(strings, bad, cd, sz, of, N=N, C=C)
    broken = cd.copy()
    broken[2, 1] = broken[2, 0]  # not strictly increasing
    with pytest.raises(CoderInputError, match="strictly increasing"):
        decode_rows_host(strings, None, broken, sz, of, N=N, C=C)
    # an escape count past 8 nibbles: with the one-bin table [0, 65536] every
    # symbol is the escape bin and leaves the state as it is, so a state of
    # all ones gives bypass groups of 15, 15, ... (count 30 > 8)
    one = np.array([[0, 65536]], dtype=np.int32)
    ones = np.array([0xFFFFFFFF] * 4, dtype=np.uint32).tobytes()
    with pytest.raises(CoderInputError, match="corrupt"):
        decode_rows_host([ones], None, one, [2], [0], N=1, C=1)
    # a count of exactly 8, derived by hand: words (low first) 0x11111118,
    # 0x11111111 give x = 0x1111111111111118; the symbol leaves x as it is;
    # count nibble 8; seven raw nibbles 1 leave x = 0x11111111 < 2^31, so word
    # 0x00000001 comes in and gives the eighth nibble 1: raw = 0x11111111, odd
    # -> -(raw >> 1) - 1
    good = np.array([0x11111118, 0x11111111, 0x00000001], dtype="<u4").tobytes()
    got = decode_rows_host([good], None, one, [2], [0], N=1, C=1)
    assert got[0, 0] == -(0x11111111 >> 1) - 1
    # the same without the third word: the eighth nibble's refill reads past the end
    with pytest.raises(CoderInputError, match="corrupt"):
        decode_rows_host([good[:8]], None, one, [2], [0], N=1, C=1)
    L = _native.lib()
    assert L.gaans_rans64_decode_host(None, None, None, None, None, None, 1, 2, 1, 1, 1, 1, None,
                                      None) == _native.EINVAL
