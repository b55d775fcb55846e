"""CompressAI RANS host harness and the routing of CompressAI strings (no GPU).

CompressAI is not installed here, so its ``compressai.ans`` module is stood in
for by one whose RansEncoder / RansDecoder call the oracle's Rans64
restatement: that checks the harness's row handling and list conversion and
the host route of ``decode_compressai_strings``, not CompressAI itself."""

import sys
import types

import numpy as np
import pytest
import torch

import oracle
from fast_compressai import synthetic
from fast_compressai.coders import CompressAIANSBackend, CoderDependencyError, gaans
from fast_compressai.coders.rans_host import RANS64_GPU_MIN_STREAMS, rans64_route


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


def test_route_by_batch_and_availability():
    assert rans64_route(1, True) == "host"
    assert rans64_route(RANS64_GPU_MIN_STREAMS - 1, True) == "host"
    assert rans64_route(RANS64_GPU_MIN_STREAMS, True) == "gpu"
    assert rans64_route(1, False) == "gpu"


def test_backend_needs_compressai(monkeypatch):
    monkeypatch.setitem(sys.modules, "compressai", None)
    assert rans64_route(1) == "gpu"
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
