"""The oracle reproduces the committed golden fixtures byte for byte
(tests/golden, written by tests/golden/make_golden.py), and decodes them."""

import numpy as np
import pytest

import oracle as O
from golden_cases import NAMES, load


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden_bytes(name):
    c = load(name)
    sym, cdfs, sizes, offs = c["symbols"], c["cdfs"], c["cdf_sizes"], c["offsets"]
    B, N = sym.shape
    idx = c["full_indexes"]
    payload = O.gaans_encode(sym, idx if c["explicit"] else None, cdfs, sizes, offs, c["p_ch"],
                             c["channels"], c["segments"])
    assert payload == c["payload"]
    assert np.array_equal(O.gaans_decode(payload, idx if c["explicit"] else None, B, N, cdfs,
                                         sizes, offs, c["p_ch"], c["channels"],
                                         c["segments"]), sym)
    for b in range(B):
        assert O.rans64_encode(sym[b], idx[b], cdfs, sizes, offs) == c["streams"][b]
        assert np.array_equal(O.rans64_decode(c["streams"][b], idx[b], cdfs, sizes, offs), sym[b])
    if name == "latents":
        assert np.array_equal(O.quantize(c["y"].reshape(B, c["channels"], -1), c["medians"])
                              .reshape(B, N), sym)
    if name == "gaussian":
        assert np.array_equal(O.build_indexes(c["scales"], c["scale_table"], float(c["bound"])),
                              c["indexes"])
        assert np.array_equal(O.quantize_elem(c["y"], c["means"]), sym)
