"""P_ch selection policy and pipeline configuration (no GPU).

``choose_p_ch`` follows the reference's policy
(``src/fast_compressai/policies/p_ch.py:35-88``); the expectations below are
worked out by hand from that policy's rules: largest P within tolerance,
else closest balance with ties to the larger P, plateau = ``patience``
consecutive neighbour pairs whose codec time changes by at most ``delta``.
"""

import pytest

import fast_compressai
from fast_compressai import (AccelerationConfig, CodingPipeline, ConfigurationError,
                             choose_p_ch, default_p_candidates, legal_p_candidates)


def rec(p, inference, codec):
    return {"p_ch": p, "inference_total_ms": inference, "codec_total_ms": codec}


def test_largest_balanced_p_is_selected():
    # ratios 0.5, 0.92, 1.08, 1.5: P=4 and P=8 pass 10%, the larger wins
    sel = choose_p_ch([rec(1, 2.0, 1.0), rec(4, 2.0, 1.84), rec(8, 2.0, 2.16),
                       rec(16, 2.0, 3.0)])
    assert (sel.selected_p_ch, sel.status, sel.reason) == (
        8, "auto_selected", "largest_relative_error_pass")
    assert sel.relative_error == pytest.approx(0.08)


def test_fallback_is_closest_balance_with_ties_to_larger_p():
    # errors 0.8, 0.5, 0.5: no pass; P=4 and P=8 tie, the larger wins
    sel = choose_p_ch([rec(1, 1.0, 0.2), rec(4, 1.0, 0.5), rec(8, 1.0, 1.5)])
    assert (sel.selected_p_ch, sel.status) == (8, "fallback_closest_balance")
    assert sel.reason == "no_candidate_within_relative_tolerance"
    assert sel.relative_error == pytest.approx(0.5)


def test_unusable_records_are_skipped_and_bad_times_rejected():
    sel = choose_p_ch([{"p_ch": 0}, {"p_ch": True}, {"p_ch": "4"}, rec(2, 1.0, 1.0)])
    assert sel.selected_p_ch == 2 and sel.relative_error == 0.0
    with pytest.raises(ValueError, match="no usable"):
        choose_p_ch([{"p_ch": None}])
    for bad in (0.0, -1.0, float("nan"), float("inf"), True, "1"):
        with pytest.raises(ValueError, match="codec_total_ms"):
            choose_p_ch([rec(1, 1.0, bad)])
    with pytest.raises(ValueError):
        choose_p_ch([rec(1, 1.0, 1.0)], relative_tolerance=1.0)
    with pytest.raises(ValueError):
        choose_p_ch([rec(1, 1.0, 1.0)], plateau_delta=-0.1)
    with pytest.raises(ValueError):
        choose_p_ch([rec(1, 1.0, 1.0)], plateau_patience=0)


def test_plateau_detection():
    # codec ms by P: 1.0, 2.0 (+100%), 2.04 (+2%), 2.08 (+2%), 3.0: two small
    # steps in a row from P=4 to P=16
    rows = [rec(1, 10.0, 1.0), rec(4, 10.0, 2.0), rec(8, 10.0, 2.04), rec(16, 10.0, 2.0808),
            rec(32, 10.0, 3.0)]
    sel = choose_p_ch(list(reversed(rows)))  # order of the records does not matter
    assert sel.plateau["detected"] is True
    assert (sel.plateau["start_p_ch"], sel.plateau["end_p_ch"]) == (4, 16)
    assert [p["from_p_ch"] for p in sel.plateau["pairs"]] == [1, 4, 8, 16]
    assert sel.plateau["pairs"][0]["relative_delta"] == pytest.approx(1.0)
    assert choose_p_ch(rows, plateau_patience=3).plateau["detected"] is False


def test_candidate_lists():
    assert legal_p_candidates(4) == (1, 2, 3, 4)
    assert legal_p_candidates(12, [12, 3, 3, 0, 13, 2.0, True]) == (3, 12)
    assert default_p_candidates(192) == (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96, 128, 192)
    assert default_p_candidates(5) == (1, 2, 3, 4)
    with pytest.raises(ValueError):
        legal_p_candidates(0)
    with pytest.raises(ValueError):
        legal_p_candidates(4, [5, 6])


def test_pipeline_configuration():
    assert AccelerationConfig(execution_mode="overlap").execution_mode == "overlap"
    with pytest.raises(ConfigurationError):
        AccelerationConfig(execution_mode="async")
    with pytest.raises(ConfigurationError):
        CodingPipeline(object(), "cuda:0", mode="async")
    with pytest.raises(ConfigurationError):
        CodingPipeline(object(), "cpu", mode="overlap")
    assert "sweep_p_ch" in fast_compressai.__all__


def test_sequential_helpers_without_a_coder_use_the_model():
    class Model(fast_compressai.api.nn.Module):
        def compress(self, x):
            return {"strings": [x], "shape": (1, 1)}

        def decompress(self, strings, shape):
            return {"x_hat": strings[0]}

    fast = fast_compressai.accelerate(Model(), coder="rans")
    outs = fast.compress_many([1, 2])
    assert [o["strings"][0] for o in outs] == [1, 2]
    assert [r["x_hat"] for r in fast.decompress_many(outs)] == [1, 2]


def test_compressai_string_packing():
    from fast_compressai.coders import gaans
    from fast_compressai.coders.factorized import is_compressai_strings

    buf, offs = gaans.pack_streams([b"\1\2\3\4", b"", b"\5\6\7\10\11\12\13\14"], "cpu")
    assert offs.tolist() == [0, 4, 4, 12] and offs.dtype.is_floating_point is False
    assert bytes(buf.numpy()) == b"\1\2\3\4\5\6\7\10\11\12\13\14"
    for bad in ([], [b"abc"], ["abcd"], [b"abcd", 3]):
        with pytest.raises(fast_compressai.CoderInputError):
            gaans.pack_streams(bad, "cpu")
    assert is_compressai_strings([b"ab", bytearray(b"cd")])
    assert not is_compressai_strings([]) and not is_compressai_strings([b"ab", None])
    assert not is_compressai_strings(b"abcd")
