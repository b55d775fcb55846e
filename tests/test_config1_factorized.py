"""The CPU-plumbing workload -- CompressAI FactorizedPrior(N=8, M=12), seed 0,
``update(force=True)``, a 1x3x64x64 uniform input, so a 12x4x4 latent with
16-bit CDFs (reference ``tests/test_factorized_prior_smoke.py:18-63``) -- run
through the GA-ANS HIP path.  CompressAI is absent, so the model is the
restatement in ``tests/compressai_factorized.py``.

GPU: ``accelerate(model, P)`` for P in {1, 4, 12} gives payload bytes equal
to the oracle's encode of CompressAI's quantize, symbols and y_hat equal to
the closed forms, and x_hat = g_s(y_hat).clamp(0, 1); CompressAI-format Rans64
streams of that latent (the ``coder="rans"`` stream format) decode on the GPU
to the same y_hat.  CPU: the restated table construction is pinned by hand
computed quantized CDFs and the CompressAI table invariants."""

import numpy as np
import pytest
import torch

import oracle
import fast_compressai
from compressai_factorized import config1_model, pmf_to_quantized_cdf
from fast_compressai.coders import WarpDivPayload


def _input(seed: int = 0) -> torch.Tensor:
    return torch.rand(1, 3, 64, 64, generator=torch.Generator().manual_seed(seed))


def test_quantized_cdf_hand_computed():
    # exact halves: no rounding, no stealing
    assert pmf_to_quantized_cdf([0.5, 0.5]) == [0, 32768, 65536]
    # two zero-frequency symbols steal one each from the only symbol above one
    assert pmf_to_quantized_cdf([1.0, 0.0, 0.0]) == [0, 65534, 65535, 65536]
    # a tail below 2^-16 rounds to zero and steals from the first of the lowest
    assert pmf_to_quantized_cdf([0.25, 0.25, 0.5, 1e-9]) == [0, 16383, 32767, 65535, 65536]
    # round half away from zero (std::round), then the integer rescale to 2^16:
    # 3/8 -> 24576, 5/8 -> 40960 sum to 2^16 exactly
    assert pmf_to_quantized_cdf([0.375, 0.625]) == [0, 24576, 65536]
    # rescale by integer division when the rounded total is not 2^16:
    # round(0.3 * 65536) = 19661, round(0.3 * 65536) = 19661 -> total 39322;
    # each becomes 65536 * 19661 // 39322 = 32768
    assert pmf_to_quantized_cdf([0.3, 0.3]) == [0, 32768, 65536]


def test_config1_tables_and_latent_shape():
    model = config1_model(0)
    eb = model.entropy_bottleneck
    cdf, lengths, offsets = eb._quantized_cdf, eb._cdf_length, eb._offset
    assert tuple(cdf.shape) == (12, 23)
    assert lengths.tolist() == [23] * 12 and offsets.tolist() == [-10] * 12
    for row in cdf.tolist():
        assert row[0] == 0 and row[-1] == 65536
        assert all(a < b for a, b in zip(row, row[1:]))
    with torch.no_grad():
        y = model.g_a(_input())
    assert tuple(y.shape) == (1, 12, 4, 4)


@pytest.mark.gpu
@pytest.mark.parametrize("p_ch", [1, 4, 12])
def test_config1_accelerate_matches_oracle(gpu_device, p_ch):
    print("case: config1 FactorizedPrior(8, 12) 1x3x64x64 P", p_ch, flush=True)
    model = config1_model(0)
    fast = fast_compressai.accelerate(model, P=p_ch, device=str(gpu_device))
    x = _input().to(gpu_device)
    eb = fast.model.entropy_bottleneck
    tabs = [t.cpu().numpy() for t in (eb._quantized_cdf, eb._cdf_length, eb._offset)]
    with torch.inference_mode():
        y = fast.model.g_a(x)
        med = eb._get_medians().detach().reshape(-1)
        out = fast.compress(x)
        payload = out["strings"][0]
        assert isinstance(payload, WarpDivPayload) and out["shape"] == (4, 4)
        rec = fast.decompress(out["strings"], out["shape"])
        y_hat = fast._coder.decode_latents(out["strings"], out["shape"])
    y_np, med_np = y.cpu().numpy(), med.cpu().numpy()
    symbols = oracle.quantize(y_np, med_np)
    assert np.array_equal(symbols, torch.round(y - med.reshape(1, -1, 1, 1)).int().cpu().numpy())
    want = oracle.gaans_encode(symbols.reshape(1, -1), None, *tabs, p_ch,
                               segments=payload.segments)
    assert payload.to_bytes() == want
    want_y_hat = oracle.dequantize(symbols, med_np)
    assert np.array_equal(y_hat.cpu().numpy(), want_y_hat)
    with torch.inference_mode():
        x_hat = fast.model.g_s(torch.from_numpy(want_y_hat).to(gpu_device)).clamp_(0, 1)
    assert torch.equal(rec["x_hat"], x_hat)

    # the same latent as a CompressAI Rans64 stream (coder="rans" format)
    idx = np.repeat(np.arange(12, dtype=np.int32), 16).reshape(1, -1)
    stream = oracle.rans64_encode(symbols.reshape(-1), idx.reshape(-1), *tabs)
    y_hat2 = fast._coder.decode_latents([[stream]], (4, 4))
    assert np.array_equal(y_hat2.cpu().numpy(), want_y_hat)
