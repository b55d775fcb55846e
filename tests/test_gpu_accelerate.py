"""accelerate(model, P, coder="warp_div") end to end on the GPU with a
FactorizedPrior stand-in (tests/factorized_stub.py), mirroring
tests/gpu/test_factorized_gaans.py:34-98 of the reference: decoded latents
equal CompressAI's quantize -> dequantize, x_hat equals g_s of that, the
source model is not mutated, and bad payloads are rejected."""

from dataclasses import replace

import numpy as np
import pytest
import torch

import fast_compressai
from fast_compressai import synthetic
from fast_compressai.coders import CoderInputError, WarpDivPayload
from fast_compressai.config import ConfigurationError
from factorized_stub import FactorizedPrior

pytestmark = pytest.mark.gpu


def make_model(M=12, seed=20261015):
    torch.manual_seed(seed)
    w = synthetic.coder_512x768(seed=seed % 1000)
    rng = np.random.default_rng(seed)
    med = rng.normal(0, 0.2, M).astype(np.float32)
    return FactorizedPrior(M, w.cdfs[:M], w.cdf_sizes[:M], w.offsets[:M], med).eval()


@pytest.mark.parametrize("batch", [1, 2])
def test_gaans_matches_quantize_dequantize_for_p_and_batch(gpu_device, batch):
    model = make_model().to(gpu_device)
    x = torch.rand(batch, 3, 64, 64, device=gpu_device)
    with torch.inference_mode():
        y = model.g_a(x)
        eb = model.entropy_bottleneck
        med = eb._extend_ndims(eb._get_medians().detach(), 2).expand(batch, -1, -1, -1)
        expected_symbols = eb.quantize(y, "symbols", med)
        expected_y_hat = eb.dequantize(expected_symbols, med)
        expected_x_hat = model.g_s(expected_y_hat).clamp_(0, 1)
    for p_ch in (1, 4, 5, 12):
        print("case: accelerate batch", batch, "P", p_ch, flush=True)
        source = {k: v.clone() for k, v in model.state_dict().items()}
        fast = fast_compressai.accelerate(model, P=p_ch, device=str(gpu_device))
        assert fast.acceleration_report.coder_status == "warp_div"
        assert fast.acceleration_report.p_ch_applied
        with torch.inference_mode():
            stream = fast.compress(x)
            payload = stream["strings"][0]
            assert isinstance(payload, WarpDivPayload) and payload.p_ch == p_ch
            timing = {}
            out = fast.decompress(stream["strings"], stream["shape"], timing=timing)
            assert set(timing) == {"decompress_codec_ms", "decompress_inference_ms"}
            fast_eb = fast.model.entropy_bottleneck
            indexes = fast_eb._build_indexes((batch, 12, *stream["shape"]), device=gpu_device)
            symbols = fast._coder.backend.decode(
                payload, indexes.reshape(batch, -1).contiguous(),
                fast_eb._quantized_cdf.contiguous(), fast_eb._cdf_length.contiguous(),
                fast_eb._offset.contiguous()).reshape_as(expected_symbols)
        assert torch.equal(symbols, expected_symbols)
        assert torch.equal(out["x_hat"], expected_x_hat)
        assert all(torch.equal(v, model.state_dict()[k]) for k, v in source.items())


def test_invalid_model_state_and_metadata_are_rejected(gpu_device):
    model = make_model().to(gpu_device)
    with pytest.raises(CoderInputError, match="P"):
        fast_compressai.accelerate(model, P=13, device=str(gpu_device))
    with pytest.raises(ConfigurationError):
        fast_compressai.accelerate(model, P=4, device="cpu")
    fresh = make_model()
    fresh.entropy_bottleneck._quantized_cdf = torch.zeros(0, dtype=torch.int32)
    with pytest.raises(CoderInputError, match="update"):
        fast_compressai.accelerate(fresh, P=4, device=str(gpu_device))
    fast = fast_compressai.accelerate(model, P=4, device=str(gpu_device))
    with torch.inference_mode():
        stream = fast.compress(torch.rand(1, 3, 64, 64, device=gpu_device))
    payload = stream["strings"][0]
    print("case: accelerate negative decompress calls", flush=True)
    with pytest.raises(CoderInputError):
        fast.decompress(stream["strings"], (8, 8))
    with pytest.raises(CoderInputError):
        fast.decompress([[b"cpu-rans"]], stream["shape"])
    with pytest.raises(CoderInputError, match="match"):
        fast.decompress([replace(payload, p_ch=3, chunk_len=48)], stream["shape"])
    with pytest.raises(CoderInputError, match="match"):
        fast.decompress([replace(payload, coding_fingerprint="0" * 64)], stream["shape"])
    with pytest.raises(CoderInputError, match="header"):
        corrupted = payload.packed.clone()
        corrupted[0] ^= 1
        fast.decompress([replace(payload, packed=corrupted)], stream["shape"])
