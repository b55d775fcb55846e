"""CPU tests of the Python surface (mirrors tests/test_warp_div_api.py and
tests/test_accelerate_api.py of the reference)."""

import importlib
from unittest import mock

import pytest
import torch
from torch import nn

import fast_compressai
from fast_compressai.coders import _native
from fast_compressai.coders.errors import CoderDependencyError, CoderInputError
from fast_compressai.coders.warp_div import WarpDivBackend, WarpDivPayload, _validate_inputs


class CompressAIStyleMock(nn.Module):
    def forward(self, x):
        return {"x_hat": x, "likelihoods": {"y": torch.ones_like(x)}}

    def compress(self, x):
        return {"strings": [[b"mock"]], "shape": tuple(x.shape)}

    def decompress(self, strings, shape):
        return {"x_hat": torch.zeros(shape), "strings": strings}


def test_catalog_is_limited_to_two_coders():
    assert fast_compressai.coder_catalog() == ("compressai-rans", "warp_div")
    with pytest.raises(ValueError):
        fast_compressai.create_coder("other")


def test_capability_is_lazy_and_reports_missing_library():
    with mock.patch("fast_compressai.coders.capabilities.torch.cuda.is_available",
                    return_value=True), \
            mock.patch("fast_compressai.coders.capabilities._native.library_available",
                       return_value=False):
        cap = fast_compressai.warp_div_capability("cuda:0")
    assert not cap.available and cap.backend == "warp_div" and "not built" in cap.reason
    with mock.patch("fast_compressai.coders.capabilities.torch.cuda.is_available",
                    return_value=True):
        assert not fast_compressai.warp_div_capability("cpu").available


def test_backend_constructor_reports_unavailable_library():
    with mock.patch("fast_compressai.coders.warp_div.warp_div_capability") as capability:
        capability.return_value = mock.Mock(available=False, reason="not built")
        with pytest.raises(CoderDependencyError, match="not built"):
            WarpDivBackend()


def test_missing_library_fails_loudly(tmp_path):
    with mock.patch.object(_native, "library_path", return_value=str(tmp_path / "none.so")), \
            mock.patch.object(_native, "_lib", None):
        with pytest.raises(CoderDependencyError):
            _native.lib()


def test_python_import_does_not_load_native_library():
    assert importlib.import_module("fast_compressai.coders.warp_div") is not None


def test_payload_rejects_non_gpu_data():
    with pytest.raises(CoderInputError):
        WarpDivPayload(packed=torch.zeros(128, dtype=torch.uint8),
                       chunk_ends=torch.zeros((1, 1), dtype=torch.uint32), header_bytes=80,
                       chunk_len=4, p_ch=1, batch=1, symbols_per_batch=4, cdf_count=1)


def test_input_contract_rejects_wrong_dtype_before_library():
    with pytest.raises(CoderInputError):
        _validate_inputs(torch.zeros((1, 4), dtype=torch.float32),
                         torch.zeros((1, 4), dtype=torch.int32),
                         torch.tensor([[0, 65536]], dtype=torch.int32),
                         torch.tensor([2], dtype=torch.int32),
                         torch.tensor([0], dtype=torch.int32), 1)


def test_p_maps_to_p_ch_and_budget_is_independent():
    with pytest.raises(fast_compressai.ConfigurationError):
        fast_compressai.accelerate(CompressAIStyleMock(), P=8, budget=0.1, device="cpu")
    acc = fast_compressai.accelerate(CompressAIStyleMock(), P=8, budget=0.1, device="cpu",
                                     coder="rans")
    assert isinstance(acc, fast_compressai.FastModel)
    assert acc.acceleration_config.p_ch == 8 and acc.acceleration_report.p_ch == 8
    assert acc.acceleration_report.status == "reference_only"
    assert acc.acceleration_report.runtime_status == "not_applied"
    assert acc.acceleration_report.speedup is None and not acc.acceleration_report.accelerated


def test_wrapper_preserves_model_paths():
    acc = fast_compressai.accelerate(CompressAIStyleMock(), P=4, budget=0.2, coder="rans")
    value = torch.ones(1, 2)
    assert "x_hat" in acc(value)
    strings = acc.compress(value)
    assert strings["shape"] == (1, 2)
    assert acc.decompress(strings, (1, 2))["x_hat"].shape == (1, 2)
    assert set(acc.state_dict()) == set()


def test_config_alias_and_validation():
    cfg = fast_compressai.AccelerationConfig.from_value({"P": 16, "budget": 0.05})
    assert cfg.p_ch == 16 and cfg.budget == 0.05 and cfg.to_dict()["p_ch"] == 16
    with pytest.raises(fast_compressai.ConfigurationError):
        fast_compressai.AccelerationConfig.from_value({"P": 4, "p_ch": 4})
    for value in (True, 0, -1, 1.5):
        with pytest.raises(fast_compressai.ConfigurationError):
            fast_compressai.AccelerationConfig(p_ch=value)
    with pytest.raises(fast_compressai.ConfigurationError):
        fast_compressai.AccelerationConfig(budget=-0.1)
    with pytest.raises(fast_compressai.ConfigurationError):
        fast_compressai.AccelerationConfig(budget=float("inf"))
    with pytest.raises(fast_compressai.ConfigurationError):
        fast_compressai.AccelerationConfig.from_value(fast_compressai.AccelerationConfig(), P=2)


def test_default_coder_is_warp_div_and_requires_supported_model():
    with pytest.raises(fast_compressai.ConfigurationError,
                       match="warp_div supports CompressAI FactorizedPrior, ScaleHyperprior"):
        fast_compressai.accelerate(CompressAIStyleMock(), P=4, device="cuda")


def test_hyperprior_models_are_routed_to_warp_div():
    # the stand-ins pass the model check; without a GPU the next check fails
    from hyperprior_stub import make_hyperprior

    from fast_compressai.api import _hyperprior_kind

    for mean_scale in (True, False):
        model = make_hyperprior(mean_scale=mean_scale)
        assert _hyperprior_kind(model) == ("mean_scale" if mean_scale else "scale")
        if not torch.cuda.is_available():
            with pytest.raises(fast_compressai.ConfigurationError, match="requires a GPU"):
                fast_compressai.accelerate(model, P=4, device="cuda")
    assert _hyperprior_kind(CompressAIStyleMock()) is None


def test_out_of_scope_options_raise():
    with pytest.raises(fast_compressai.ConfigurationError):
        fast_compressai.accelerate(CompressAIStyleMock(), coder="rans", calibration_data=object())


def test_compile_remains_compatible():
    assert isinstance(fast_compressai.compile(nn.Identity()), fast_compressai.FastModel)


def test_compressai_rans_backend_needs_compressai():
    try:
        import compressai  # noqa: F401
    except ImportError:
        with pytest.raises(CoderDependencyError):
            fast_compressai.create_coder("compressai-rans")
