"""``accelerate()`` routing and the ``FastModel`` wrapper.

Keeps the reference's entry point (``src/fast_compressai/api.py:132-192``,
``:322-330``, ``:386-448``, ``:451-532``):
``accelerate(model, P=None, budget=None, *, config=None, device=None,
sample=None, coder=None, ...) -> FastModel``.  ``coder="warp_div"`` (the
default) deep-copies a FactorizedPrior to the GPU and routes
``compress``/``decompress`` through the GA-ANS HIP coder with ``P`` latent
channels per chunk; ``coder="rans"`` keeps the model's own entropy path.
Beyond the reference (whose warp_div path accepts only FactorizedPrior,
``api.py:177-182``), ScaleHyperprior and MeanScaleHyperprior models are
routed too: z through the factorized path, y through the fused
GaussianConditional kernels (``coders/hyperprior.py``).

Out of scope here (mixed-precision operator selection, not the coder path):
``calibration_data``, ``precision_config_path`` and ``sample`` profiling;
they raise ``ConfigurationError`` instead of being silently ignored.
"""

from __future__ import annotations

import copy
from dataclasses import asdict, dataclass, field
from typing import Any, Mapping

import torch
from torch import nn

from .config import AccelerationConfig, ConfigurationError


@dataclass(frozen=True)
class AccelerationReport:
    """Status of what ``accelerate`` applied (fields of the reference's
    ``AccelerationReport``, ``api.py:88-124``)."""

    status: str
    model_class: str
    adapter_family: str
    p_ch: int | None
    quality_budget: float
    quality_metric: str
    profiling_status: str
    precision_selection_status: str
    selected_candidate: str
    psnr_drop_db: float | None
    reference_latency_ms: float | None
    candidate_latency_ms: float | None
    coder_status: str
    p_ch_applied: bool
    runtime_status: str
    speedup: float | None
    message: str
    p_ch_selection_status: str = "explicit"
    p_ch_selection_reason: str | None = None
    p_ch_sweep: tuple[Mapping[str, Any], ...] = field(default_factory=tuple)

    @property
    def accelerated(self) -> bool:
        return self.runtime_status == "applied" and self.speedup is not None and self.speedup > 1.0

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


class FastModel(nn.Module):
    """Wrapper that keeps a model's public compression paths; when a GA-ANS
    coder is attached, ``compress``/``decompress`` go through it."""

    def __init__(self, model: nn.Module, device: str | None = None) -> None:
        super().__init__()
        self.model = model
        if device is not None:
            self.to(device)

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        return self.model(*args, **kwargs)

    def compress(self, *args: Any, **kwargs: Any) -> Any:
        coder = self.__dict__.get("_coder")
        if coder is not None:
            return coder.compress(*args, **kwargs)
        return self.model.compress(*args, **kwargs)

    def decompress(self, *args: Any, **kwargs: Any) -> Any:
        coder = self.__dict__.get("_coder")
        if coder is not None:
            return coder.decompress(*args, **kwargs)
        return self.model.decompress(*args, **kwargs)

    def compress_many(self, inputs: Any) -> list:
        """``compress`` of every input; with ``execution_mode="overlap"`` the
        transforms and the coder run on two streams (``pipeline.py``)."""
        pipeline = self.__dict__.get("_pipeline")
        if pipeline is not None:
            return pipeline.compress_many(inputs)
        return [self.compress(x) for x in inputs]

    def decompress_many(self, items: Any) -> list:
        """``decompress`` of every ``compress`` result (dicts with ``strings``
        and ``shape``), overlapped like ``compress_many``."""
        pipeline = self.__dict__.get("_pipeline")
        if pipeline is not None:
            return pipeline.decompress_many(items)
        return [self.decompress(it["strings"], it["shape"]) for it in items]

    def update(self, *args: Any, **kwargs: Any) -> Any:
        return self.model.update(*args, **kwargs)

    def state_dict(self, *args: Any, **kwargs: Any) -> Any:
        return self.model.state_dict(*args, **kwargs)

    def load_state_dict(self, *args: Any, **kwargs: Any) -> Any:
        return self.model.load_state_dict(*args, **kwargs)

    def __getattr__(self, name: str) -> Any:
        try:
            return super().__getattr__(name)
        except AttributeError:
            modules = object.__getattribute__(self, "_modules")
            model = modules.get("model")
            if model is not None:
                return getattr(model, name)
            raise


def compile(model: nn.Module, config: Any = None) -> FastModel:  # noqa: A001 - reference name
    """Wrap ``model`` without changing any of its paths (reference ``compile``)."""
    if not isinstance(model, nn.Module):
        raise TypeError(f"model must be an instance of torch.nn.Module, got {type(model).__name__}")
    device = None
    if isinstance(config, Mapping):
        device = config.get("device")
    elif config is not None:
        device = getattr(config, "device", None)
    return FastModel(model, device=device)


_ENTROPY_CONTRACT = ("_quantized_cdf", "_cdf_length", "_offset", "_get_medians", "channels")


def _is_factorized_prior(model: nn.Module) -> bool:
    """CompressAI installed: exactly ``compressai.models.FactorizedPrior``
    (reference ``api.py:177-182``).  Without CompressAI: a model of that
    class name implementing its contract (``g_a``, ``g_s`` and an
    EntropyBottleneck-style ``entropy_bottleneck``)."""
    try:
        from compressai.models import FactorizedPrior
    except ImportError:
        FactorizedPrior = None
    if FactorizedPrior is not None:
        return type(model) is FactorizedPrior
    eb = getattr(model, "entropy_bottleneck", None)
    return (type(model).__name__ == "FactorizedPrior" and hasattr(model, "g_a")
            and hasattr(model, "g_s") and eb is not None
            and all(hasattr(eb, name) for name in _ENTROPY_CONTRACT))


_GC_CONTRACT = ("_quantized_cdf", "_cdf_length", "_offset", "scale_table")


def _hyperprior_kind(model: nn.Module) -> str | None:
    """"mean_scale" for CompressAI's ``MeanScaleHyperprior``, "scale" for
    ``ScaleHyperprior`` (exact types when CompressAI is installed; without
    it, a model of that class name implementing its contract: ``g_a``,
    ``g_s``, ``h_a``, ``h_s``, an EntropyBottleneck and a GaussianConditional
    with a scale table), else None."""
    try:
        from compressai.models import MeanScaleHyperprior, ScaleHyperprior
    except ImportError:
        MeanScaleHyperprior = ScaleHyperprior = None
    if MeanScaleHyperprior is not None:
        if type(model) is MeanScaleHyperprior:
            return "mean_scale"
        return "scale" if type(model) is ScaleHyperprior else None
    name = type(model).__name__
    if name not in ("MeanScaleHyperprior", "ScaleHyperprior"):
        return None
    eb = getattr(model, "entropy_bottleneck", None)
    gc = getattr(model, "gaussian_conditional", None)
    if (eb is None or gc is None
            or not all(hasattr(model, f) for f in ("g_a", "g_s", "h_a", "h_s"))
            or not all(hasattr(eb, f) for f in _ENTROPY_CONTRACT)
            or not all(hasattr(gc, f) for f in _GC_CONTRACT)):
        return None
    return "mean_scale" if name == "MeanScaleHyperprior" else "scale"


def accelerate(
    model: nn.Module,
    P: int | None = None,
    budget: float | None = None,
    *,
    config: AccelerationConfig | Mapping[str, Any] | None = None,
    device: str | None = None,
    sample: Any | None = None,
    coder: str | None = None,
    calibration_data: Any | None = None,
    dataset_name: str | None = None,
    precision_config_path: str | None = None,
    precision_config_output_dir: str | None = None,
) -> FastModel:
    """Attach the GA-ANS coder (``coder="warp_div"``) or keep the model's own
    RANS path (``coder="rans"``).  ``P`` is GA-ANS ``p_ch``."""
    if not isinstance(model, nn.Module):
        raise TypeError(f"model must be an instance of torch.nn.Module, got {type(model).__name__}")
    cfg = AccelerationConfig.from_value(config, P=P, budget=budget, device=device, coder=coder,
                                        precision_config_path=precision_config_path)
    if calibration_data is not None or cfg.precision_config_path is not None:
        raise ConfigurationError(
            "mixed-precision operator selection (calibration_data / precision_config_path) "
            "is not part of this coder build")
    del dataset_name, precision_config_output_dir
    p_status = "explicit" if cfg.p_ch is not None else "default"
    if cfg.coder == "warp_div":
        hyper = None if _is_factorized_prior(model) else _hyperprior_kind(model)
        if hyper is None and not _is_factorized_prior(model):
            raise ConfigurationError(
                "warp_div supports CompressAI FactorizedPrior, ScaleHyperprior and "
                "MeanScaleHyperprior")
        if sample is not None:
            raise ConfigurationError(
                "warp_div precision selection uses calibration_data; legacy sample profiling is unavailable")
        target = torch.device(cfg.device or "cuda")
        if target.type != "cuda":
            raise ConfigurationError("warp_div requires device='cuda'")
        if not torch.cuda.is_available():
            raise ConfigurationError("warp_div requires a GPU")
        runtime_model = copy.deepcopy(model).to(target).eval()
        p_ch = cfg.p_ch if cfg.p_ch is not None else 1
        if hyper is None:
            from .coders.factorized import FactorizedWarpDivCodec

            codec = FactorizedWarpDivCodec(runtime_model, p_ch, segments=cfg.segments)
        else:
            from .coders.hyperprior import HyperpriorWarpDivCodec

            codec = HyperpriorWarpDivCodec(runtime_model, p_ch, mean_scale=hyper == "mean_scale",
                                           segments=cfg.segments)
        wrapped = FastModel(runtime_model, device=str(target))
        wrapped._coder = codec
        from .pipeline import CodingPipeline

        wrapped._pipeline = CodingPipeline(codec, target, cfg.execution_mode)
        report = AccelerationReport(
            status="coder_applied", model_class=type(model).__qualname__,
            adapter_family="compressai", p_ch=p_ch, quality_budget=float(cfg.budget),
            quality_metric="psnr_drop_db", profiling_status="not_run",
            precision_selection_status="not_run", selected_candidate="fp32",
            psnr_drop_db=None, reference_latency_ms=None, candidate_latency_ms=None,
            coder_status="warp_div", p_ch_applied=True, runtime_status="not_applied",
            speedup=None, p_ch_selection_status=p_status,
            message=("The MI355X GA-ANS coder is applied to compress/decompress with P_ch="
                     f"{p_ch}; transforms stay FP32 and payloads are device-local; "
                     f"compress_many/decompress_many run {cfg.execution_mode}."),
        )
    else:
        if sample is not None:
            raise ConfigurationError("sample profiling (BF16 transform selection) is not part of this build")
        wrapped = FastModel(model, device=cfg.device)
        report = AccelerationReport(
            status="reference_only", model_class=type(model).__qualname__,
            adapter_family="compressai", p_ch=cfg.p_ch, quality_budget=float(cfg.budget),
            quality_metric="psnr_drop_db", profiling_status="not_run",
            precision_selection_status="not_run", selected_candidate="fp32",
            psnr_drop_db=None, reference_latency_ms=None, candidate_latency_ms=None,
            coder_status="rans", p_ch_applied=False, runtime_status="not_applied",
            speedup=None, p_ch_selection_status=p_status,
            message="Reference wrapper returned; the model's own RANS entropy path is kept.",
        )
    wrapped.acceleration_config = cfg
    wrapped.acceleration_report = report
    return wrapped
