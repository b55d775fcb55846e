"""Public configuration of ``accelerate``.

``AccelerationConfig`` keeps the reference's fields and validation
(``src/fast_compressai/config.py:14-101``): ``P`` is stored as ``p_ch``
(latent channels per independently coded GA-ANS chunk), ``coder`` is
``"warp_div"`` (default) or ``"rans"``, and a mapping may spell ``P`` or
``p_ch`` but not both.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass
from typing import Any, Mapping


class ConfigurationError(ValueError):
    """Raised when an acceleration configuration is invalid."""


_FIELDS = {"p_ch", "budget", "coder", "device", "profile_path", "precision_config_path",
           "execution_mode"}


@dataclass(frozen=True)
class AccelerationConfig:
    p_ch: int | None = None
    budget: float = 0.0
    coder: str = "warp_div"
    device: str | None = None
    profile_path: str | None = None
    precision_config_path: str | None = None
    execution_mode: str = "sequential"

    def __post_init__(self) -> None:
        if self.p_ch is not None and (type(self.p_ch) is not int or self.p_ch <= 0):
            raise ConfigurationError("P (p_ch) must be a positive integer or None")
        if self.coder not in {"warp_div", "rans"}:
            raise ConfigurationError("coder must be 'warp_div' or 'rans'")
        if isinstance(self.budget, bool) or not isinstance(self.budget, (int, float)):
            raise ConfigurationError("budget must be a non-negative finite RD/quality value")
        if self.budget < 0 or not math.isfinite(float(self.budget)):
            raise ConfigurationError("budget must be a non-negative finite RD/quality value")
        for name in ("device", "profile_path", "precision_config_path"):
            value = getattr(self, name)
            if value is not None and not isinstance(value, str):
                raise ConfigurationError(f"{name} must be a string or None")
        if self.execution_mode not in {"sequential", "overlap"}:
            raise ConfigurationError("execution_mode must be 'sequential' or 'overlap'")

    @classmethod
    def from_value(cls, value: "AccelerationConfig | Mapping[str, Any] | None", *,
                   P: int | None = None, budget: float | None = None, device: str | None = None,
                   coder: str | None = None,
                   precision_config_path: str | None = None) -> "AccelerationConfig":
        overrides = {"p_ch": P, "budget": budget, "device": device, "coder": coder,
                     "precision_config_path": precision_config_path}
        if value is None:
            return cls(p_ch=P, budget=0.0 if budget is None else budget, device=device,
                       coder="warp_div" if coder is None else coder,
                       precision_config_path=precision_config_path)
        if isinstance(value, cls):
            if any(v is not None for v in overrides.values()):
                raise ConfigurationError("do not combine config with P/budget/device/coder overrides")
            return value
        if isinstance(value, Mapping):
            data = dict(value)
            if "P" in data:
                if "p_ch" in data:
                    raise ConfigurationError("use only one of P and p_ch")
                data["p_ch"] = data.pop("P")
            for key, override in overrides.items():
                if override is not None:
                    if key in data:
                        raise ConfigurationError(f"{key} specified both in config and as an argument")
                    data[key] = override
            unknown = set(data) - _FIELDS
            if unknown:
                raise ConfigurationError(
                    f"unknown acceleration config field(s): {', '.join(sorted(map(str, unknown)))}")
            try:
                return cls(**data)
            except TypeError as exc:
                raise ConfigurationError(str(exc)) from exc
        raise ConfigurationError("config must be None, AccelerationConfig, or a mapping")

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)
