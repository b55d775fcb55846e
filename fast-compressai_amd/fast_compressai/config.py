"""Public configuration of ``accelerate``.

``AccelerationConfig`` has the reference's fields, defaults and accepted
values (``src/fast_compressai/config.py:14-101``), so configurations written
for it load here (plus ``segments``, the GA-ANS coding units per chunk: 1 to
256, or None for the coder's choice): ``p_ch`` (spelled ``P`` in a mapping; latent channels per
independently coded GA-ANS chunk) is a positive int or None, ``coder`` is
``"warp_div"`` (default) or ``"rans"``, ``budget`` a finite non-negative
number, ``execution_mode`` ``"sequential"`` or ``"overlap"``, the paths and
the device strings.  Validation is a table of per-field rules; a mapping is
merged with the keyword overrides, and a key given twice (``P`` and
``p_ch``, or a mapping key and the same keyword) is rejected.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass, fields
from typing import Any, Callable, Mapping


class ConfigurationError(ValueError):
    """Raised when an acceleration configuration is invalid."""


def _optional_str(value: Any) -> bool:
    return value is None or isinstance(value, str)


def _p_ch_ok(value: Any) -> bool:
    return value is None or (type(value) is int and value > 0)


def _budget_ok(value: Any) -> bool:
    return (isinstance(value, (int, float)) and not isinstance(value, bool)
            and math.isfinite(float(value)) and value >= 0)


# field -> (rule, what the field must be)
_RULES: dict[str, tuple[Callable[[Any], bool], str]] = {
    "p_ch": (_p_ch_ok, "P (p_ch) must be a positive integer or None"),
    "budget": (_budget_ok, "budget must be a finite, non-negative number"),
    "coder": (lambda v: v in ("warp_div", "rans"), "coder must be 'warp_div' or 'rans'"),
    "device": (_optional_str, "device must be a string or None"),
    "profile_path": (_optional_str, "profile_path must be a string or None"),
    "precision_config_path": (_optional_str, "precision_config_path must be a string or None"),
    "execution_mode": (lambda v: v in ("sequential", "overlap"),
                       "execution_mode must be 'sequential' or 'overlap'"),
    "segments": (lambda v: v is None or (type(v) is int and 1 <= v <= 256),
                 "segments must be an int in [1, 256] (coding units per chunk), or None (automatic)"),
}


@dataclass(frozen=True)
class AccelerationConfig:
    p_ch: int | None = None
    budget: float = 0.0
    coder: str = "warp_div"
    device: str | None = None
    profile_path: str | None = None
    precision_config_path: str | None = None
    execution_mode: str = "sequential"
    # GA-ANS coding units per chunk (beyond the reference's fields); None lets
    # the coder choose per shape
    segments: int | None = None

    def __post_init__(self) -> None:
        for name, (rule, message) in _RULES.items():
            if not rule(getattr(self, name)):
                raise ConfigurationError(message)

    @classmethod
    def from_value(cls, value: "AccelerationConfig | Mapping[str, Any] | None", *,
                   P: int | None = None, budget: float | None = None, device: str | None = None,
                   coder: str | None = None,
                   precision_config_path: str | None = None) -> "AccelerationConfig":
        """Build a config from None (defaults), an existing config (returned
        as is; keyword overrides are not combined with it) or a mapping,
        with the keyword arguments applied on top."""
        given = {k: v for k, v in (("p_ch", P), ("budget", budget), ("device", device),
                                   ("coder", coder),
                                   ("precision_config_path", precision_config_path))
                 if v is not None}
        if isinstance(value, cls):
            if given:
                raise ConfigurationError(
                    "an AccelerationConfig cannot be combined with P/budget/device/coder/"
                    "precision_config_path arguments")
            return value
        if value is None:
            base: dict[str, Any] = {}
        elif isinstance(value, Mapping):
            base = _canonical_keys(value)
        else:
            raise ConfigurationError("config must be None, an AccelerationConfig or a mapping")
        twice = sorted(set(base) & set(given))
        if twice:
            raise ConfigurationError(
                f"{', '.join(twice)} given both in the config mapping and as an argument")
        merged = {**base, **given}
        known = {f.name for f in fields(cls)}
        extra = sorted(map(str, set(merged) - known))
        if extra:
            raise ConfigurationError(f"unknown acceleration config field(s): {', '.join(extra)}")
        return cls(**merged)

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


def _canonical_keys(mapping: Mapping[str, Any]) -> dict[str, Any]:
    """The mapping with ``P`` renamed to ``p_ch`` (only one of the two may
    be present)."""
    data = dict(mapping)
    if "P" in data:
        if "p_ch" in data:
            raise ConfigurationError("give P or p_ch, not both")
        data["p_ch"] = data.pop("P")
    return data
