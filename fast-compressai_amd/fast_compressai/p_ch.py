"""GA-ANS chunk size (P_ch) selection, measured with this coder.

``choose_p_ch`` keeps the reference's policy
(``src/fast_compressai/policies/p_ch.py:35-88``): among the measured P values,
take the largest one whose codec-to-inference time ratio is within
``relative_tolerance`` of 1 (balanced co-design, lower bpp for larger P),
else the one closest to balance (ties to the larger P); a run of small
codec-time changes between neighbouring P values is reported as a plateau.
``sweep_p_ch`` measures P values on a model with this repository's coder:
the reference's sweep (``src/fast_compressai/profiling/p_ch.py:16-84``) runs
inside its calibration pipeline, which is not part of this build, so here it
takes the sample images directly.
"""

from __future__ import annotations

import math
import statistics
from dataclasses import dataclass
from typing import Any, Mapping, Sequence

import torch


@dataclass(frozen=True)
class PChSelection:
    selected_p_ch: int
    status: str
    reason: str
    relative_error: float
    plateau: Mapping[str, object]


def legal_p_candidates(channel_count: int,
                       candidates: Sequence[int] | None = None) -> tuple[int, ...]:
    """Sorted distinct integer candidates in [1, channel_count]."""
    if type(channel_count) is not int or channel_count < 1:
        raise ValueError("channel_count must be a positive integer")
    pool = range(1, channel_count + 1) if candidates is None else candidates
    legal = sorted({p for p in pool if type(p) is int and 1 <= p <= channel_count})
    if not legal:
        raise ValueError("no legal P_ch candidates")
    return tuple(legal)


def default_p_candidates(channel_count: int) -> tuple[int, ...]:
    return legal_p_candidates(channel_count, (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96,
                                              128, 192, 256, 320))


def _positive(value: object, name: str) -> float:
    if (isinstance(value, bool) or not isinstance(value, (int, float))
            or not math.isfinite(float(value)) or value <= 0):
        raise ValueError(f"{name} must be a finite positive number")
    return float(value)


def choose_p_ch(measurements: Sequence[Mapping[str, object]], *,
                relative_tolerance: float = 0.10, plateau_delta: float = 0.05,
                plateau_patience: int = 2) -> PChSelection:
    """Pick P from records holding ``p_ch``, ``inference_total_ms`` and
    ``codec_total_ms`` (records without a positive integer ``p_ch`` are
    skipped)."""
    if not 0 <= relative_tolerance < 1:
        raise ValueError("relative_tolerance must be in [0, 1)")
    if plateau_delta < 0:
        raise ValueError("plateau_delta must be non-negative")
    if type(plateau_patience) is not int or plateau_patience < 1:
        raise ValueError("plateau_patience must be positive")
    rows = []  # (p, ratio error, codec ms)
    for m in measurements:
        p = m.get("p_ch")
        if type(p) is not int or p < 1:
            continue
        inference = _positive(m.get("inference_total_ms"), "inference_total_ms")
        codec = _positive(m.get("codec_total_ms"), "codec_total_ms")
        rows.append((p, abs(codec / inference - 1.0), codec))
    if not rows:
        raise ValueError("no usable P_ch measurements")
    rows.sort()
    pairs = [{"from_p_ch": a[0], "to_p_ch": b[0],
              "relative_delta": abs(b[2] - a[2]) / max(a[2], 1e-12)}
             for a, b in zip(rows, rows[1:])]
    plateau: dict[str, object] = {"detected": False, "pairs": pairs}
    streak = 0
    for i, pair in enumerate(pairs):
        streak = streak + 1 if pair["relative_delta"] <= plateau_delta else 0
        if streak >= plateau_patience:
            plateau.update(detected=True, start_p_ch=pairs[i - streak + 1]["from_p_ch"],
                           end_p_ch=pair["to_p_ch"],
                           interpretation="codec-time changes within measurement variation")
            break
    balanced = [r for r in rows if r[1] <= relative_tolerance]
    if balanced:
        p, err, _ = max(balanced, key=lambda r: r[0])
        return PChSelection(p, "auto_selected", "largest_relative_error_pass", err, plateau)
    p, err, _ = min(rows, key=lambda r: (r[1], -r[0]))
    return PChSelection(p, "fallback_closest_balance", "no_candidate_within_relative_tolerance",
                        err, plateau)


def sweep_p_ch(model: Any, samples: Sequence[torch.Tensor], *,
               candidates: Sequence[int] | None = None, warmup: int = 1,
               repetitions: int = 3, relative_tolerance: float = 0.10,
               plateau_delta: float = 0.05, plateau_patience: int = 2,
               device: str = "cuda") -> tuple[PChSelection, tuple[dict, ...]]:
    """Measure each legal P on ``samples`` (GPU NCHW images in [0, 1]) with
    ``accelerate(model, P=p)``: median inference and codec milliseconds of
    compress and decompress (event-timed phases), bpp of the payloads, and
    the balance the policy selects on.  Returns ``(selection, records)``."""
    from .api import accelerate

    if not samples:
        raise ValueError("sweep_p_ch needs at least one sample image")
    if type(warmup) is not int or warmup < 0 or type(repetitions) is not int or repetitions < 1:
        raise ValueError("warmup must be >= 0 and repetitions >= 1")
    channels = _latent_channels(model, samples[0], device)
    pool = legal_p_candidates(channels, candidates or default_p_candidates(channels))
    records = []
    for p in pool:
        fast = accelerate(model, P=p, device=device)
        times: dict[str, list[float]] = {}
        bits = pixels = 0
        for rep in range(warmup + repetitions):
            for x in samples:
                t: dict[str, float] = {}
                out = fast._coder.compress(x, timing=t)
                fast._coder.decompress(out["strings"], out["shape"], timing=t)
                if rep >= warmup:
                    for k, v in t.items():
                        times.setdefault(k, []).append(v)
                    if rep == warmup:
                        bits += 8 * sum(int(s.packed.numel()) for s in out["strings"])
                        pixels += int(x.size(0)) * int(x.size(-2)) * int(x.size(-1))
        med = {k: statistics.median(v) for k, v in times.items()}
        inference = med["compress_inference_ms"] + med["decompress_inference_ms"]
        codec = med["compress_codec_ms"] + med["decompress_codec_ms"]
        records.append({
            "p_ch": p, "bpp": bits / pixels, **med,
            "inference_total_ms": inference, "codec_total_ms": codec,
            "codec_to_inference_ratio": codec / max(inference, 1e-12),
            "sample_count": len(samples), "warmup": warmup, "repetitions": repetitions,
            "payload_semantics": "device_local_warp_div_packed_payload",
        })
    selection = choose_p_ch(records, relative_tolerance=relative_tolerance,
                            plateau_delta=plateau_delta, plateau_patience=plateau_patience)
    for r in records:
        r["relative_time_error"] = abs(r["codec_to_inference_ratio"] - 1.0)
        r["passed_balance"] = r["relative_time_error"] <= relative_tolerance
        r["selected"] = r["p_ch"] == selection.selected_p_ch
    return selection, tuple(records)


def _latent_channels(model: Any, sample: torch.Tensor, device: str) -> int:
    """Channels of y (the latent P chunks; a hyperprior's z clamps P to its
    own channel count), from one analysis pass of the accelerated model."""
    from .api import accelerate

    latents = accelerate(model, P=1, device=device)._coder.analyze(sample)
    y = latents[0] if isinstance(latents, tuple) else latents
    return int(y.size(1))
