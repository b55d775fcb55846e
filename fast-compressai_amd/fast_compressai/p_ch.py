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

import numpy as np
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
    """The distinct candidates that are chunk widths the coder accepts for
    ``channel_count`` latent channels (ints in [1, channel_count]), ascending;
    all widths when ``candidates`` is None."""
    if isinstance(channel_count, bool) or not isinstance(channel_count, int) or channel_count < 1:
        raise ValueError(f"channel_count must be a positive int, got {channel_count!r}")
    if candidates is None:
        return tuple(range(1, channel_count + 1))
    width_ok = np.frompyfunc(lambda p: type(p) is int and 0 < p <= channel_count, 1, 1)
    pool = np.array(list(candidates), dtype=object)
    kept = np.unique(pool[width_ok(pool).astype(bool)].astype(np.int64)) if pool.size else pool
    if kept.size == 0:
        raise ValueError(f"none of the P_ch candidates is a width in [1, {channel_count}]")
    return tuple(int(p) for p in kept)


def default_p_candidates(channel_count: int) -> tuple[int, ...]:
    return legal_p_candidates(channel_count, (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96,
                                              128, 192, 256, 320))


@dataclass(frozen=True)
class _Measured:
    """One usable measurement: P, the codec's time and its imbalance
    ``|codec / inference - 1|``."""

    p: int
    codec_ms: float
    imbalance: float


def _measured(record: Mapping[str, object]) -> _Measured | None:
    p = record.get("p_ch")
    if type(p) is not int or p < 1:
        return None  # not a P measurement
    times = []
    for key in ("inference_total_ms", "codec_total_ms"):
        v = record.get(key)
        ok = isinstance(v, (int, float)) and not isinstance(v, bool) and math.isfinite(v) and v > 0
        if not ok:
            raise ValueError(f"{key} of the P_ch={p} record must be a finite positive number")
        times.append(float(v))
    inference, codec = times
    return _Measured(p, codec, abs(codec / inference - 1.0))


def _plateau(points: Sequence[_Measured], delta: float, patience: int) -> dict[str, object]:
    """Neighbouring P values whose codec times differ by at most ``delta``
    (relative) are flat steps; the first ``patience`` flat steps in a row are
    reported as a plateau (diagnostic only)."""
    codec = np.array([pt.codec_ms for pt in points])
    rel = np.abs(np.diff(codec)) / np.maximum(codec[:-1], 1e-12)
    steps = [{"from_p_ch": a.p, "to_p_ch": b.p, "relative_delta": float(r)}
             for a, b, r in zip(points, points[1:], rel)]
    out: dict[str, object] = {"detected": False, "pairs": steps}
    if len(steps) < patience:
        return out
    flat = (rel <= delta).astype(np.int64)
    # flat steps in a window of `patience` ending at each step
    window = np.convolve(flat, np.ones(patience, dtype=np.int64))[: len(flat)]
    ends = np.flatnonzero(window >= patience)
    if ends.size:
        end = int(ends[0])
        out.update(detected=True, start_p_ch=steps[end - patience + 1]["from_p_ch"],
                   end_p_ch=steps[end]["to_p_ch"],
                   interpretation="codec-time changes within measurement variation")
    return out


def choose_p_ch(measurements: Sequence[Mapping[str, object]], *,
                relative_tolerance: float = 0.10, plateau_delta: float = 0.05,
                plateau_patience: int = 2) -> PChSelection:
    """Pick P from records holding ``p_ch``, ``inference_total_ms`` and
    ``codec_total_ms`` (records without a positive integer ``p_ch`` are
    skipped).  Each candidate is ranked by ``(balanced, P)`` when it is
    balanced (imbalance within ``relative_tolerance``), else by ``(not
    balanced, -imbalance, P)``: the best is the largest balanced P (fewer
    chunks: fewer flushed states, lower bpp) or, when none is balanced, the
    most balanced P, ties to the larger one."""
    if not 0 <= relative_tolerance < 1:
        raise ValueError(f"relative_tolerance must lie in [0, 1), got {relative_tolerance!r}")
    if plateau_delta < 0:
        raise ValueError(f"plateau_delta must be >= 0, got {plateau_delta!r}")
    if type(plateau_patience) is not int or plateau_patience < 1:
        raise ValueError(f"plateau_patience must be an int >= 1, got {plateau_patience!r}")
    points = sorted((pt for pt in map(_measured, measurements) if pt is not None),
                    key=lambda pt: (pt.p, pt.codec_ms))
    if not points:
        raise ValueError("no usable P_ch measurement among the records")
    plateau = _plateau(points, plateau_delta, plateau_patience)

    def rank(pt: _Measured):
        if pt.imbalance <= relative_tolerance:
            return (1, pt.p, 0.0)
        return (0, -pt.imbalance, pt.p)

    best = max(points, key=rank)
    if best.imbalance <= relative_tolerance:
        return PChSelection(best.p, "auto_selected", "largest_relative_error_pass",
                            best.imbalance, plateau)
    return PChSelection(best.p, "fallback_closest_balance",
                        "no_candidate_within_relative_tolerance", best.imbalance, plateau)


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
