"""Seeded synthetic latents and 16-bit quantized CDF tables.

Shapes of the coder benchmarks: a 512x768 image under a 16x-downsampling
M=192 factorized prior (1x192x32x48), a mean-scale hyperprior
(GaussianConditional-style per-element table indexes), a 2160x3840 image
(1x320x136x240) and a 64-image batch (64x192x32x48) in a skewed and a
near-uniform draw.

Tables follow CompressAI's layout (``_quantized_cdf`` rows zero-padded to
``Lmax``, ``_cdf_length = pmf_length + 2``, ``_offset = -pmf_center``; the
last symbol of a table is the escape bin).  The pmf quantizer here is this
module's own (every bin gets at least one count, the remainder goes to the
largest bin); it is not CompressAI's ``pmf_to_quantized_cdf``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

PRECISION = 16
TOTAL = 1 << PRECISION


def quantize_pmf(pmf: np.ndarray, tail: float) -> np.ndarray:
    """pmf (n,) + tail mass -> CDF of n + 2 entries, 0 .. 65536, every bin >= 1."""
    probs = np.concatenate([np.asarray(pmf, dtype=np.float64), [max(tail, 0.0)]])
    probs = np.clip(probs, 0.0, None)
    probs = probs / probs.sum()
    n = probs.size
    freq = np.floor(probs * (TOTAL - n)).astype(np.int64) + 1
    freq[int(np.argmax(freq))] += TOTAL - int(freq.sum())
    cdf = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(freq, out=cdf[1:])
    assert cdf[-1] == TOTAL and np.all(np.diff(cdf) >= 1)
    return cdf.astype(np.int32)


def laplace_pmf(scale: float, radius: int) -> tuple[np.ndarray, float]:
    k = np.arange(-radius, radius + 1, dtype=np.float64)

    def cdf(x):
        return np.where(x < 0, 0.5 * np.exp(np.minimum(x, 0) / scale),
                        1.0 - 0.5 * np.exp(-np.maximum(x, 0) / scale))

    pmf = cdf(k + 0.5) - cdf(k - 0.5)
    return pmf, max(0.0, 1.0 - float(pmf.sum()))


def gaussian_pmf(scale: float, radius: int) -> tuple[np.ndarray, float]:
    from scipy.special import ndtr

    k = np.arange(-radius, radius + 1, dtype=np.float64)
    pmf = ndtr((k + 0.5) / scale) - ndtr((k - 0.5) / scale)
    return pmf, max(0.0, 1.0 - float(pmf.sum()))


def build_tables(pmfs_tails: list[tuple[np.ndarray, float]]):
    """-> cdfs [M, Lmax] int32 (zero-padded), cdf_sizes [M], offsets [M]."""
    cdf_rows = [quantize_pmf(p, t) for p, t in pmfs_tails]
    Lmax = max(r.size for r in cdf_rows)
    cdfs = np.zeros((len(cdf_rows), Lmax), dtype=np.int32)
    for i, r in enumerate(cdf_rows):
        cdfs[i, : r.size] = r
    sizes = np.array([r.size for r in cdf_rows], dtype=np.int32)
    offsets = np.array([-((p.size - 1) // 2) for p, _ in pmfs_tails], dtype=np.int32)
    return cdfs, sizes, offsets


@dataclass
class Workload:
    name: str
    symbols: np.ndarray          # int32 [B, N]
    indexes: np.ndarray | None   # int32 [B, N]; None = channel-major (table = channel)
    cdfs: np.ndarray
    cdf_sizes: np.ndarray
    offsets: np.ndarray
    channels: int
    p_ch: int
    raw_rgb_bytes: int           # B * H * W * 3 of the source images

    @property
    def batch(self) -> int:
        return int(self.symbols.shape[0])

    @property
    def n(self) -> int:
        return int(self.symbols.shape[1])

    def explicit_indexes(self) -> np.ndarray:
        if self.indexes is not None:
            return self.indexes
        hw = self.n // self.channels
        row = np.repeat(np.arange(self.channels, dtype=np.int32), hw)
        return np.broadcast_to(row, self.symbols.shape).copy()


def _factorized(name, B, C, H, W, scale_lo, scale_hi, max_cdf, P, img_hw, seed):
    rng = np.random.default_rng(seed)
    scales = np.exp(rng.uniform(math.log(scale_lo), math.log(scale_hi), C))
    max_radius = (max_cdf - 3) // 2
    tabs = []
    for s in scales:
        radius = int(min(max_radius, max(1, math.ceil(s * 20.7))))
        tabs.append(laplace_pmf(float(s), radius))
    cdfs, sizes, offsets = build_tables(tabs)
    lap = rng.laplace(0.0, scales[None, :, None], size=(B, C, H * W))
    symbols = np.rint(lap).astype(np.int32).reshape(B, C * H * W)
    return Workload(name, symbols, None, cdfs, sizes, offsets, C, P,
                    B * img_hw[0] * img_hw[1] * 3)


def coder_512x768(seed: int = 0, batch: int = 1, p_ch: int = 4) -> Workload:
    """1x192x32x48 symbols (512x768 RGB, M=192, 16x downsampling), per-channel
    Laplacian scale log-uniform [0.1, 8], CDFs <= 64 entries, P = 4."""
    return _factorized("factorized 1x192x32x48 (512x768 RGB, M=192)", batch, 192, 32, 48,
                       0.1, 8.0, 64, p_ch, (512, 768), seed)


def highres_2160x3840(seed: int = 0, p_ch: int = 8) -> Workload:
    """1x320x136x240 (2160x3840 RGB, M=320), scale log-uniform [0.1, 32],
    CDFs <= 256 entries, P = 8."""
    return _factorized("factorized 1x320x136x240 (2160x3840 RGB, M=320)", 1, 320, 136, 240,
                       0.1, 32.0, 256, p_ch, (2160, 3840), seed)


def batch_skew(seed: int = 0, p_ch: int = 16, batch: int = 64) -> Workload:
    """64x192x32x48 with Laplacian scale 0.1 in every channel (P(0) ~ 0.993)."""
    w = _factorized(f"batch {batch}x192x32x48 skew (scale 0.1)", batch, 192, 32, 48,
                    0.1, 0.1 + 1e-12, 64, p_ch, (512, 768), seed)
    return w


def batch_uniform(seed: int = 0, p_ch: int = 16, batch: int = 64) -> Workload:
    """64x192x32x48 near-uniform over [-127, 127] with 256-entry CDFs: the pmf
    covers [-127, 126] (254 values) and 127 takes the escape path."""
    rng = np.random.default_rng(seed)
    C, HW = 192, 32 * 48
    pmf = np.full(254, 1.0 / 255.0)
    cdfs, sizes, offsets = build_tables([(pmf, 1.0 / 255.0)] * C)
    offsets[:] = -127
    symbols = rng.integers(-127, 128, size=(batch, C * HW), dtype=np.int32)
    return Workload(f"batch {batch}x192x32x48 near-uniform +-127", symbols, None, cdfs, sizes,
                    offsets, C, p_ch, batch * 512 * 768 * 3)


def hyperprior_512x768(seed: int = 0, p_ch: int = 4):
    """Mean-scale hyperprior: y 1x192x32x48 with per-element indexes into 64
    Gaussian tables (scales log-spaced 0.11 .. 256, tail mass 1e-9), means
    N(0, 1); z 1x128x8x12 factorized.  Returns (y workload, z workload,
    y latents fp32, means fp32)."""
    rng = np.random.default_rng(seed)
    scale_table = np.exp(np.linspace(math.log(0.11), math.log(256.0), 64))
    multiplier = 6.109410204869  # -Phi^-1(1e-9 / 2)
    tabs = [gaussian_pmf(float(s), int(math.ceil(s * multiplier))) for s in scale_table]
    cdfs, sizes, offsets = build_tables(tabs)
    C, H, W = 192, 32, 48
    idx = rng.integers(0, 64, size=(1, C * H * W), dtype=np.int32)
    means = rng.standard_normal((1, C * H * W)).astype(np.float32)
    noise = rng.standard_normal((1, C * H * W)) * scale_table[idx]
    y = (means.astype(np.float64) + noise).astype(np.float32)
    symbols = np.rint((y - means).astype(np.float32)).astype(np.int32)
    yw = Workload("hyperprior y 1x192x32x48 (64 Gaussian tables)", symbols, idx, cdfs, sizes,
                  offsets, C, p_ch, 512 * 768 * 3)
    zw = _factorized("hyperprior z 1x128x8x12", 1, 128, 8, 12, 0.1, 8.0, 64,
                     min(p_ch, 128), (512, 768), seed + 1)
    return yw, zw, y, means
