"""ScaleHyperprior / MeanScaleHyperprior stand-ins implementing the parts of
CompressAI's contract the GA-ANS hyperprior codec uses (CompressAI is not
installed here).  Follows CompressAI's published structure: ``y = g_a(x)``;
``z = h_a(|y|)`` (scale) or ``h_a(y)`` (mean-scale); ``h_s(z_hat)`` gives the
scales, or scales and means (``chunk(2, 1)``); the GaussianConditional has a
log-spaced ``scale_table`` (0.11 .. 256, 64 levels), a ``lower_bound_scale``
with ``bound`` = 0.11 and one quantized CDF per scale.  The tables come from
this repository's own Gaussian quantizer (``synthetic.gaussian_pmf``), not
from CompressAI's ``pmf_to_quantized_cdf``."""

import math

import numpy as np
import torch
from torch import nn

from factorized_stub import EntropyBottleneck
from fast_compressai import synthetic


class LowerBound(nn.Module):
    def __init__(self, bound: float) -> None:
        super().__init__()
        self.register_buffer("bound", torch.tensor([float(bound)]))

    def forward(self, x):
        return torch.max(x, self.bound)


class GaussianConditional(nn.Module):
    def __init__(self, scale_table, cdfs, sizes, offsets, scale_bound: float = 0.11) -> None:
        super().__init__()
        self.register_buffer("scale_table", torch.as_tensor(scale_table, dtype=torch.float32))
        self.lower_bound_scale = LowerBound(scale_bound)
        self.register_buffer("_quantized_cdf", torch.as_tensor(np.asarray(cdfs, np.int32)))
        self.register_buffer("_cdf_length", torch.as_tensor(np.asarray(sizes, np.int32)))
        self.register_buffer("_offset", torch.as_tensor(np.asarray(offsets, np.int32)))

    def build_indexes(self, scales):
        """CompressAI's loop: (L - 1) minus the scale-table entries (but the
        last) that the lower-bounded scale does not exceed."""
        scales = self.lower_bound_scale(scales)
        indexes = scales.new_full(scales.size(), len(self.scale_table) - 1).int()
        for s in self.scale_table[:-1]:
            indexes -= (scales <= s).int()
        return indexes


def gaussian_tables():
    scale_table = np.exp(np.linspace(math.log(0.11), math.log(256.0), 64)).astype(np.float32)
    multiplier = 6.109410204869  # -Phi^-1(1e-9 / 2), CompressAI's tail mass 1e-9
    tabs = [synthetic.gaussian_pmf(float(s), int(math.ceil(float(s) * multiplier)))
            for s in scale_table]
    cdfs, sizes, offsets = synthetic.build_tables(tabs)
    return scale_table, cdfs, sizes, offsets


class _Hyperprior(nn.Module):
    mean_scale = False

    def __init__(self, M: int = 16, Nz: int = 8, seed: int = 0) -> None:
        super().__init__()
        torch.manual_seed(seed)
        out = 2 * M if self.mean_scale else M
        self.g_a = nn.Sequential(nn.Conv2d(3, M, 4, stride=4), nn.Conv2d(M, M, 1))
        self.h_a = nn.Sequential(nn.Conv2d(M, Nz, 2, stride=2))
        self.h_s = nn.Sequential(nn.ConvTranspose2d(Nz, out, 2, stride=2))
        self.g_s = nn.Sequential(nn.ConvTranspose2d(M, 3, 4, stride=4))
        with torch.no_grad():
            self.g_a[1].weight.mul_(6.0)
            self.h_s[0].weight.mul_(3.0)
        w = synthetic.coder_512x768(seed=seed % 1000)
        rng = np.random.default_rng(seed)
        self.entropy_bottleneck = EntropyBottleneck(
            Nz, w.cdfs[:Nz], w.cdf_sizes[:Nz], w.offsets[:Nz],
            rng.normal(0, 0.2, Nz).astype(np.float32))
        table, cdfs, sizes, offsets = gaussian_tables()
        self.gaussian_conditional = GaussianConditional(table, cdfs, sizes, offsets)

    def compress(self, x):
        raise NotImplementedError("the stand-in has no CPU RANS path")


class ScaleHyperprior(_Hyperprior):
    mean_scale = False


class MeanScaleHyperprior(_Hyperprior):
    mean_scale = True


def make_hyperprior(mean_scale: bool, M: int = 16, Nz: int = 8, seed: int = 0):
    cls = MeanScaleHyperprior if mean_scale else ScaleHyperprior
    return cls(M, Nz, seed).eval()


def reference_y_hat(model, x):
    """CompressAI's quantize -> dequantize of y for the stand-in (torch)."""
    with torch.no_grad():
        y = model.g_a(x)
        z = model.h_a(y if model.mean_scale else torch.abs(y))
        eb = model.entropy_bottleneck
        med = eb._get_medians().detach().reshape(1, -1, 1, 1)
        z_hat = eb.dequantize(eb.quantize(z, "symbols", med), med)
        params = model.h_s(z_hat)
        if model.mean_scale:
            scales, means = params.chunk(2, 1)
            symbols = torch.round(y - means).int()
            y_hat = symbols.type_as(means) + means
        else:
            scales, means = params, None
            symbols = torch.round(y).int()
            y_hat = symbols.float()
        indexes = model.gaussian_conditional.build_indexes(scales)
    return y, z, z_hat, scales, means, symbols, indexes, y_hat
