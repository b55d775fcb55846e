"""CompressAI's ``FactorizedPrior(N, M)`` restated for the tests (CompressAI is
not installed here and cannot be fetched).  TEST INFRASTRUCTURE: it stands in
for the model of the reference's CPU smoke test
(``tests/test_factorized_prior_smoke.py:18-63``: ``FactorizedPrior(N=8, M=12)``,
``update(force=True)``, a 1x3x64x64 input, hence a 12x4x4 latent) so that the
GA-ANS path can run on that exact shape and on tables built the way
CompressAI builds them.

Restated from CompressAI's published algorithms (``compressai>=1.2``, the
unpinned dependency of the reference's ``pyproject.toml:16-18``):

* ``FactorizedPrior``: ``g_a`` = four 5x5 stride-2 convolutions (padding 2)
  with GDN between them, ``g_s`` the transposed mirror with inverse GDN
  (output padding 1).  GDN is ``x / sqrt(beta + conv1x1(x^2, gamma))`` with
  CompressAI's initial ``beta = 1``, ``gamma = 0.1 I`` (the non-negative
  reparametrisation is left out: it only changes the stored parameters).
* ``EntropyBottleneck(M)``: the factorized density with filters (3, 3, 3),
  ``init_scale = 10``, matrices filled with ``log(expm1(1 / scale /
  filters[i + 1]))`` (``scale = 10 ** (1 / 4)``), biases uniform in
  [-0.5, 0.5], factors zero, quantiles ``[-10, 0, 10]``, tail mass 1e-9;
  ``update()`` evaluates the pmf on ``[median - minima, median + maxima]`` with
  the likelihood ``sigmoid(upper) - sigmoid(lower)`` and appends the tail mass;
  ``_cdf_length = pmf_length + 2``, ``_offset = -minima``.
* ``pmf_to_quantized_cdf`` (CompressAI ``cpp_exts/ops/ops.cpp``, ported there
  from ryg_rans): ``round(p * 2^16)`` per symbol, rescaled to the total by
  integer division, prefix sums, last entry forced to ``2^16``, then every
  zero-frequency symbol steals one from the lowest frequency above one.

The exact values CompressAI would produce from ``torch.manual_seed`` depend on
its parameter creation order and are **parity unpinned** here; what the tests
rely on is the shape (12x4x4 latent, 23-entry tables, offsets -10) and the
CompressAI semantics of ``quantize`` / ``dequantize`` / ``_build_indexes``.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn


def pmf_to_quantized_cdf(pmf, precision: int = 16) -> list[int]:
    """Quantized CDF (``len(pmf) + 1`` entries, 0 .. 2^precision, strictly
    increasing) of a pmf whose entries are fp32 values."""
    p32 = np.asarray(pmf, dtype=np.float32)
    if p32.ndim != 1 or p32.size == 0 or np.any(~np.isfinite(p32)) or np.any(p32 < 0):
        raise ValueError("pmf must be a non-empty vector of finite non-negative values")
    one = 1 << precision
    # std::round of the fp32 product (exact: a power-of-two scale), half away from zero
    scaled = p32 * np.float32(one)
    freq = [0] + [int(math.floor(float(v) + 0.5)) for v in scaled]
    total = sum(freq)
    if total == 0:
        raise ValueError("at least one pmf entry must be non-zero")
    freq = [(one * f) // total for f in freq]
    cdf = list(np.cumsum(freq, dtype=np.int64))
    cdf = [int(c) for c in cdf]
    cdf[-1] = one
    for i in range(len(cdf) - 1):
        if cdf[i] == cdf[i + 1]:
            best_freq, best = None, -1
            for j in range(len(cdf) - 1):
                f = cdf[j + 1] - cdf[j]
                if f > 1 and (best_freq is None or f < best_freq):
                    best_freq, best = f, j
            if best < 0:
                raise ValueError("no frequency to steal")
            if best < i:
                for j in range(best + 1, i + 1):
                    cdf[j] -= 1
            else:
                for j in range(i + 1, best + 1):
                    cdf[j] += 1
    return cdf


class GDN(nn.Module):
    def __init__(self, channels: int, inverse: bool = False) -> None:
        super().__init__()
        self.inverse = inverse
        self.beta = nn.Parameter(torch.ones(channels))
        self.gamma = nn.Parameter(0.1 * torch.eye(channels).reshape(channels, channels, 1, 1))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        norm = torch.sqrt(F.conv2d(x * x, self.gamma, self.beta))
        return x * norm if self.inverse else x / norm


class EntropyBottleneck(nn.Module):
    tail_mass = 1e-9

    def __init__(self, channels: int, filters=(3, 3, 3), init_scale: float = 10.0) -> None:
        super().__init__()
        self.channels = int(channels)
        self.filters = tuple(int(f) for f in filters)
        full = (1,) + self.filters + (1,)
        scale = init_scale ** (1 / (len(self.filters) + 1))
        for i in range(len(self.filters) + 1):
            init = float(np.log(np.expm1(1 / scale / full[i + 1])))
            self.register_parameter(
                f"_matrix{i}", nn.Parameter(torch.full((channels, full[i + 1], full[i]), init)))
            bias = torch.empty(channels, full[i + 1], 1)
            nn.init.uniform_(bias, -0.5, 0.5)
            self.register_parameter(f"_bias{i}", nn.Parameter(bias))
            if i < len(self.filters):
                self.register_parameter(
                    f"_factor{i}", nn.Parameter(torch.zeros(channels, full[i + 1], 1)))
        self.quantiles = nn.Parameter(
            torch.tensor([-init_scale, 0.0, init_scale]).repeat(channels, 1, 1))
        self.register_buffer("_quantized_cdf", torch.zeros(0, dtype=torch.int32))
        self.register_buffer("_cdf_length", torch.zeros(0, dtype=torch.int32))
        self.register_buffer("_offset", torch.zeros(0, dtype=torch.int32))

    def _logits_cumulative(self, inputs: torch.Tensor) -> torch.Tensor:
        logits = inputs
        for i in range(len(self.filters) + 1):
            logits = torch.matmul(F.softplus(getattr(self, f"_matrix{i}").detach()), logits)
            logits = logits + getattr(self, f"_bias{i}").detach()
            if i < len(self.filters):
                logits = logits + torch.tanh(getattr(self, f"_factor{i}").detach()) * torch.tanh(
                    logits)
        return logits

    def _likelihood(self, inputs: torch.Tensor):
        lower = self._logits_cumulative(inputs - 0.5)
        upper = self._logits_cumulative(inputs + 0.5)
        return torch.sigmoid(upper) - torch.sigmoid(lower), lower, upper

    @torch.no_grad()
    def update(self, force: bool = False) -> bool:
        if self._offset.numel() > 0 and not force:
            return False
        q = self.quantiles.detach()
        medians = q[:, 0, 1]
        minima = torch.clamp(torch.ceil(medians - q[:, 0, 0]).int(), min=0)
        maxima = torch.clamp(torch.ceil(q[:, 0, 2] - medians).int(), min=0)
        pmf_start = medians - minima
        pmf_length = maxima + minima + 1
        max_length = int(pmf_length.max())
        samples = torch.arange(max_length, device=q.device)[None, :] + pmf_start[:, None, None]
        pmf, lower, upper = self._likelihood(samples)
        pmf = pmf[:, 0, :]
        tail = torch.sigmoid(lower[:, 0, :1]) + torch.sigmoid(-upper[:, 0, -1:])
        cdf = torch.zeros((self.channels, max_length + 2), dtype=torch.int32)
        for c in range(self.channels):
            n = int(pmf_length[c])
            prob = torch.cat((pmf[c, :n], tail[c]), dim=0).cpu().numpy()
            row = pmf_to_quantized_cdf(prob)
            cdf[c, : len(row)] = torch.tensor(row, dtype=torch.int32)
        dev = self.quantiles.device
        self._quantized_cdf = cdf.to(dev)
        self._cdf_length = (pmf_length + 2).int().to(dev)
        self._offset = (-minima).int().to(dev)
        return True

    def _get_medians(self) -> torch.Tensor:
        return self.quantiles[:, :, 1:2]

    @staticmethod
    def _extend_ndims(tensor: torch.Tensor, n: int) -> torch.Tensor:
        return tensor.reshape(-1, *([1] * n)) if n > 0 else tensor.reshape(-1)

    def _build_indexes(self, size, device=None) -> torch.Tensor:
        view = [1] * len(size)
        view[1] = -1
        idx = torch.arange(size[1], device=device).view(*view).int()
        return idx.repeat(size[0], 1, *size[2:])

    @staticmethod
    def quantize(inputs, mode, means=None):
        out = inputs.clone()
        if means is not None:
            out -= means
        out = torch.round(out)
        if mode == "dequantize":
            return out + means if means is not None else out
        assert mode == "symbols", mode
        return out.int()

    @staticmethod
    def dequantize(inputs, means=None, dtype=torch.float):
        if means is not None:
            out = inputs.type_as(means)
            out += means
            return out
        return inputs.type(dtype)


def _conv(cin: int, cout: int) -> nn.Conv2d:
    return nn.Conv2d(cin, cout, 5, stride=2, padding=2)


def _deconv(cin: int, cout: int) -> nn.ConvTranspose2d:
    return nn.ConvTranspose2d(cin, cout, 5, stride=2, padding=2, output_padding=1)


class FactorizedPrior(nn.Module):
    def __init__(self, N: int, M: int) -> None:
        super().__init__()
        self.entropy_bottleneck = EntropyBottleneck(M)
        self.g_a = nn.Sequential(_conv(3, N), GDN(N), _conv(N, N), GDN(N), _conv(N, N), GDN(N),
                                 _conv(N, M))
        self.g_s = nn.Sequential(_deconv(M, N), GDN(N, True), _deconv(N, N), GDN(N, True),
                                 _deconv(N, N), GDN(N, True), _deconv(N, 3))

    def update(self, force: bool = False) -> bool:
        return self.entropy_bottleneck.update(force=force)

    def compress(self, x):
        raise NotImplementedError("the restated model has no CPU RANS path")


def config1_model(seed: int = 0) -> FactorizedPrior:
    """FactorizedPrior(N=8, M=12) under ``torch.manual_seed(seed)``, tables
    built with ``update(force=True)``, in eval mode on the CPU."""
    torch.manual_seed(seed)
    model = FactorizedPrior(N=8, M=12)
    assert model.update(force=True)
    return model.eval()
