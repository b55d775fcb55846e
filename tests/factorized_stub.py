"""A FactorizedPrior stand-in that implements the parts of CompressAI's
FactorizedPrior / EntropyBottleneck contract the GA-ANS codec uses (CompressAI
is not installed here).  Follows CompressAI's published semantics:
``_get_medians() = quantiles[:, :, 1:2]``; ``quantize(y, "symbols", means) =
round(y - means).int()``; ``dequantize(s, means) = s.type_as(means) + means``;
``_build_indexes`` = channel index broadcast over NCHW; tables in
``_quantized_cdf`` / ``_cdf_length`` / ``_offset``."""

import numpy as np
import torch
from torch import nn


class EntropyBottleneck(nn.Module):
    def __init__(self, channels: int, cdfs, sizes, offsets, medians) -> None:
        super().__init__()
        self.channels = channels
        med = torch.as_tensor(medians, dtype=torch.float32).reshape(channels, 1, 1)
        self.quantiles = nn.Parameter(torch.cat([med - 10, med, med + 10], dim=-1))
        self.register_buffer("_quantized_cdf", torch.as_tensor(np.asarray(cdfs, np.int32)))
        self.register_buffer("_cdf_length", torch.as_tensor(np.asarray(sizes, np.int32)))
        self.register_buffer("_offset", torch.as_tensor(np.asarray(offsets, np.int32)))

    def _get_medians(self) -> torch.Tensor:
        return self.quantiles[:, :, 1:2]

    @staticmethod
    def _extend_ndims(tensor, n):
        return tensor.reshape(-1, *([1] * n)) if n > 0 else tensor.reshape(-1)

    def _build_indexes(self, size, device=None):
        dims = len(size)
        N, C = size[0], size[1]
        view_dims = np.ones((dims,), dtype=np.int64)
        view_dims[1] = -1
        indexes = torch.arange(C, device=device).view(*view_dims)
        indexes = indexes.int()
        return indexes.repeat(N, 1, *size[2:])

    def quantize(self, inputs, mode, means=None):
        outputs = inputs.clone()
        if means is not None:
            outputs -= means
        outputs = torch.round(outputs)
        if mode == "dequantize":
            if means is not None:
                outputs += means
            return outputs
        assert mode == "symbols", mode
        return outputs.int()

    @staticmethod
    def dequantize(inputs, means=None, dtype=torch.float):
        if means is not None:
            outputs = inputs.type_as(means)
            outputs += means
        else:
            outputs = inputs.type(dtype)
        return outputs


class FactorizedPrior(nn.Module):
    def __init__(self, M: int, cdfs, sizes, offsets, medians, scale: float = 8.0) -> None:
        super().__init__()
        self.g_a = nn.Sequential(nn.Conv2d(3, M, 4, stride=4), nn.Conv2d(M, M, 1))
        self.g_s = nn.Sequential(nn.ConvTranspose2d(M, 3, 4, stride=4))
        with torch.no_grad():
            self.g_a[1].weight.mul_(scale)
        self.entropy_bottleneck = EntropyBottleneck(M, cdfs, sizes, offsets, medians)

    def compress(self, x):
        raise NotImplementedError("the stand-in has no CPU RANS path")
