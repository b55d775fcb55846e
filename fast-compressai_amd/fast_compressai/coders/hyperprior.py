"""Scale and mean-scale hyperprior entropy paths on the GA-ANS HIP coder.

CompressAI's ``ScaleHyperprior`` / ``MeanScaleHyperprior`` code two latents:
``z = h_a(|y|)`` (or ``h_a(y)``) through an EntropyBottleneck, and ``y``
through a GaussianConditional whose per-element table index comes from the
scales predicted by ``h_s(z_hat)`` (``build_indexes``), with the predicted
means subtracted before rounding in the mean-scale model.  This codec keeps
the transforms and replaces both entropy coders:

* z: the factorized path (channel-major tables, per-channel medians, quantize
  and dequantize fused into the kernels), as ``FactorizedWarpDivCodec``;
* y: ``gaans_encode_gaussian`` / ``gaans_decode_gaussian``, whose mapper waves
  compute ``build_indexes`` (a binary search over the scale table in LDS),
  ``int32(rint(y - mean))`` and ``fp32(symbol) + mean`` per element, so
  neither the int32 indexes nor the symbols are materialised (CompressAI's
  ``build_indexes`` runs one compare-and-subtract kernel pair per scale).

The reference's ``accelerate()`` accepts only ``FactorizedPrior``
(``src/fast_compressai/api.py:177-182``); this is the "mean-scale hyperprior
routing" next step of its coder path.  The payloads keep the reference's
``{"strings": [...], "shape": z.shape[-2:]}`` layout of CompressAI's
hyperprior ``compress``: ``strings = [y payload, z payload]``.
"""

from __future__ import annotations

import torch

from . import gaans
from .errors import CoderInputError
from .factorized import _Span, is_compressai_strings
from .tables import TableCache
from .warp_div import WarpDivBackend, WarpDivPayload, coding_fingerprint


def _tables(module, what: str):
    cdfs = getattr(module, "_quantized_cdf", None)
    lengths = getattr(module, "_cdf_length", None)
    offsets = getattr(module, "_offset", None)
    if (not isinstance(cdfs, torch.Tensor) or cdfs.ndim != 2 or cdfs.numel() == 0
            or lengths.numel() != cdfs.size(0) or offsets.numel() != cdfs.size(0)):
        raise CoderInputError(
            f"{what} tables are not initialized; call model.update() before accelerate()")
    return (cdfs.to(torch.int32).contiguous(), lengths.to(torch.int32).contiguous(),
            offsets.to(torch.int32).contiguous())


def _payload(enc, p_ch: int, B: int, N: int, C: int, tables) -> WarpDivPayload:
    return WarpDivPayload._from_encoder(
        packed=enc.packed, header_bytes=enc.header_bytes,
        chunk_len=enc.chunk_len, p_ch=p_ch, batch=B, symbols_per_batch=N, cdf_count=tables.M,
        coding_fingerprint=coding_fingerprint(tables.digest, B, N, C, tables.M),
        channels=None if C == tables.M else C, segments=enc.segments)


class HyperpriorWarpDivCodec:
    """Keep the hyperprior's transforms; code z and y with the GA-ANS kernels.

    ``mean_scale``: True for ``MeanScaleHyperprior`` (``h_s`` predicts scales
    and means, ``z = h_a(y)``), False for ``ScaleHyperprior`` (scales only,
    ``z = h_a(|y|)``)."""

    def __init__(self, model, p_ch: int, mean_scale: bool,
                 segments: int | None = None) -> None:
        self.model = model
        self.p_ch = p_ch
        self.mean_scale = mean_scale
        self.segments = segments  # coding units per chunk; None: chosen per shape
        self.backend = WarpDivBackend()
        self._cache = TableCache(capacity=4)
        eb, gc = model.entropy_bottleneck, model.gaussian_conditional
        _tables(eb, "entropy bottleneck")
        cdfs, _, _ = _tables(gc, "gaussian conditional")
        table = getattr(gc, "scale_table", None)
        if not isinstance(table, torch.Tensor) or table.ndim != 1 or table.numel() < 1:
            raise CoderInputError("gaussian conditional has no scale table; call model.update()")
        if table.numel() != cdfs.size(0):
            raise CoderInputError("scale table and gaussian conditional tables differ in length")
        if p_ch < 1:
            raise CoderInputError("P must be a positive integer")
        bound = getattr(getattr(gc, "lower_bound_scale", None), "bound", None)
        self.scale_bound = float(bound.reshape(-1)[0]) if isinstance(bound, torch.Tensor) else \
            float(getattr(gc, "scale_bound", 0.11))
        t = table.detach().to(torch.float32)
        # the fused index search needs a finite, non-decreasing table (CompressAI's
        # log-spaced default is); otherwise indexes are built with torch
        self.fused_indexes = bool(torch.isfinite(t).all()) and bool((t[1:] >= t[:-1]).all())

    # ---- tables -------------------------------------------------------------
    def _prepared(self, module, what: str, device):
        cdfs, lengths, offsets = _tables(module, what)
        if cdfs.device != device:
            cdfs, lengths, offsets = cdfs.to(device), lengths.to(device), offsets.to(device)
        return self._cache.get(cdfs, lengths, offsets)

    def _scale_table(self, device) -> torch.Tensor:
        t = self.model.gaussian_conditional.scale_table.detach()
        return t.to(device=device, dtype=torch.float32).contiguous()

    def _build_indexes(self, scales: torch.Tensor) -> torch.Tensor:
        """CompressAI's GaussianConditional.build_indexes (used only when the
        scale table is not sorted)."""
        gc = self.model.gaussian_conditional
        bound = torch.tensor(self.scale_bound, device=scales.device, dtype=scales.dtype)
        lb = torch.max(scales, bound)
        table = gc.scale_table.to(scales.device)
        indexes = torch.full(scales.shape, table.numel() - 1, dtype=torch.int32,
                             device=scales.device)
        for s in table[:-1]:
            indexes -= (lb <= s).int()
        return indexes

    # ---- z (EntropyBottleneck) ------------------------------------------------
    def _z_encode(self, z: torch.Tensor):
        eb = self.model.entropy_bottleneck
        if z.size(1) != eb.channels:
            raise CoderInputError("hyper-latent channel count does not match the entropy bottleneck")
        tables = self._prepared(eb, "entropy bottleneck", z.device)
        med = eb._get_medians().detach().reshape(-1).to(torch.float32).contiguous()
        B, C, N = int(z.size(0)), int(z.size(1)), int(z[0].numel())
        P = min(self.p_ch, C)
        S = gaans.resolve_segments(self.segments, tables, B, N, C, P, z.device)
        enc = gaans.encode(tables, B, N, C, P, z.device, y=z.to(torch.float32).contiguous(),
                           medians=med, segments=S)
        # z_hat = dequantize(quantize(z)), as CompressAI's compress recomputes it
        m4 = med.reshape(1, C, 1, 1)
        z_hat = torch.round(z.to(torch.float32) - m4).int().to(torch.float32) + m4
        return _payload(enc, P, B, N, C, tables), z_hat

    def _z_decode(self, payload: WarpDivPayload, shape) -> torch.Tensor:
        eb = self.model.entropy_bottleneck
        C = eb.channels
        if payload.coded_channels != C or payload.symbols_per_batch != C * shape[0] * shape[1]:
            raise CoderInputError("z payload does not match the entropy bottleneck and shape")
        tables = self._prepared(eb, "entropy bottleneck", payload.packed.device)
        B, N = payload.batch, payload.symbols_per_batch
        if payload.cdf_count != tables.M or (
                payload.coding_fingerprint is not None and payload.coding_fingerprint
                != coding_fingerprint(tables.digest, B, N, C, tables.M)):
            raise CoderInputError("coding tables do not match the z payload")
        med = eb._get_medians().detach().reshape(-1).to(torch.float32).contiguous()
        z_hat = gaans.decode(payload.packed, tables, B, N, C, payload.p_ch, payload.packed.device,
                             medians=med, segments=payload.segments)
        return z_hat.reshape(B, C, *shape)

    def _params(self, z_hat: torch.Tensor):
        out = self.model.h_s(z_hat)
        if self.mean_scale:
            scales, means = out.chunk(2, 1)
            return scales.to(torch.float32).contiguous(), means.to(torch.float32).contiguous()
        return out.to(torch.float32).contiguous(), None

    # ---- phases (the pipeline runs analysis / synthesis and coding on
    # different streams; compress / decompress chain them) --------------------
    def analyze(self, x: torch.Tensor):
        """Inference half of compress: ``y = g_a(x)``, ``z = h_a(y)`` (mean-scale)
        or ``h_a(|y|)`` (scale)."""
        if not isinstance(x, torch.Tensor) or x.device.type != "cuda" or x.ndim != 4:
            raise CoderInputError("warp_div hyperprior compress expects a GPU NCHW tensor")
        with torch.no_grad():
            y = self.model.g_a(x)
            z = self.model.h_a(y if self.mean_scale else torch.abs(y))
        return y, z

    def encode_latents(self, latents):
        """Coding half of compress: z through the factorized kernels, ``h_s``,
        y through the Gaussian kernels."""
        y, z = latents
        with torch.no_grad():
            z_payload, z_hat = self._z_encode(z)
            scales, means = self._params(z_hat)
            gc = self.model.gaussian_conditional
            tables = self._prepared(gc, "gaussian conditional", y.device)
            B, C, N = int(y.size(0)), int(y.size(1)), int(y[0].numel())
            if scales.shape != y.shape or (means is not None and means.shape != y.shape):
                raise CoderInputError("h_s output does not match the latent shape")
            if not 1 <= self.p_ch <= C:
                raise CoderInputError(f"P must be between 1 and {C} for this model")
            yf = y.to(torch.float32).contiguous()
            S = gaans.resolve_segments(self.segments, tables, B, N, C, self.p_ch, y.device)
            if self.fused_indexes:
                enc = gaans.encode_gaussian(tables, B, N, C, self.p_ch, y.device, y=yf,
                                            scales=scales, scale_table=self._scale_table(y.device),
                                            scale_bound=self.scale_bound, means=means,
                                            segments=S)
            else:
                idx = self._build_indexes(scales).reshape(B, N).contiguous()
                sym = torch.round(yf - means if means is not None else yf).int()
                enc = gaans.encode(tables, B, N, C, self.p_ch, y.device,
                                   symbols=sym.reshape(B, N).contiguous(), indexes=idx,
                                   segments=S)
            y_payload = _payload(enc, self.p_ch, B, N, C, tables)
            return {"strings": [y_payload, z_payload], "shape": tuple(z.shape[-2:])}

    def decode_latents(self, strings, shape) -> torch.Tensor:
        """Coding half of decompress: z decode, ``h_s``, y decode to ``y_hat``.
        CompressAI's own bitstreams (``strings = [y bytes per image, z bytes
        per image]``) decode on the GPU too, one lane per image stream."""
        if (isinstance(strings, (list, tuple)) and len(strings) == 2
                and all(is_compressai_strings(s) for s in strings)):
            return self._decode_compressai(strings, shape)
        if (not isinstance(strings, (list, tuple)) or len(strings) != 2
                or not all(isinstance(s, WarpDivPayload) for s in strings)):
            raise CoderInputError("warp_div hyperprior decompress expects strings=[y, z] payloads")
        if (not isinstance(shape, (tuple, list, torch.Size)) or len(shape) != 2
                or any(type(d) is not int or d <= 0 for d in shape)):
            raise CoderInputError("warp_div decompress expects a positive (height, width) shape")
        y_payload, z_payload = strings
        with torch.no_grad():
            z_hat = self._z_decode(z_payload, shape)
            scales, means = self._params(z_hat)
            gc = self.model.gaussian_conditional
            tables = self._prepared(gc, "gaussian conditional", y_payload.packed.device)
            B, C = int(scales.size(0)), int(scales.size(1))
            N = int(scales[0].numel())
            if (y_payload.batch != B or y_payload.symbols_per_batch != N
                    or y_payload.coded_channels != C or y_payload.p_ch != self.p_ch):
                raise CoderInputError("y payload does not match the predicted latent shape")
            if y_payload.cdf_count != tables.M or (
                    y_payload.coding_fingerprint is not None and y_payload.coding_fingerprint
                    != coding_fingerprint(tables.digest, B, N, C, tables.M)):
                raise CoderInputError("coding tables do not match the y payload")
            if self.fused_indexes:
                y_hat = gaans.decode_gaussian(y_payload.packed, tables, B, N, C, self.p_ch,
                                              y_payload.packed.device, scales=scales,
                                              scale_table=self._scale_table(scales.device),
                                              scale_bound=self.scale_bound, means=means,
                                              segments=y_payload.segments)
            else:
                idx = self._build_indexes(scales).reshape(B, N).contiguous()
                sym = gaans.decode(y_payload.packed, tables, B, N, C, self.p_ch,
                                   y_payload.packed.device, indexes=idx,
                                   segments=y_payload.segments)
                y_hat = sym.to(torch.float32)
                if means is not None:
                    y_hat = y_hat + means.reshape(B, N)
            return y_hat.reshape(scales.shape)

    def _decode_compressai(self, strings, shape) -> torch.Tensor:
        """CompressAI's hyperprior decompress of its own bitstreams: z by the
        EntropyBottleneck (table = channel, + medians), scales (and means)
        from ``h_s``, y by the GaussianConditional with ``build_indexes``
        (computed with torch), ``y_hat = float(symbol) (+ means)``."""
        if (not isinstance(shape, (tuple, list, torch.Size)) or len(shape) != 2
                or any(type(d) is not int or d <= 0 for d in shape)):
            raise CoderInputError("decompress expects a positive (height, width) shape")
        y_strings, z_strings = strings
        if len(y_strings) != len(z_strings):
            raise CoderInputError("y and z string lists differ in length")
        eb, gc = self.model.entropy_bottleneck, self.model.gaussian_conditional
        device = eb._quantized_cdf.device
        B, Cz = len(z_strings), eb.channels
        with torch.no_grad():
            ztab = self._prepared(eb, "entropy bottleneck", device)
            zs = gaans.decode_compressai_strings(z_strings, ztab, _tables(eb, "entropy bottleneck"),
                                                 B, Cz * shape[0] * shape[1], Cz, device)
            med = eb._extend_ndims(eb._get_medians().detach(), 2)
            z_hat = zs.reshape(B, Cz, *shape).type_as(med) + med
            scales, means = self._params(z_hat)
            C, N = int(scales.size(1)), int(scales[0].numel())
            ytab = self._prepared(gc, "gaussian conditional", device)
            idx = self._build_indexes(scales).reshape(B, N).contiguous()
            ys = gaans.decode_compressai_strings(y_strings, ytab,
                                                 _tables(gc, "gaussian conditional"), B, N, C,
                                                 device, indexes=idx)
            y_hat = ys.reshape(scales.shape).to(torch.float32)
            return y_hat + means if means is not None else y_hat

    def synthesize(self, y_hat: torch.Tensor):
        """Inference half of decompress: ``x_hat = g_s(y_hat).clamp(0, 1)``."""
        with torch.no_grad():
            return {"x_hat": self.model.g_s(y_hat).clamp_(0, 1)}

    # ---- the model's public paths -------------------------------------------
    def compress(self, x: torch.Tensor, timing: dict[str, float] | None = None):
        if timing is None:
            return self.encode_latents(self.analyze(x))
        with _Span(timing, "compress_inference_ms"):
            latents = self.analyze(x)
        with _Span(timing, "compress_codec_ms"):
            return self.encode_latents(latents)

    def decompress(self, strings, shape, timing: dict[str, float] | None = None):
        if timing is None:
            return self.synthesize(self.decode_latents(strings, shape))
        with _Span(timing, "decompress_codec_ms"):
            y_hat = self.decode_latents(strings, shape)
        with _Span(timing, "decompress_inference_ms"):
            return self.synthesize(y_hat)
