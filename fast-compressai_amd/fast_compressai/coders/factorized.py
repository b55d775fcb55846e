"""FactorizedPrior entropy path on the GA-ANS HIP coder.

Same contract as the reference's ``FactorizedWarpDivCodec``
(``src/fast_compressai/coders/factorized.py:11-107``): Balle's transforms and
quantizer semantics are kept, the entropy coder is replaced.  The difference
is that quantize and dequantize are fused into the coder kernels: the encode
kernel reads the fp32 latents and computes ``int32(rint(y - median))`` itself
(CompressAI ``EntropyModel.quantize(y, "symbols", medians)``), and the decode
kernel writes ``fp32(symbol) + median`` (``EntropyModel.dequantize``), so the
int32 symbol and index tensors of the reference path are never materialised.
"""

from __future__ import annotations

import torch

from . import gaans
from .errors import CoderInputError
from .tables import TableCache
from .warp_div import WarpDivBackend, WarpDivPayload, coding_fingerprint


class FactorizedWarpDivCodec:
    """Keep Balle's transforms/quantizer while replacing its entropy coder."""

    def __init__(self, model, p_ch: int, segments: int | None = None) -> None:
        self.model = model
        self.p_ch = p_ch
        self.segments = segments  # coding units per chunk; None: chosen per shape
        self.backend = WarpDivBackend()
        self._cache = TableCache(capacity=2)
        entropy = model.entropy_bottleneck
        if not 1 <= p_ch <= entropy.channels:
            raise CoderInputError(f"P must be between 1 and {entropy.channels} for this model")
        self._tables(entropy)

    @staticmethod
    def _tables(entropy):
        cdfs = getattr(entropy, "_quantized_cdf", None)
        lengths = getattr(entropy, "_cdf_length", None)
        offsets = getattr(entropy, "_offset", None)
        if (not isinstance(cdfs, torch.Tensor) or cdfs.ndim != 2 or cdfs.numel() == 0
                or lengths.numel() != cdfs.size(0) or offsets.numel() != cdfs.size(0)):
            raise CoderInputError(
                "entropy tables are not initialized; call model.update() before accelerate()")
        return (cdfs.to(torch.int32).contiguous(), lengths.to(torch.int32).contiguous(),
                offsets.to(torch.int32).contiguous())

    def _prepared(self, entropy, device):
        cdfs, lengths, offsets = self._tables(entropy)
        if cdfs.device != device:
            cdfs, lengths, offsets = cdfs.to(device), lengths.to(device), offsets.to(device)
        return self._cache.get(cdfs, lengths, offsets)

    @staticmethod
    def _medians(entropy) -> torch.Tensor:
        return entropy._get_medians().detach().reshape(-1)

    # ---- phases (the pipeline runs analysis / synthesis and coding on
    # different streams; compress / decompress chain them) --------------------
    def analyze(self, x: torch.Tensor) -> torch.Tensor:
        """Inference half of compress: ``y = g_a(x)``."""
        if not isinstance(x, torch.Tensor) or x.device.type != "cuda" or x.ndim != 4:
            raise CoderInputError("warp_div FactorizedPrior.compress expects a GPU NCHW tensor")
        with torch.no_grad():
            return self.model.g_a(x)

    def encode_latents(self, y: torch.Tensor):
        """Coding half of compress: quantize + GA-ANS encode of ``y``."""
        entropy = self.model.entropy_bottleneck
        if y.size(1) != entropy.channels:
            raise CoderInputError("latent channel count does not match entropy bottleneck")
        with torch.no_grad():
            tables = self._prepared(entropy, y.device)
            medians = self._medians(entropy)
            B, C = int(y.size(0)), int(y.size(1))
            N = int(y[0].numel())
            S = gaans.resolve_segments(self.segments, tables, B, N, C, self.p_ch, y.device)
            if y.dtype == torch.float32 and medians.dtype == torch.float32:
                enc = gaans.encode(tables, B, N, C, self.p_ch, y.device,
                                   y=y.contiguous(), medians=medians.contiguous(), segments=S)
            else:
                # non-fp32 latents: CompressAI's own quantize, then the coder
                ext = entropy._extend_ndims(entropy._get_medians().detach(), y.ndim - 2)
                symbols = entropy.quantize(y, "symbols", ext.expand(B, *([-1] * (y.ndim - 1))))
                enc = gaans.encode(tables, B, N, C, self.p_ch, y.device,
                                   symbols=symbols.reshape(B, -1).to(torch.int32).contiguous(),
                                   segments=S)
            payload = WarpDivPayload._from_encoder(
                packed=enc.packed, header_bytes=enc.header_bytes,
                chunk_len=enc.chunk_len, p_ch=self.p_ch, batch=B, symbols_per_batch=N,
                cdf_count=tables.M,
                coding_fingerprint=coding_fingerprint(tables.digest, B, N, C, tables.M),
                segments=S,
            )
            return {"strings": [payload], "shape": tuple(y.shape[-2:])}

    def decode_latents(self, strings, shape) -> torch.Tensor:
        """Coding half of decompress: GA-ANS decode + dequantize to ``y_hat``.
        CompressAI's own bitstreams (``strings = [[bytes per image]]`` from
        ``FactorizedPrior.compress`` with its RANS coder) decode on the GPU
        too, one lane per image stream."""
        if (isinstance(strings, (list, tuple)) and len(strings) == 1
                and is_compressai_strings(strings[0])):
            return self._decode_compressai(strings[0], shape)
        if (not isinstance(strings, (list, tuple)) or len(strings) != 1
                or not isinstance(strings[0], WarpDivPayload)):
            raise CoderInputError("warp_div decompress expects strings=[WarpDivPayload]")
        if (not isinstance(shape, (tuple, list, torch.Size)) or len(shape) != 2
                or any(type(dimension) is not int or dimension <= 0 for dimension in shape)):
            raise CoderInputError("warp_div decompress expects a positive (height, width) shape")
        payload = strings[0]
        if payload.p_ch != self.p_ch:
            raise CoderInputError("payload P_ch does not match the configured coder")
        entropy = self.model.entropy_bottleneck
        channels = entropy.channels
        if payload.symbols_per_batch != channels * shape[0] * shape[1]:
            raise CoderInputError("payload symbol count does not match the latent shape")
        if payload.coded_channels != channels:
            raise CoderInputError("payload channel count does not match the entropy bottleneck")
        cdfs, _, _ = self._tables(entropy)
        if payload.packed.device != cdfs.device:
            raise CoderInputError("payload and entropy model must be on the same GPU device")
        tables = self._prepared(entropy, cdfs.device)
        B, N = payload.batch, payload.symbols_per_batch
        if payload.cdf_count != tables.M or (
                payload.coding_fingerprint is not None and payload.coding_fingerprint
                != coding_fingerprint(tables.digest, B, N, channels, tables.M)):
            raise CoderInputError("coding tables or indexes do not match warp_div payload")
        with torch.no_grad():
            output_shape = (B, channels, *shape)
            medians = self._medians(entropy)
            S = payload.segments
            if medians.dtype == torch.float32:
                return gaans.decode(payload.packed, tables, B, N, channels, self.p_ch,
                                    payload.packed.device, medians=medians.contiguous(),
                                    segments=S).reshape(output_shape)
            symbols = gaans.decode(payload.packed, tables, B, N, channels, self.p_ch,
                                   payload.packed.device, segments=S).reshape(output_shape)
            ext = entropy._extend_ndims(entropy._get_medians().detach(), len(shape))
            ext = ext.expand(B, *([-1] * (len(shape) + 1)))
            return entropy.dequantize(symbols, ext, ext.dtype)

    def _decode_compressai(self, streams, shape) -> torch.Tensor:
        """EntropyBottleneck.decompress of CompressAI bitstreams: table =
        channel, ``y_hat = float(symbol) + median``; small batches go to
        CompressAI's host decoder when it is importable (see
        ``gaans.decode_compressai_strings``)."""
        if (not isinstance(shape, (tuple, list, torch.Size)) or len(shape) != 2
                or any(type(d) is not int or d <= 0 for d in shape)):
            raise CoderInputError("decompress expects a positive (height, width) shape")
        entropy = self.model.entropy_bottleneck
        C = entropy.channels
        raw = self._tables(entropy)
        device = raw[0].device
        tables = self._prepared(entropy, device)
        B, N = len(streams), C * shape[0] * shape[1]
        with torch.no_grad():
            symbols = gaans.decode_compressai_strings(streams, tables, raw, B, N, C, device)
            medians = entropy._extend_ndims(entropy._get_medians().detach(), 2)
            return symbols.reshape(B, C, *shape).type_as(medians) + medians

    def synthesize(self, y_hat: torch.Tensor):
        """Inference half of decompress: ``x_hat = g_s(y_hat).clamp(0, 1)``."""
        with torch.no_grad():
            return {"x_hat": self.model.g_s(y_hat).clamp_(0, 1)}

    # ---- the model's public paths -------------------------------------------
    def compress(self, x: torch.Tensor, timing: dict[str, float] | None = None):
        if timing is None:
            return self.encode_latents(self.analyze(x))
        with _Span(timing, "compress_inference_ms"):
            y = self.analyze(x)
        with _Span(timing, "compress_codec_ms"):
            return self.encode_latents(y)

    def decompress(self, strings, shape, timing: dict[str, float] | None = None):
        if timing is None:
            return self.synthesize(self.decode_latents(strings, shape))
        with _Span(timing, "decompress_codec_ms"):
            y_hat = self.decode_latents(strings, shape)
        with _Span(timing, "decompress_inference_ms"):
            return self.synthesize(y_hat)


def is_compressai_strings(value) -> bool:
    """A CompressAI ``compress`` string list: one ``bytes`` per image."""
    return (isinstance(value, (list, tuple)) and len(value) > 0
            and all(isinstance(s, (bytes, bytearray)) for s in value))


class _Span:
    """Event-timed region on the current stream; stores milliseconds in
    ``timing[key]`` (keys of the reference's ``timing`` dict,
    ``src/fast_compressai/coders/factorized.py:33-107``)."""

    def __init__(self, timing: dict[str, float], key: str) -> None:
        self.timing, self.key = timing, key

    def __enter__(self):
        self.start = torch.cuda.Event(enable_timing=True)
        self.end = torch.cuda.Event(enable_timing=True)
        self.start.record()
        return self

    def __exit__(self, *exc):
        self.end.record()
        self.end.synchronize()
        self.timing[self.key] = float(self.start.elapsed_time(self.end))
        return False
