"""Sequential and overlapped compress / decompress over a sequence of inputs.

The reference declares ``AccelerationConfig.execution_mode`` ("sequential" or
"overlap", ``src/fast_compressai/config.py:29``, ``:46-47``) but runs every
call sequentially.  Here "overlap" runs the transforms (``g_a`` / ``g_s``,
plus ``h_a`` for hyperpriors) on the caller's current stream and the entropy
coding phase on a second stream of the same device (default priority),
ordered by events:

* compress: the host launches ``analyze(x[i + 1])`` before it codes item
  ``i``, so the GPU runs the next item's analysis transform while the coder
  kernels of item ``i`` run, and the host's one wait per encode falls inside
  that window;
* decompress: item ``i``'s synthesis transform is launched right after its
  decode, and runs while the host waits for the decode of item ``i + 1``.

Results are the same objects, bit for bit, as the sequential path's: only
the streams differ.  Tensors handed from one stream to the other are
registered with ``record_stream``, and the caller's stream waits for the
coder stream before returning, so outputs are ready for work the caller
enqueues next.
"""

from __future__ import annotations

from typing import Any, Iterable

import torch

from .config import ConfigurationError

MODES = ("sequential", "overlap")


def _tensors(value) -> list[torch.Tensor]:
    if isinstance(value, torch.Tensor):
        return [value]
    if isinstance(value, (tuple, list)):
        return [t for v in value for t in _tensors(v)]
    return []


class CodingPipeline:
    """Runs a GA-ANS codec's phases (``analyze``, ``encode_latents``,
    ``decode_latents``, ``synthesize``) over sequences of inputs."""

    def __init__(self, codec: Any, device: torch.device | str, mode: str = "sequential") -> None:
        if mode not in MODES:
            raise ConfigurationError("execution_mode must be 'sequential' or 'overlap'")
        self.codec = codec
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ConfigurationError("the coding pipeline requires a GPU device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.mode = mode
        self._stream: torch.cuda.Stream | None = None

    def coder_stream(self) -> torch.cuda.Stream:
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=self.device)  # default priority
        return self._stream

    # ---- compress ---------------------------------------------------------------
    def compress_many(self, inputs: Iterable[torch.Tensor]) -> list[dict]:
        if self.mode == "sequential":
            return [self.codec.compress(x) for x in inputs]
        with torch.cuda.device(self.device):
            main = torch.cuda.current_stream(self.device)
            coder = self.coder_stream()
            out: list[dict] = []
            pending = None
            try:
                for x in inputs:
                    latents = self.codec.analyze(x)      # caller's stream
                    ready = torch.cuda.Event()
                    ready.record(main)
                    if pending is not None:
                        out.append(self._encode(coder, main, *pending))
                    pending = (latents, ready)
                if pending is not None:
                    out.append(self._encode(coder, main, *pending))
            finally:
                main.wait_stream(coder)
            return out

    def _encode(self, coder, main, latents, ready) -> dict:
        coder.wait_event(ready)
        with torch.cuda.stream(coder):
            result = self.codec.encode_latents(latents)
        for t in _tensors(latents):
            t.record_stream(coder)
        for payload in result["strings"]:
            payload.packed.record_stream(main)
        return result

    # ---- decompress -------------------------------------------------------------
    def decompress_many(self, items: Iterable[dict]) -> list[dict]:
        if self.mode == "sequential":
            return [self.codec.decompress(it["strings"], it["shape"]) for it in items]
        with torch.cuda.device(self.device):
            main = torch.cuda.current_stream(self.device)
            coder = self.coder_stream()
            coder.wait_stream(main)  # payloads written on the caller's stream
            out: list[dict] = []
            for it in items:
                with torch.cuda.stream(coder):
                    y_hat = self.codec.decode_latents(it["strings"], it["shape"])
                    decoded = torch.cuda.Event()
                    decoded.record(coder)
                for payload in it["strings"]:
                    payload.packed.record_stream(coder)
                main.wait_event(decoded)
                y_hat.record_stream(main)
                out.append(self.codec.synthesize(y_hat))  # caller's stream
            return out
