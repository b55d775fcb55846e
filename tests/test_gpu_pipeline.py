"""execution_mode="overlap" (transforms and coder on two streams) gives the
same payload bytes and reconstructions as the sequential path, for the
FactorizedPrior and hyperprior stand-ins; sweep_p_ch measures every
candidate and selects by the policy."""

import numpy as np
import pytest
import torch

import fast_compressai
from fast_compressai import synthetic
from factorized_stub import FactorizedPrior
from hyperprior_stub import make_hyperprior

pytestmark = pytest.mark.gpu


def factorized(M=12, seed=7):
    torch.manual_seed(seed)
    w = synthetic.coder_512x768(seed=seed)
    med = np.random.default_rng(seed).normal(0, 0.2, M).astype(np.float32)
    return FactorizedPrior(M, w.cdfs[:M], w.cdf_sizes[:M], w.offsets[:M], med).eval()


def images(device, n=5):
    g = torch.Generator(device="cpu").manual_seed(3)
    sizes = [(1, 64, 64), (2, 64, 96), (1, 128, 64), (3, 64, 64), (1, 96, 96)][:n]
    return [torch.rand(b, 3, h, w, generator=g).to(device) for b, h, w in sizes]


def payload_bytes(out):
    return [s.packed.cpu().numpy().tobytes() for s in out["strings"]]


@pytest.mark.parametrize("kind", ["factorized", "scale", "mean_scale"])
def test_overlap_matches_sequential(gpu_device, kind):
    model = factorized() if kind == "factorized" else make_hyperprior(kind == "mean_scale")
    xs = images(gpu_device)
    seq = fast_compressai.accelerate(model, P=4, device=str(gpu_device))
    ovl = fast_compressai.accelerate(model, P=4, device=str(gpu_device),
                                     config={"execution_mode": "overlap"})
    assert ovl._pipeline.mode == "overlap"
    print("case: pipeline", kind, flush=True)
    a = seq.compress_many(xs)
    b = ovl.compress_many(xs)
    assert len(a) == len(b) == len(xs)
    for ra, rb in zip(a, b):
        assert ra["shape"] == rb["shape"] and payload_bytes(ra) == payload_bytes(rb)
    xa = seq.decompress_many(a)
    xb = ovl.decompress_many(b)
    for ra, rb in zip(xa, xb):
        assert torch.equal(ra["x_hat"], rb["x_hat"])
    # the overlapped decompress also reads payloads of the sequential path
    for ra, rc in zip(xa, ovl.decompress_many(a)):
        assert torch.equal(ra["x_hat"], rc["x_hat"])
    # and the single-call API gives the same as the sequence
    one = seq.decompress(a[1]["strings"], a[1]["shape"])
    assert torch.equal(one["x_hat"], xa[1]["x_hat"])


def test_sweep_p_ch_measures_and_selects(gpu_device):
    model = factorized()
    xs = images(gpu_device, 2)
    print("case: sweep_p_ch", flush=True)
    sel, recs = fast_compressai.sweep_p_ch(model, xs, candidates=(1, 4, 12, 99), warmup=1,
                                           repetitions=2, device=str(gpu_device))
    assert [r["p_ch"] for r in recs] == [1, 4, 12]
    assert sel.selected_p_ch in (1, 4, 12)
    assert sum(r["selected"] for r in recs) == 1
    for r in recs:
        for k in ("compress_inference_ms", "compress_codec_ms", "decompress_codec_ms",
                  "decompress_inference_ms", "inference_total_ms", "codec_total_ms"):
            assert r[k] > 0
        assert r["bpp"] > 0 and r["sample_count"] == 2
    again = fast_compressai.choose_p_ch(recs)
    assert again.selected_p_ch == sel.selected_p_ch
    # fewer chunk flushes: the payload never grows with P on the same images
    bpps = [r["bpp"] for r in recs]
    assert bpps[0] >= bpps[1] >= bpps[2]
