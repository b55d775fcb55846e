"""GaussianConditional path (scale and mean-scale hyperpriors) on the GPU.

* The fused kernels (``gaans_encode_gaussian`` / ``gaans_decode_gaussian``:
  build_indexes + quantize / dequantize inside the coder) against the oracle:
  indexes from ``oracle.build_indexes`` (CompressAI's loop, restated),
  symbols from ``oracle.quantize_elem``, payload bytes from
  ``oracle.gaans_encode`` with those indexes, y_hat from
  ``oracle.dequantize_elem`` -- bit for bit.
* ``accelerate()`` on ScaleHyperprior / MeanScaleHyperprior stand-ins
  (tests/hyperprior_stub.py): decoded latents and x_hat equal CompressAI's
  quantize -> dequantize semantics computed with torch.
"""

import math

import numpy as np
import pytest
import torch

import fast_compressai
import oracle as O
from fast_compressai.coders import CoderInputError, WarpDivPayload, gaans
from fast_compressai.coders.tables import prepare_tables
from hyperprior_stub import gaussian_tables, make_hyperprior, reference_y_hat

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def gaussian_case(B, C, H, W, seed, with_means=True, edge=False):
    rng = np.random.default_rng(seed)
    table, cdfs, sizes, offsets = gaussian_tables()
    n = C * H * W
    scales = np.exp(rng.uniform(math.log(0.05), math.log(300.0), (B, n))).astype(np.float32)
    if edge:  # table values, the bound, non-finite scales
        scales[0, :64] = table
        scales[0, 64:70] = [np.nan, np.inf, -np.inf, 0.0, 0.11, -3.0]
    means = rng.normal(0, 1, (B, n)).astype(np.float32) if with_means else None
    noise = rng.standard_normal((B, n)) * np.nan_to_num(np.clip(scales, 0.11, 256), nan=256)
    y = ((means if means is not None else 0.0) + noise).astype(np.float32)
    return table, cdfs, sizes, offsets, y, means, scales


# the mean-scale hyperprior's y at full size for every P of the sweep; a
# 1x192x33x48 latent at P=24 (38,016-symbol chunks: 594 steps, so with one
# segment the encoder's 16-step blocks end with a partial block); small
# ragged shapes (1x24x5x7 at P=5: 3-step chunks, the most segments)
@pytest.mark.parametrize("with_means", [True, False])
@pytest.mark.parametrize("shape,p_ch,segments", [
    ((1, 192, 32, 48), 1, 1), ((1, 192, 32, 48), 4, 1), ((1, 192, 32, 48), 16, 2),
    ((1, 192, 32, 48), 64, 4), ((1, 192, 32, 48), 192, 8), ((1, 192, 33, 48), 24, 1),
    ((1, 192, 33, 48), 24, 4), ((2, 16, 8, 12), 1, 1), ((2, 16, 8, 12), 16, 2),
    ((1, 24, 5, 7), 5, 3)])
def test_fused_gaussian_matches_oracle(gpu_device, shape, p_ch, segments, with_means):
    B, C, H, W = shape
    say("case: gaussian", shape, "P", p_ch, "segments", segments, "means", with_means)
    table, cdfs, sizes, offsets, y, means, scales = gaussian_case(
        B, C, H, W, seed=C + p_ch, with_means=with_means, edge=True)
    N = C * H * W
    idx = O.build_indexes(scales, table, 0.11)
    sym = O.quantize_elem(y, means)
    ref = O.gaans_encode(sym, idx, cdfs, sizes, offsets, p_ch, C, segments)
    tables = prepare_tables(dev(cdfs, gpu_device), dev(sizes, gpu_device), dev(offsets, gpu_device))
    dm = dev(means, gpu_device) if means is not None else None
    enc = gaans.encode_gaussian(tables, B, N, C, p_ch, gpu_device, y=dev(y, gpu_device),
                                scales=dev(scales, gpu_device),
                                scale_table=dev(table, gpu_device), scale_bound=0.11, means=dm,
                                segments=segments)
    got = enc.packed.cpu().numpy().tobytes()
    assert len(got) == len(ref) and got == ref
    y_hat = gaans.decode_gaussian(enc.packed, tables, B, N, C, p_ch, gpu_device,
                                  scales=dev(scales, gpu_device),
                                  scale_table=dev(table, gpu_device), scale_bound=0.11, means=dm,
                                  segments=segments)
    want = O.dequantize_elem(sym, means)
    assert np.array_equal(y_hat.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_fused_gaussian_detects_other_scales(gpu_device):
    B, C, H, W = 1, 16, 8, 12
    table, cdfs, sizes, offsets, y, means, scales = gaussian_case(B, C, H, W, seed=3)
    N = C * H * W
    tables = prepare_tables(dev(cdfs, gpu_device), dev(sizes, gpu_device), dev(offsets, gpu_device))
    args = dict(scale_table=dev(table, gpu_device), scale_bound=0.11,
                means=dev(means, gpu_device))
    enc = gaans.encode_gaussian(tables, B, N, C, 4, gpu_device, y=dev(y, gpu_device),
                                scales=dev(scales, gpu_device), **args)
    other = scales.copy()
    other[0, 17] = 200.0 if scales[0, 17] < 10.0 else 0.2  # another table for one element
    say("case: gaussian decode with other scales")
    with pytest.raises(CoderInputError):
        gaans.decode_gaussian(enc.packed, tables, B, N, C, 4, gpu_device,
                              scales=dev(other, gpu_device), **args)


@pytest.mark.parametrize("mean_scale", [True, False])
def test_accelerate_hyperprior_matches_quantize_dequantize(gpu_device, mean_scale):
    model = make_hyperprior(mean_scale=mean_scale).to(gpu_device)
    x = torch.rand(2, 3, 64, 64, device=gpu_device)
    y, z, z_hat, scales, means, symbols, indexes, y_hat = reference_y_hat(model, x)
    with torch.no_grad():
        x_ref = model.g_s(y_hat).clamp_(0, 1)
    for p_ch in (1, 4, 16):
        say("case: accelerate hyperprior mean_scale", mean_scale, "P", p_ch)
        fast = fast_compressai.accelerate(model, P=p_ch, device=str(gpu_device))
        assert fast.acceleration_report.coder_status == "warp_div"
        out = fast.compress(x)
        y_payload, z_payload = out["strings"]
        assert isinstance(y_payload, WarpDivPayload) and y_payload.p_ch == p_ch
        assert out["shape"] == tuple(z.shape[-2:])
        # y payload: the symbols and indexes of CompressAI's GaussianConditional
        gc = fast.model.gaussian_conditional
        B, N = y.size(0), y[0].numel()
        dec = fast._coder.backend.decode(
            y_payload, indexes.reshape(B, N).contiguous(), gc._quantized_cdf.contiguous(),
            gc._cdf_length.contiguous(), gc._offset.contiguous())
        assert torch.equal(dec.reshape_as(symbols), symbols)
        res = fast.decompress(out["strings"], out["shape"])
        assert torch.equal(res["x_hat"], x_ref)


def test_hyperprior_unsorted_scale_table_falls_back(gpu_device):
    model = make_hyperprior(mean_scale=True).to(gpu_device)
    gc = model.gaussian_conditional
    # swap two table entries (and their CDFs), so the table is no longer sorted
    perm = torch.arange(64, device=gpu_device)
    perm[[10, 11]] = perm[[11, 10]]
    with torch.no_grad():
        gc.scale_table.copy_(gc.scale_table[perm])
        gc._quantized_cdf.copy_(gc._quantized_cdf[perm])
        gc._cdf_length.copy_(gc._cdf_length[perm])
        gc._offset.copy_(gc._offset[perm])
    x = torch.rand(1, 3, 64, 64, device=gpu_device)
    *_, y_hat = reference_y_hat(model, x)
    with torch.no_grad():
        x_ref = model.g_s(y_hat).clamp_(0, 1)
    fast = fast_compressai.accelerate(model, P=4, device=str(gpu_device))
    assert not fast._coder.fused_indexes
    say("case: unsorted scale table")
    out = fast.compress(x)
    assert torch.equal(fast.decompress(out["strings"], out["shape"])["x_hat"], x_ref)


def test_hyperprior_payload_mismatch_rejected(gpu_device):
    model = make_hyperprior(mean_scale=True).to(gpu_device)
    x = torch.rand(1, 3, 64, 64, device=gpu_device)
    fast = fast_compressai.accelerate(model, P=4, device=str(gpu_device))
    out = fast.compress(x)
    y_payload, z_payload = out["strings"]
    say("case: swapped hyperprior payloads")
    with pytest.raises(CoderInputError):
        fast.decompress([z_payload, y_payload], out["shape"])
    with pytest.raises(CoderInputError):
        fast.decompress([y_payload], out["shape"])
