"""The HIP kernels reproduce the committed golden fixtures (tests/golden)
byte for byte: GA-ANS payloads from int32 symbols (explicit and implicit
indexes), from fp32 latents (quantize fused) and from the Gaussian path
(build_indexes + quantize fused); decodes return the fixtures' symbols or
their dequantized values; the Rans64 streams decode to the same symbols."""

import numpy as np
import pytest
import torch

import oracle as O
from fast_compressai.coders import gaans
from fast_compressai.coders.tables import prepare_tables
from golden_cases import NAMES, load

pytestmark = pytest.mark.gpu


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


@pytest.mark.parametrize("name", NAMES)
def test_kernels_reproduce_golden_bytes(gpu_device, name):
    c = load(name)
    print("case: golden", name, flush=True)
    sym = c["symbols"]
    B, N = sym.shape
    C, P, S = c["channels"], c["p_ch"], c["segments"]
    tables = prepare_tables(dev(c["cdfs"], gpu_device), dev(c["cdf_sizes"], gpu_device),
                            dev(c["offsets"], gpu_device))
    idx = dev(c["full_indexes"], gpu_device) if c["explicit"] else None
    if name == "latents":
        med = dev(c["medians"], gpu_device)
        enc = gaans.encode(tables, B, N, C, P, gpu_device, y=dev(c["y"], gpu_device), medians=med,
                           segments=S)
        out = gaans.decode(enc.packed, tables, B, N, C, P, gpu_device, medians=med, segments=S)
        want = O.dequantize(sym.reshape(B, C, -1), c["medians"]).reshape(B, N)
    elif name == "gaussian":
        g = dict(scales=dev(c["scales"], gpu_device), scale_table=dev(c["scale_table"], gpu_device),
                 scale_bound=float(c["bound"]), means=dev(c["means"], gpu_device), segments=S)
        enc = gaans.encode_gaussian(tables, B, N, C, P, gpu_device, y=dev(c["y"], gpu_device), **g)
        out = gaans.decode_gaussian(enc.packed, tables, B, N, C, P, gpu_device, **g)
        want = O.dequantize_elem(sym, c["means"])
    else:
        enc = gaans.encode(tables, B, N, C, P, gpu_device, symbols=dev(sym, gpu_device),
                           indexes=idx, segments=S)
        out = gaans.decode(enc.packed, tables, B, N, C, P, gpu_device, indexes=idx, segments=S)
        want = sym
    assert enc.packed.cpu().numpy().tobytes() == c["payload"]
    got = out.cpu().numpy()
    assert got.dtype == want.dtype and np.array_equal(got.view(np.uint32), want.view(np.uint32))
    buf, offs = gaans.pack_streams(c["streams"], gpu_device)
    full = dev(c["full_indexes"], gpu_device)
    r = gaans.decode_rans64(buf, offs, tables, B, N, C, gpu_device,
                            indexes=full if c["explicit"] else None)
    assert np.array_equal(r.cpu().numpy(), sym)
