"""Writes the golden fixtures of the GA-ANS wave64 format and of the
CompressAI-equivalent Rans64 stream: small seeded inputs and the bytes the
oracle (oracle/gaans_oracle.c) produces for them, as .npz files next to this
script.  Run from the repository root after oracle.build():

    python tests/golden/make_golden.py

The tests load the fixtures (numpy.load, no pickle) and check that the oracle
and the HIP kernels reproduce these bytes exactly, so a change of the format
shows up as a fixture mismatch rather than as a silent drift of both sides.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(REPO, "oracle"), os.path.join(REPO, "fast-compressai_amd")]

import oracle as O  # noqa: E402
from fast_compressai import synthetic  # noqa: E402


def laplace_tables(M, max_cdf, seed):
    w = synthetic._factorized("golden", 1, M, 1, 1, 0.1, 6.0, max_cdf, 1, (16, 16), seed)
    return w.cdfs, w.cdf_sizes, w.offsets


def cases():
    rng = np.random.default_rng(20261201)
    # 1. explicit indexes, ragged last chunk (C=6, P=4), escapes; two segments
    #    per chunk (the last chunk has two steps)
    cdfs, sizes, offs = laplace_tables(6, 24, 1)
    B, C, HW = 2, 6, 37
    idx = rng.integers(0, 6, size=(B, C * HW), dtype=np.int32)
    sym = np.rint(rng.laplace(0, 3, size=(B, C * HW))).astype(np.int32)
    sym[0, 5] = 1000
    sym[1, 77] = -70000
    yield "symbols_explicit", dict(symbols=sym, indexes=idx, cdfs=cdfs, cdf_sizes=sizes,
                                   offsets=offs, p_ch=np.int32(4), channels=np.int32(C),
                                   segments=np.int32(2))
    # 2. implicit indexes (table = channel), one lane-short chunk (HW*P < 64)
    B, C, HW = 3, 6, 5
    sym = np.rint(rng.laplace(0, 2, size=(B, C * HW))).astype(np.int32)
    yield "symbols_implicit", dict(symbols=sym, indexes=np.zeros(0, np.int32), cdfs=cdfs,
                                   cdf_sizes=sizes, offsets=offs, p_ch=np.int32(2),
                                   channels=np.int32(C), segments=np.int32(1))
    # 3. fused quantize: fp32 latents and per-channel medians; three segments
    #    (one step each)
    B, C, HW = 1, 6, 50
    med = rng.normal(0, 0.3, C).astype(np.float32)
    y = (rng.laplace(0, 2, size=(B, C, HW)) + med[None, :, None]).astype(np.float32)
    y[0, 0, :4] = [0.5, 1.5, -0.5, -2.5]  # ties round to even
    sym = O.quantize(y, med).reshape(B, -1)
    yield "latents", dict(y=y.reshape(B, -1), medians=med, symbols=sym, cdfs=cdfs,
                          cdf_sizes=sizes, offsets=offs, p_ch=np.int32(3), channels=np.int32(C),
                          segments=np.int32(3))
    # 4. Gaussian: build_indexes over a log-spaced scale table, means
    table, gcdfs, gsizes, goffs = gaussian_tables()
    B, C, HW = 1, 4, 40
    scales = np.exp(rng.uniform(np.log(0.05), np.log(40.0), (B, C * HW))).astype(np.float32)
    scales[0, :4] = [np.nan, np.inf, 0.0, table[3]]
    means = rng.normal(0, 1, (B, C * HW)).astype(np.float32)
    y = (means + rng.normal(0, 1, (B, C * HW)) * np.nan_to_num(np.clip(scales, 0.11, 40.0),
                                                               nan=40.0)).astype(np.float32)
    idx = O.build_indexes(scales, table, 0.11)
    sym = O.quantize_elem(y, means)
    yield "gaussian", dict(y=y, scales=scales, means=means, scale_table=table, bound=np.float32(0.11),
                           indexes=idx, symbols=sym, cdfs=gcdfs, cdf_sizes=gsizes, offsets=goffs,
                           p_ch=np.int32(2), channels=np.int32(C), segments=np.int32(2))


def gaussian_tables():
    import math
    table = np.exp(np.linspace(math.log(0.11), math.log(40.0), 16)).astype(np.float32)
    tabs = [synthetic.gaussian_pmf(float(s), int(math.ceil(float(s) * 6.109410204869)))
            for s in table]
    cdfs, sizes, offsets = synthetic.build_tables(tabs)
    return table, cdfs, sizes, offsets


def main():
    O.build()
    for name, c in cases():
        sym, cdfs, sizes, offs = c["symbols"], c["cdfs"], c["cdf_sizes"], c["offsets"]
        B, N = sym.shape
        C = int(c["channels"])
        idx = c.get("indexes")
        full = (idx if idx is not None and idx.size else
                np.repeat(np.arange(C, dtype=np.int32), N // C)[None].repeat(B, 0))
        payload = O.gaans_encode(sym, full if idx is not None and idx.size else None, cdfs,
                                 sizes, offs, int(c["p_ch"]), C, int(c["segments"]))
        streams = [O.rans64_encode(sym[b], full[b], cdfs, sizes, offs) for b in range(B)]
        lens = np.array([len(s) for s in streams], np.int64)
        np.savez(os.path.join(HERE, f"{name}.npz"), **c,
                 payload=np.frombuffer(payload, np.uint8),
                 rans64=np.frombuffer(b"".join(streams), np.uint8), rans64_lengths=lens)
        print(name, "payload", len(payload), "rans64", int(lens.sum()))


if __name__ == "__main__":
    main()
