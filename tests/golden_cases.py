"""Loader of the golden fixtures in tests/golden (written by
tests/golden/make_golden.py): seeded inputs plus the exact GA-ANS payload and
Rans64 stream bytes."""

import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ("symbols_explicit", "symbols_implicit", "latents", "gaussian")


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        c = {k: z[k] for k in z.files}
    c["payload"] = c["payload"].tobytes()
    lens = c["rans64_lengths"]
    blob = c["rans64"].tobytes()
    ends = np.cumsum(lens)
    c["streams"] = [blob[e - n:e] for n, e in zip(lens, ends)]
    c["channels"] = int(c["channels"])
    c["p_ch"] = int(c["p_ch"])
    c["segments"] = int(c["segments"])
    sym = c["symbols"]
    B, N = sym.shape
    idx = c.get("indexes")
    c["explicit"] = idx is not None and idx.size > 0 and name != "latents"
    c["full_indexes"] = idx if c["explicit"] else np.repeat(
        np.arange(c["channels"], dtype=np.int32), N // c["channels"])[None].repeat(B, 0)
    return c
