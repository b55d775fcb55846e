"""Fuzz driver of the library's host-only code (csrc/gaans_host.cpp: table
preparation, layout, segment choice, self test), run by
tests/test_sanitizers.py in a child process against a g++ build with
AddressSanitizer and UndefinedBehaviorSanitizer:

    python tests/host_fuzz.py <libgaans_host.so> [iterations]

Valid tables must prepare (and give a blob of the announced size whose
descriptor is consistent); malformed ones (bad sizes, CDFs that do not start
at 0, end at 65536 or increase, extreme values and offsets, NULL pointers,
short buffers) must be refused with an error code; shapes and segment counts
outside the layout's limits must be refused.  The sanitizers turn any
out-of-bounds access or undefined operation into a non-zero exit.
"""

import ctypes
import sys

import numpy as np

I32_MIN, I32_MAX = -(2**31), 2**31 - 1


class Tables(ctypes.Structure):  # gaans_tables (include/gaans_w64.h)
    _fields_ = [("dev", ctypes.c_void_p), ("bytes", ctypes.c_int64), ("M", ctypes.c_int32),
                ("max_nsym", ctypes.c_int32), ("total_nsym", ctypes.c_int64),
                ("digest", ctypes.c_uint64), ("max_dense", ctypes.c_int32),
                ("flags", ctypes.c_int32), ("total_dense", ctypes.c_int64),
                ("mean_bits", ctypes.c_float), ("max_wide", ctypes.c_int32),
                ("total_wide", ctypes.c_int64)]


class Layout(ctypes.Structure):  # gaans_layout
    _fields_ = [(n, ctypes.c_int64) for n in (
        "B", "N", "C", "P", "S", "HW", "K", "chunk_len", "U", "header_bytes",
        "max_payload_bytes", "cap_words", "workspace_bytes", "ws_chunk_words",
        "ws_chunk_status", "ws_index_hash", "ws_end_off", "ws_info", "ws_states", "ws_words",
        "ws_esc", "ws_esc_raw", "ws_look")]


def load(path):
    L = ctypes.CDLL(path)
    p, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    L.gaans_tables_bytes.argtypes = [p, p, i32, i32, ctypes.POINTER(i64)]
    L.gaans_tables_prepare.argtypes = [p, p, p, i32, i32, p, i64, ctypes.POINTER(Tables)]
    L.gaans_get_layout.argtypes = [i64, i64, i64, i64, i32, ctypes.POINTER(Layout)]
    L.gaans_choose_segments.argtypes = [ctypes.POINTER(Tables), i64, i64, i64, i64,
                                        ctypes.c_double, i64, ctypes.POINTER(i32)]
    L.gaans_rans64_decode_host.argtypes = [p, p, p, p, p, p, i32, i32, i64, i64, i64, i32, p, p]
    L.gaans_last_error.restype = ctypes.c_char_p
    return L


def valid_cdf(rng, S):
    f = rng.integers(1, 1000, S - 1).astype(np.float64)
    if rng.random() < 0.3:  # a few tiny frequencies: dense lookup buckets
        f[rng.integers(0, S - 1, max(1, (S - 1) // 3))] = 1e-9
    f = np.floor(f / f.sum() * (65536 - (S - 1))).astype(np.int64) + 1
    f[np.argmax(f)] += 65536 - f.sum()
    return np.concatenate([[0], np.cumsum(f)]).astype(np.int64)


def tables(rng, M, Lmax):
    cdfs = np.zeros((M, Lmax), np.int32)
    sizes = np.zeros(M, np.int32)
    for t in range(M):
        S = int(rng.integers(2, Lmax + 1))
        cdfs[t, :S] = valid_cdf(rng, S)
        sizes[t] = S
    offs = rng.integers(-1000, 1000, M).astype(np.int32)
    return cdfs, sizes, offs


def prepare(L, cdfs, sizes, offs, M=None, Lmax=None, short=0, null=None):
    M = cdfs.shape[0] if M is None else M
    Lmax = cdfs.shape[1] if Lmax is None else Lmax
    ptr = lambda a, name: None if null == name else a.ctypes.data
    nb = ctypes.c_int64(-1)
    rc = L.gaans_tables_bytes(ptr(cdfs, "cdfs"), ptr(sizes, "sizes"), M, Lmax, ctypes.byref(nb))
    if rc:
        return rc, None
    out = np.zeros(max(int(nb.value) - short, 1), np.uint8)
    d = Tables()
    rc = L.gaans_tables_prepare(ptr(cdfs, "cdfs"), ptr(sizes, "sizes"), ptr(offs, "offs"), M,
                                Lmax, None if null == "out" else out.ctypes.data,
                                int(nb.value) - short, ctypes.byref(d))
    return rc, (d, nb.value)


def check_valid(L, rng):
    M, Lmax = int(rng.integers(1, 40)), int(rng.integers(2, 300))
    cdfs, sizes, offs = tables(rng, M, Lmax)
    if rng.random() < 0.2:
        offs[rng.integers(0, M)] = rng.choice([I32_MIN, I32_MAX, I32_MIN + 65535, I32_MAX - 65535])
    rc, got = prepare(L, cdfs, sizes, offs)
    assert rc == 0, L.gaans_last_error()
    d, nb = got
    assert d.bytes == nb and d.M == M and d.total_nsym == int((sizes - 1).sum())
    assert d.max_nsym == int((sizes - 1).max()) and 0 <= d.max_dense and d.max_dense <= d.total_dense
    assert 0.0 <= d.mean_bits <= 16.0
    # the segment choice on this descriptor, for random shapes
    for _ in range(4):
        C = int(rng.integers(1, 300))
        HW, P = int(rng.integers(1, 5000)), int(rng.integers(1, C + 1))
        out = ctypes.c_int32(0)
        rc = L.gaans_choose_segments(ctypes.byref(d), int(rng.integers(1, 70)), C * HW, C, P,
                                     float(rng.choice([0.0, 0.006, 0.1, 10.0])),
                                     int(rng.integers(-5, 2000)), ctypes.byref(out))
        assert rc == 0 and 1 <= out.value <= 256, L.gaans_last_error()


def check_malformed(L, rng):
    M, Lmax = int(rng.integers(1, 12)), int(rng.integers(2, 80))
    cdfs, sizes, offs = tables(rng, M, Lmax)
    t = int(rng.integers(0, M))
    S = int(sizes[t])
    kind = int(rng.integers(0, 12))
    kw = {}
    if kind == 0:
        sizes[t] = rng.choice([0, 1, -1, Lmax + 1, 65537, I32_MIN, I32_MAX])
    elif kind == 1:
        cdfs[t, 0] = rng.choice([1, -1, I32_MIN, 65536])
    elif kind == 2:
        cdfs[t, S - 1] = rng.choice([65535, 65537, I32_MAX, 0])
    elif kind == 3 and S >= 3:
        j = int(rng.integers(1, S - 1))
        cdfs[t, j] = cdfs[t, j - 1]  # not strictly increasing
    elif kind == 4:
        cdfs[t, :S] = rng.integers(I32_MIN, I32_MAX, S, dtype=np.int64).astype(np.int32)
    elif kind == 5:
        kw["M"] = int(rng.choice([0, -1, 65537, I32_MIN]))
    elif kind == 6:
        kw["Lmax"] = int(rng.choice([1, 0, -3]))
    elif kind == 7:
        kw["null"] = str(rng.choice(["cdfs", "sizes", "offs", "out"]))
    elif kind == 8:
        kw["short"] = int(rng.integers(1, 64))
    elif kind == 9 and S >= 3:
        cdfs[t, 1:S - 1] = cdfs[t, 1:S - 1][::-1]  # decreasing middle
    elif kind == 10:
        cdfs[t, :S] = np.linspace(0, 65536, S).astype(np.int32)[::-1]
    else:
        cdfs[t, S - 1] = 65536
        cdfs[t, max(S - 2, 0)] = 65536  # a zero frequency at the end
    rc, _ = prepare(L, cdfs, sizes, offs, **kw)
    M_, Lmax_ = kw.get("M", M), kw.get("Lmax", Lmax)
    valid = M_ == M and Lmax_ == Lmax and "null" not in kw and "short" not in kw
    valid = valid and all(table_ok(cdfs[u], int(sizes[u]), Lmax) for u in range(M))
    assert (rc == 0) == valid, (kind, rc, L.gaans_last_error())


def table_ok(c, S, Lmax):
    if not 2 <= S <= min(Lmax, 65536):
        return False
    c = c[:S].astype(np.int64)
    return c[0] == 0 and c[-1] == 65536 and bool(np.all(np.diff(c) > 0))


def check_layout(L, rng):
    for _ in range(8):
        vals = [int(rng.choice([rng.integers(-3, 70), rng.integers(1, 2**20), 2**31, 2**40]))
                for _ in range(4)]
        S = int(rng.choice([rng.integers(-2, 300), 2**31 - 1, -(2**31)]))
        lay = Layout()
        rc = L.gaans_get_layout(vals[0], vals[1], vals[2], vals[3], S, ctypes.byref(lay))
        if rc == 0:
            B, N, C, P = vals
            assert N % C == 0 and 1 <= P <= C and 1 <= lay.S <= 256
            assert lay.U == B * lay.K * lay.S and lay.workspace_bytes > 0
            assert lay.max_payload_bytes >= lay.header_bytes


def check_rans64_host(L, rng):
    """The host Rans64 decoder on byte strings that are random, empty, odd
    lengths or random tails of words, with valid or malformed tables and
    indexes in and out of range: every call returns, and nothing is read or
    written out of bounds (ASan)."""
    M, Lmax = int(rng.integers(1, 10)), int(rng.integers(2, 120))
    cdfs, sizes, offs = tables(rng, M, Lmax)
    if rng.random() < 0.2:
        t = int(rng.integers(0, M))
        cdfs[t, 0] = 5  # malformed: rejected before any stream is read
    B = int(rng.integers(1, 6))
    C = int(rng.integers(1, M + 1))
    N = C * int(rng.integers(1, 40))
    strings = []
    for _ in range(B):
        n = int(rng.choice([0, 3, 4, 8, 12, int(rng.integers(0, 4 * N + 16))]))
        strings.append(rng.integers(0, 256, n, dtype=np.int64).astype(np.uint8).tobytes())
    so = np.zeros(B + 1, np.int64)
    np.cumsum([len(x) for x in strings], out=so[1:])
    buf = np.frombuffer(b"".join(strings) + b"\0", np.uint8)  # never empty
    idx = None
    if rng.random() < 0.5:
        idx = rng.integers(-2, M + 2, (B, N), dtype=np.int64).astype(np.int32)
    out = np.zeros((B, N), np.int32)
    st = ctypes.c_uint32(0)
    rc = L.gaans_rans64_decode_host(buf.ctypes.data, so.ctypes.data,
                                    None if idx is None else idx.ctypes.data, cdfs.ctypes.data,
                                    sizes.ctypes.data, offs.ctypes.data, M, Lmax, B, N, C,
                                    int(rng.integers(0, 4)), out.ctypes.data, ctypes.byref(st))
    tables_valid = all(table_ok(cdfs[u], int(sizes[u]), Lmax) for u in range(M))
    assert (rc == 0) == tables_valid, (rc, L.gaans_last_error())
    if rc == 0:
        assert st.value & ~0x12 == 0  # GAANS_ST_CORRUPT | GAANS_ST_INDEX only


def main():
    L = load(sys.argv[1])
    iters = int(sys.argv[2]) if len(sys.argv) > 2 else 300
    assert L.gaans_host_selftest() == 0, L.gaans_last_error()
    rng = np.random.default_rng(2026)
    for _ in range(iters):
        check_valid(L, rng)
        check_malformed(L, rng)
        check_layout(L, rng)
        check_rans64_host(L, rng)
    d = Tables()
    out = ctypes.c_int32(0)
    for bits, budget in ((float("nan"), 0.01), (-1.0, 0.01), (2.0, float("nan")), (2.0, -1.0)):
        d.mean_bits = bits
        assert L.gaans_choose_segments(ctypes.byref(d), 1, 64 * 100, 1, 1, budget, 0,
                                       ctypes.byref(out)) != 0
    print("host fuzz ok", iters, "iterations")


if __name__ == "__main__":
    main()
