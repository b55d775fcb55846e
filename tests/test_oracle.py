"""Pins the CPU oracle (oracle/gaans_oracle.c) before it is trusted as the
checker of the HIP kernels.

* Rans64 (CompressAI-equivalent) stream: hand-derived known-answer vectors,
  including the survey's KAT for cdf [0, 32768, 65536] and the escape cases of
  the reference's CPU coder tests (tests/test_coders.py:25-31, :78-81).
* wave64 format: hand-derived payloads in which every coding step can be
  followed on paper (freq-1 tables make each renormalisation word equal to a
  known symbol), so lane order, group order, the escape section (nibble
  order, word order, pad), states and the header layout are each pinned by a
  literal value.
* Round trips of the reference's GPU test cases
  (tests/gpu/test_warp_div_cuda.py:18-41) and of random cases.
* Quantize/dequantize closed forms against torch's own round / add.
"""

import math
import struct

import numpy as np
import pytest
import torch

import oracle as O

CDF2 = [[0, 32768, 65536]]  # two bins: value 0 and the escape bin


# ---------------------------------------------------------------------------
# Rans64 single stream (CompressAI BufferedRansEncoder equivalent)
# ---------------------------------------------------------------------------

def words(data: bytes):
    return list(struct.unpack(f"<{len(data) // 4}I", data))


def test_rans64_kat_single_symbol():
    # x = 2^31 < x_max = 2^62, so x' = (2^31 / 2^15) << 16 = 2^32; flush (lo, hi) = (0, 1)
    assert O.rans64_encode([0], [0], CDF2, [3], [0]).hex() == "0000000001000000"


def test_rans64_kat_escape_pattern_of_reference_cpu_test():
    # symbols [0, 1, 0, 1]: with cdf_size 3 the value 1 is the escape bin, raw = 0,
    # so each 1 pushes main(32768, 32768) + bits(0).  Reverse encoding from 2^31:
    #   bits(0): 2^35; main esc: 2^36 + 2^15; main 0: 2^37 + 2^16;
    #   bits(0): 2^41 + 2^20; main esc: 2^42 + 2^21 + 2^15; main 0: 2^43 + 2^22 + 2^16
    x = 2**43 + 2**22 + 2**16
    data = O.rans64_encode([0, 1, 0, 1], [0] * 4, CDF2, [3], [0])
    assert words(data) == [x & 0xFFFFFFFF, x >> 32]
    assert list(O.rans64_decode(data, [0] * 4, CDF2, [3], [0])) == [0, 1, 0, 1]


def test_rans64_kat_escape_value_two():
    # symbol 2 -> raw 2 (one nibble): bits(2): 2^35 + 2; bits(n=1): 2^39 + 33;
    # main esc: (2^39 + 33) / 2^15 = 2^24 r 33 -> 2^40 + 33 + 32768
    x = 2**40 + 32801
    data = O.rans64_encode([2], [0], CDF2, [3], [0])
    assert data.hex() == "2180000000010000"
    assert words(data) == [x & 0xFFFFFFFF, x >> 32]
    assert list(O.rans64_decode(data, [0], CDF2, [3], [0])) == [2]


def test_rans64_kat_renormalisation_word():
    # cdf [0, 1, 2, 65536]: symbol 1 has start 1, freq 1 (x_max = 2^47).
    # last symbol: x = 2^31 << 16 | 1 = 2^47 + 1; first symbol: x >= 2^47 emits its
    # low word 1, x = 2^15, x' = 2^31 + 1.  Memory order: flush lo, flush hi, word.
    cdf = [[0, 1, 2, 65536]]
    data = O.rans64_encode([1, 1], [0, 0], cdf, [4], [0])
    assert words(data) == [0x80000001, 0x00000000, 0x00000001]
    assert list(O.rans64_decode(data, [0, 0], cdf, [4], [0])) == [1, 1]


def test_rans64_reference_cpu_cases_round_trip():
    for syms in ([0, 1, 0, 1], [2], [0], [5, -3, 1000000, 0, -(2**26)]):
        data = O.rans64_encode(syms, [0] * len(syms), CDF2, [3], [0])
        assert list(O.rans64_decode(data, [0] * len(syms), CDF2, [3], [0])) == syms


def test_rans64_length_close_to_information_content():
    rng = np.random.default_rng(1)
    freq = np.array([30000, 20000, 10000, 5000, 536])
    cdf = [np.concatenate([[0], np.cumsum(freq)]).tolist()]
    p = freq[:-1] / freq[:-1].sum()
    syms = rng.choice(4, size=200000, p=p)
    data = O.rans64_encode(syms, np.zeros_like(syms), cdf, [6], [0])
    info_bits = float(-np.log2(freq[syms] / 65536.0).sum())
    bits = 8 * len(data)
    assert info_bits <= bits <= info_bits * 1.001 + 64


# ---------------------------------------------------------------------------
# wave64 GA-ANS format
# ---------------------------------------------------------------------------

def fnv1a64(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_fnv1a_published_vectors():
    assert fnv1a64(b"") == 0xCBF29CE484222325
    assert fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert fnv1a64(b"foobar") == 0x85944171F73967E8


def table_digest_bytes(cdfs, sizes, offsets) -> bytes:
    out = struct.pack("<I", len(sizes))
    for row, s, o in zip(cdfs, sizes, offsets):
        out += struct.pack("<Ii", s, o) + struct.pack(f"<{s}I", *row[:s])
    return out


def test_table_digest_definition():
    cdfs = np.array([[0, 8192, 16384, 32768, 65536], [0, 32768, 65536, 0, 0]], np.int32)
    sizes, offs = [5, 3], [-2, 7]
    assert O.table_digest(cdfs, sizes, offs) == fnv1a64(table_digest_bytes(cdfs, sizes, offs))


def fmix32(h):
    """MurmurHash3's 32-bit finaliser (Appleby)."""
    h &= 0xFFFFFFFF
    h ^= h >> 16
    h = (h * 0x85EBCA6B) & 0xFFFFFFFF
    h ^= h >> 13
    h = (h * 0xC2B2AE35) & 0xFFFFFFFF
    return h ^ (h >> 16)


def hash_of(tables_per_position):
    h = 0
    for p, tb in enumerate(tables_per_position):
        h += fmix32(p * 0x9E3779B9 + tb + 1)
    return h & 0xFFFFFFFF


def test_index_term_is_murmur3_finaliser():
    # published value of MurmurHash3's fmix32: fmix32(1) = 0x514E28B7, and the
    # finaliser fixes 0; position 0 of table 0 hashes key 1
    assert fmix32(1) == 0x514E28B7 and fmix32(0) == 0
    assert O.index_term(0, 0) == 0x514E28B7
    for p, tb in ((1, 0), (0, 5), (4, 1), (261119, 319), (2**31 - 1, 65535)):
        assert O.index_term(p, tb) == fmix32(p * 0x9E3779B9 + tb + 1)


def test_index_hash_detects_a_swapped_pair():
    # tables 0 and 1 traded between positions p and p + 4: with the additive
    # term (tb + 1) XOR p*0x9E3779B9 (0x9E3779B9 = 1 mod 4) the sums agree;
    # the finaliser separates them
    def additive(tabs):
        return sum((tb + 1) ^ ((p * 0x9E3779B9) & 0xFFFFFFFF)
                   for p, tb in enumerate(tabs)) & 0xFFFFFFFF
    base = [0, 1, 2, 1, 2, 1, 0, 0]
    swapped = list(base)
    swapped[0], swapped[4] = base[4], base[0]
    assert swapped != base and additive(swapped) == additive(base)
    assert hash_of(swapped) != hash_of(base)
    # the oracle's payload records the finaliser hash of each chunk
    cdfs = np.array([[0, 32768, 65536]] * 3, np.int32)
    for tabs in (base, swapped):
        data = O.gaans_encode(np.zeros((1, 8), np.int32), np.array([tabs], np.int32), cdfs,
                              [3] * 3, [0] * 3, 1, channels=1)
        assert struct.unpack_from("<I", data, 64 + 4)[0] == hash_of(tabs)


def header_words(B, N, C, P, K, chunk_len, M, digest, segments=1):
    return [0x31574147, 5, B, N, C, P, K, chunk_len, M, 0x00041040,
            digest & 0xFFFFFFFF, digest >> 32, segments, 0, 0, 0]


def test_gaans_kat_two_lanes_no_renorm():
    # 2 symbols, 2 lanes, table cdf [0, 32768, 65536]: each lane x = 2^16 ->
    # (2^16 / 2^15) << 16 = 2^17, no word.  Payload: 80-byte header, 2 states.
    cdfs, sizes, offs = CDF2, [3], [0]
    data = O.gaans_encode([[0, 0]], None, cdfs, sizes, offs, 1)
    dg = fnv1a64(table_digest_bytes(cdfs, sizes, offs))
    hdr = header_words(1, 2, 1, 1, 1, 2, 1, dg) + [8, hash_of([0, 0]), 0, 0]
    assert data == struct.pack("<20I", *hdr) + struct.pack("<2I", 1 << 17, 1 << 17)
    assert O.gaans_decode(data, None, 1, 2, cdfs, sizes, offs, 1).tolist() == [[0, 0]]


def kat_130():
    # Table: 17 symbols, values 0..15 have freq 1 (start = value), 16 is the
    # escape bin (start 16, freq 65520).  A freq-1 symbol v maps x in
    # [2^16, 2^17) to: emit x & 0xffff, x = 0x10000 + v.  So every word a lane
    # emits is the symbol it coded one step earlier (0 for the initial state).
    S = 18
    cdf = list(range(17)) + [65536]
    s = [(5 * p + 3) % 16 for p in range(130)]
    s[3] = -1    # step 0, lane 3: raw = -2 * -1 - 1 = 1, one nibble
    s[70] = 56   # step 1, lane 6: raw = 2 * (56 - 16) = 0x50, two nibbles
    s[129] = 17  # step 2, lane 1: raw = 2 * (17 - 16) = 2, one nibble
    return [cdf], [S], [0], s


def test_gaans_kat_lane_order_group_order_and_escape_section():
    cdfs, sizes, offs, s = kat_130()
    data = O.gaans_encode([s], None, cdfs, sizes, offs, 1)
    # An escape codes the bin (start 16, freq 65520): from x = 0x10000 + u
    # (u < 16) it gives ((x // 65520) << 16) + x % 65520 + 16 = 0x10020 + u with
    # no word.  Step t=2 (lanes 0, 1): lane 0 emits its initial 0x0000, lane 1
    # (escape) becomes 0x10020.  Step t=1: lane 0 emits s[128], lane 1 emits
    # 0x0020, lane 6 (escape) emits nothing and becomes 0x10020, the other
    # lanes emit 0x0000.  Step t=0: lane l emits s[64 + l], lane 6 emits 0x0020,
    # lane 3 (escape) emits nothing and ends at 0x10020 + s[67]; the others end
    # at 0x10000 + s[l].  Groups are prepended, so the stream is step 0's group,
    # then step 1's, then step 2's: 63 + 63 + 1 = 127 words.
    g0 = [s[64 + l] for l in range(64) if l != 3]
    g0[5] = 0x0020  # lane 6 (index 5 once lane 3 is dropped)
    g1 = [s[128], 0x0020] + [0] * 61
    stream = g0 + g1 + [0]
    assert len(stream) == 127
    # escape section, position order: p=3 -> [1, 1], p=70 -> [2, 0, 5],
    # p=129 -> [1, 2]; nibbles 1,1,2,0 | 5,1,2 -> words 0x0211, 0x0215, stored
    # last word first at the chunk end, after a zero pad (127 + 2 is odd)
    stream += [0, 0x0215, 0x0211]
    states = [0x10000 + s[l] for l in range(64)]
    states[3] = 0x10020 + s[67]
    chunk = struct.pack("<64I", *states) + struct.pack(f"<{len(stream)}H", *stream)
    assert len(chunk) == 516
    dg = fnv1a64(table_digest_bytes(cdfs, sizes, offs))
    hdr = header_words(1, 130, 1, 1, 1, 130, 1, dg) + [516, hash_of([0] * 130), 0, 0]
    assert data == struct.pack("<20I", *hdr) + chunk
    assert O.gaans_decode(data, None, 1, 130, cdfs, sizes, offs, 1).tolist() == [s]


def test_gaans_kat_three_segments():
    # the 130-symbol chunk (3 steps) in S = 3 segments: unit s is step s alone,
    # coded from fresh states.  Unit 0 (positions 0..63): every lane but 3
    # emits its initial 0x0000 and holds 0x10000 + s[l]; lane 3 (escape, raw 1:
    # nibbles 1, 1 -> word 0x0011) holds 0x10020.  63 + 1 words: no pad.
    # Unit 1 (64..127): the same with s[64 + l], lane 6 escapes (raw 0x50:
    # nibbles 2, 0, 5 -> word 0x0502).  Unit 2 (128, 129; two lanes): lane 0
    # emits 0x0000 and holds 0x10000 + s[128]; lane 1 escapes (raw 2: nibbles
    # 1, 2 -> word 0x0021) and holds 0x10020; 1 + 1 words, no pad.
    cdfs, sizes, offs, s = kat_130()
    data = O.gaans_encode([s], None, cdfs, sizes, offs, 1, segments=3)
    st0 = [0x10000 + s[l] for l in range(64)]
    st0[3] = 0x10020
    st1 = [0x10000 + s[64 + l] for l in range(64)]
    st1[6] = 0x10020
    u0 = struct.pack("<64I", *st0) + struct.pack("<64H", *([0] * 63 + [0x0011]))
    u1 = struct.pack("<64I", *st1) + struct.pack("<64H", *([0] * 63 + [0x0502]))
    u2 = struct.pack("<2I", 0x10000 + s[128], 0x10020) + struct.pack("<2H", 0, 0x0021)
    assert (len(u0), len(u1), len(u2)) == (384, 384, 12)
    dg = fnv1a64(table_digest_bytes(cdfs, sizes, offs))
    # 3 units: header 64 + 24 bytes, padded to 96
    hdr = header_words(1, 130, 1, 1, 1, 130, 1, dg, segments=3) + [
        384, 768, 780, hash_of([0] * 64), hash_of([0] * 64), hash_of([0] * 2), 0, 0]
    assert data == struct.pack("<24I", *hdr) + u0 + u1 + u2
    assert O.gaans_decode(data, None, 1, 130, cdfs, sizes, offs, 1, segments=3).tolist() == [s]
    # the segment count is part of the format: decoding with another one fails
    for other in (1, 2):
        with pytest.raises(O.OracleError):
            O.gaans_decode(data, None, 1, 130, cdfs, sizes, offs, 1, segments=other)


def test_gaans_kat_two_interleaved_segments():
    # the 130-symbol chunk (3 steps) in S = 2 segments: unit 0 is steps 0 and
    # 2 (positions 0..63, then 128 and 129 as its step 1), unit 1 is step 1.
    # Unit 0, walked last step first: at its step 1 lane 0 emits its initial
    # 0x0000 and holds 0x10000 + s[128]; lane 1 escapes (raw 2) and holds
    # 0x10020; the other lanes are inactive.  At its step 0 lane 0 emits
    # s[128] and lane 1 emits 0x0020 (both then hold 0x10000 + s[l]), lane 3
    # escapes (raw 1) from 0x10000 to 0x10020 with no word, every other lane
    # emits 0x0000.  Stream: step 0's group (63 words), then step 1's (1).
    # Escapes in unit position order: p=3 -> [1, 1], p=65 -> [1, 2]: nibbles
    # 1,1,1,2 -> word 0x2111; 64 + 1 words is odd, so a zero pad precedes it.
    # Unit 1 is step 1 coded alone (as unit 1 of the three-segment case).
    cdfs, sizes, offs, s = kat_130()
    data = O.gaans_encode([s], None, cdfs, sizes, offs, 1, segments=2)
    st0 = [0x10000 + s[l] for l in range(64)]
    st0[3] = 0x10020
    w0 = [s[128], 0x0020] + [0] * 61 + [0] + [0, 0x2111]
    st1 = [0x10000 + s[64 + l] for l in range(64)]
    st1[6] = 0x10020
    u0 = struct.pack("<64I", *st0) + struct.pack(f"<{len(w0)}H", *w0)
    u1 = struct.pack("<64I", *st1) + struct.pack("<64H", *([0] * 63 + [0x0502]))
    assert (len(u0), len(u1)) == (388, 384)
    dg = fnv1a64(table_digest_bytes(cdfs, sizes, offs))
    hdr = header_words(1, 130, 1, 1, 1, 130, 1, dg, segments=2) + [
        388, 772, hash_of([0] * 66), hash_of([0] * 64)]
    assert data == struct.pack("<20I", *hdr) + u0 + u1
    assert O.gaans_decode(data, None, 1, 130, cdfs, sizes, offs, 1, segments=2).tolist() == [s]


def segment_steps(T, S):
    """Steps of a T-step chunk in segment s, in the unit's order: s, s + S, ..."""
    return [list(range(s, T, S)) for s in range(S)]


def test_gaans_segments_are_independent_units():
    # Every unit of an S-segment payload is, byte for byte, the one-chunk
    # payload of its own positions, in its steps' order, coded alone (B = 1,
    # one channel, the positions' tables as explicit indexes): same states,
    # words, escapes and index hash.  The segments' steps are computed here
    # independently of the oracle.
    rng = np.random.default_rng(5)
    for trial in range(20):
        B, C = int(rng.integers(1, 3)), int(rng.integers(1, 6))
        HW, P = int(rng.integers(1, 500)), int(rng.integers(1, C + 1))
        N, K = C * HW, -(-C // P)
        cdfs, sizes, offs = random_tables(rng, C, int(rng.integers(2, 20)))
        s = rng.integers(-30, 30, (B, N)).astype(np.int32)
        Tmin = -(-(N - (K - 1) * P * HW) // 64)
        S = int(rng.integers(1, min(Tmin, 9) + 1))
        data = O.gaans_encode(s, None, cdfs, sizes, offs, P, segments=S)
        U = B * K * S
        hb = (64 + 8 * U + 15) // 16 * 16
        ends = struct.unpack_from(f"<{U}I", data, 64)
        hashes = struct.unpack_from(f"<{U}I", data, 64 + 4 * U)
        prev, g = 0, 0
        for b in range(B):
            for k in range(K):
                cs, ce = k * P * HW, min((k + 1) * P * HW, N)
                for steps in segment_steps(-(-(ce - cs) // 64), S):
                    assert steps
                    pos = np.concatenate([np.arange(cs + 64 * j, min(cs + 64 * j + 64, ce))
                                          for j in steps])
                    seg = s[b, pos][None]
                    tabs = (pos // HW).astype(np.int32)[None]
                    alone = O.gaans_encode(seg, tabs, cdfs, sizes, offs, 1, channels=1)
                    hb1 = (64 + 8 + 15) // 16 * 16
                    assert data[hb + prev: hb + ends[g]] == alone[hb1:]
                    assert hashes[g] == struct.unpack_from("<I", alone, 68)[0]
                    prev, g = ends[g], g + 1
        assert hb + prev == len(data)
        out = O.gaans_decode(data, None, B, N, cdfs, sizes, offs, P, segments=S)
        assert (out == s).all()


def test_gaans_segment_count_limits():
    cdfs, sizes, offs = CDF2, [3], [0]
    z = np.zeros((1, 200), np.int32)  # one chunk of 4 steps
    for S in (1, 2, 3, 4):
        data = O.gaans_encode(z, None, cdfs, sizes, offs, 1, segments=S)
        assert O.gaans_decode(data, None, 1, 200, cdfs, sizes, offs, 1, segments=S).tolist() == z.tolist()
    # at least one step per segment, at most 256 segments, at least one
    for S in (0, 5, -1):
        with pytest.raises(O.OracleError):
            O.gaans_encode(z, None, cdfs, sizes, offs, 1, segments=S)
    # the limit is set by the shortest chunk of a row: C = 3, P = 2, HW = 64:
    # chunks of 2 and 1 steps
    z3 = np.zeros((1, 192), np.int32)
    t3 = [[0, 32768, 65536]] * 3
    O.gaans_encode(z3, None, t3, [3] * 3, [0] * 3, 2, segments=1)
    with pytest.raises(O.OracleError):
        O.gaans_encode(z3, None, t3, [3] * 3, [0] * 3, 2, segments=2)
    big = np.zeros((1, 64 * 300), np.int32)
    O.gaans_encode(big, None, cdfs, sizes, offs, 1, segments=256)
    with pytest.raises(O.OracleError):
        O.gaans_encode(big, None, cdfs, sizes, offs, 1, segments=257)


def test_gaans_escape_section_word_order_without_pad():
    # one escape with raw 0x12345 (5 nibbles): nibbles 5,5,4,3 | 2,1 -> words
    # 0x3455, 0x0012 at the chunk end, last word first; no rANS words (one lane,
    # escape bin freq 32768 from x = 2^16 gives 2^17 + 32768, no emit), so
    # W + Q = 2 is even and there is no pad
    cdfs, sizes, offs = CDF2, [3], [0]
    raw = 0x12345  # odd: value -(raw >> 1) - 1
    sym = -(raw >> 1) - 1
    data = O.gaans_encode([[sym]], None, cdfs, sizes, offs, 1)
    hb = (64 + 8 + 15) // 16 * 16
    chunk = data[hb:]
    assert struct.unpack("<IHH", chunk) == ((1 << 17) + 32768, 0x0012, 0x3455)
    assert O.gaans_decode(data, None, 1, 1, cdfs, sizes, offs, 1).tolist() == [[sym]]
    bad = bytearray(data)
    bad[hb + 5] |= 0x80  # an unused nibble of the last escape word (bits 12..15)
    with pytest.raises(O.OracleError):
        O.gaans_decode(bytes(bad), None, 1, 1, cdfs, sizes, offs, 1)


def test_gaans_escape_count_must_be_minimal():
    # one escape of raw 2 (even: value (raw >> 1) + maxv = 2): nibbles 1, 2 ->
    # escape word 0x0021; the state 2^17 + 32768 emits nothing, so W = 0,
    # Q = 1 and a zero pad word precedes the escape word.  Rewriting the entry
    # as count 2, nibbles 2, 0 (same raw, same word count) must be rejected.
    cdfs, sizes, offs = CDF2, [3], [0]
    data = O.gaans_encode([[2]], None, cdfs, sizes, offs, 1)
    hb = (64 + 8 + 15) // 16 * 16
    assert struct.unpack("<IHH", data[hb:]) == ((1 << 17) + 32768, 0, 0x0021)
    assert O.gaans_decode(data, None, 1, 1, cdfs, sizes, offs, 1).tolist() == [[2]]
    bad = bytearray(data)
    struct.pack_into("<H", bad, hb + 6, 0x0022)
    with pytest.raises(O.OracleError) as err:
        O.gaans_decode(bytes(bad), None, 1, 1, cdfs, sizes, offs, 1)
    assert err.value.code == -6  # payload corrupt


def test_tables_beyond_16_bit_symbol_numbers_rejected():
    # escape symbols (cdf size - 2) and table numbers are 16-bit in the decoder
    cdf = np.arange(65537, dtype=np.int32)[None, :]
    with pytest.raises(O.OracleError):
        O.gaans_encode([[0]], None, cdf, [65537], [0], 1)
    cdf = np.arange(65536, dtype=np.int32)[None, :].copy()
    cdf[0, -1] = 65536
    data = O.gaans_encode([[70000]], None, cdf, [65536], [0], 1)
    assert O.gaans_decode(data, None, 1, 1, cdf, [65536], [0], 1).tolist() == [[70000]]


def test_gaans_chunking_and_header_offsets():
    # 3 channels of HW = 2, P = 2 -> chunks of 4 and 2 symbols; 2 rows.
    cdfs = np.array([[0, 32768, 65536]] * 3, np.int32)
    sym = np.zeros((2, 6), np.int32)
    data = O.gaans_encode(sym, None, cdfs, [3] * 3, [0] * 3, 2)
    hb = (64 + 8 * 4 + 15) // 16 * 16
    ends = struct.unpack_from("<4I", data, 64)
    assert ends == (16, 24, 40, 48)  # 4 states, 2 states, 4, 2 (no words)
    assert len(data) == hb + 48
    hashes = struct.unpack_from("<4I", data, 64 + 16)
    assert hashes == (hash_of([0, 0, 1, 1]), hash_of([2, 2]), hash_of([0, 0, 1, 1]),
                      hash_of([2, 2]))


REF_CDFS = [[0, 8192, 16384, 32768, 65536]] * 4
REF_OFFS = [-2, -1, 0, 1]


@pytest.mark.parametrize("symbols,p_ch", [([0, 1, 2, 3] * 16, 1), ([0, 1, 2, 3] * 16, 2),
                                          ([0, 1, 2, 3] * 16, 4),
                                          ([-100, 100, -101, 102] * 16, 2)])
def test_gaans_reference_gpu_test_cases_round_trip(symbols, p_ch):
    # tests/gpu/test_warp_div_cuda.py:18-41: four tables, indexes [0,1,2,3]*16
    s = np.array([symbols], np.int32)
    idx = np.array([[0, 1, 2, 3] * 16], np.int32)
    data = O.gaans_encode(s, idx, REF_CDFS, [5] * 4, REF_OFFS, p_ch)
    assert (O.gaans_decode(data, idx, 1, 64, REF_CDFS, [5] * 4, REF_OFFS, p_ch) == s).all()


def random_tables(rng, M, max_size):
    cdfs = np.zeros((M, max_size), np.int32)
    sizes = np.zeros(M, np.int32)
    for t in range(M):
        S = int(rng.integers(2, max_size + 1))
        f = rng.integers(1, 1000, S - 1).astype(np.float64)
        f = np.floor(f / f.sum() * (65536 - (S - 1))).astype(np.int64) + 1
        f[np.argmax(f)] += 65536 - f.sum()
        cdfs[t, :S] = np.concatenate([[0], np.cumsum(f)])
        sizes[t] = S
    return cdfs, sizes, rng.integers(-20, 20, M).astype(np.int32)


def test_gaans_random_round_trips_and_implicit_indexes():
    rng = np.random.default_rng(0)
    for trial in range(60):
        B, C = int(rng.integers(1, 3)), int(rng.integers(1, 9))
        HW, P = int(rng.integers(1, 150)), int(rng.integers(1, C + 1))
        cdfs, sizes, offs = random_tables(rng, C, int(rng.integers(2, 24)))
        s = rng.integers(-40, 40, (B, C * HW)).astype(np.int32)
        if trial % 4 == 0:
            s.flat[int(rng.integers(s.size))] = 2**30 + 5
        idx = np.broadcast_to(np.repeat(np.arange(C, dtype=np.int32), HW), s.shape)
        data = O.gaans_encode(s, None, cdfs, sizes, offs, P)
        assert data == O.gaans_encode(s, idx, cdfs, sizes, offs, P)
        assert (O.gaans_decode(data, idx, B, C * HW, cdfs, sizes, offs, P) == s).all()


def test_gaans_escape_extremes_and_range_error():
    cdfs, sizes = CDF2, [3]
    s = np.array([[-(2**31), 2**31 - 1, 0, 1, 2**31 - 2]], np.int32)
    data = O.gaans_encode(s, None, cdfs, sizes, [0], 1)
    assert (O.gaans_decode(data, None, 1, 5, cdfs, sizes, [0], 1) == s).all()
    with pytest.raises(O.OracleError) as err:  # raw = 2 * (2^31 - 1 + 100 - 1) >= 2^32
        O.gaans_encode(np.array([[2**31 - 1]], np.int32), None, cdfs, sizes, [-100], 1)
    assert err.value.code == -4


def test_gaans_detects_corruption_and_mismatch():
    rng = np.random.default_rng(3)
    cdfs, sizes, offs = random_tables(rng, 4, 16)
    s = rng.integers(-5, 5, (1, 4 * 100)).astype(np.int32)
    data = bytearray(O.gaans_encode(s, None, cdfs, sizes, offs, 2))
    hb = (64 + 8 * 2 + 15) // 16 * 16
    bad = bytearray(data)
    bad[hb + 300] ^= 0x40  # inside the first chunk's word stream
    with pytest.raises(O.OracleError):
        out = O.gaans_decode(bytes(bad), None, 1, 400, cdfs, sizes, offs, 2)
        assert not (out == s).all()
        raise O.OracleError(-6, "undetected corruption")
    other = cdfs.copy()
    other[0, 1] += 1
    with pytest.raises(O.OracleError) as err:
        O.gaans_decode(bytes(data), None, 1, 400, other, sizes, offs, 2)
    assert err.value.code == -7
    idx = np.broadcast_to(np.repeat(np.arange(4, dtype=np.int32), 100), (1, 400)).copy()
    idx[0, 5] = 1  # same first chunk, other table for one symbol
    with pytest.raises(O.OracleError):
        O.gaans_decode(bytes(data), idx, 1, 400, cdfs, sizes, offs, 2)


def test_gaans_bpp_overhead_is_the_lane_flush():
    # per chunk the format adds ~64 states * 32 bits over the ideal stream;
    # a single CompressAI-style stream carries one 64-bit flush.  The rest is
    # the quantisation loss of 32-bit states renormalised by 16 bits (x / freq
    # can be small), here under 0.5% with 73% of the symbols escapes.
    rng = np.random.default_rng(5)
    cdfs, sizes, offs = random_tables(rng, 8, 32)
    s = rng.integers(-6, 6, (1, 8 * 4096)).astype(np.int32)
    idx = np.repeat(np.arange(8, dtype=np.int32), 4096)
    single = len(O.rans64_encode(s[0], idx, cdfs, sizes, offs))
    for P in (1, 2, 8):
        data = O.gaans_encode(s, None, cdfs, sizes, offs, P)
        K = math.ceil(8 / P)
        hb = (64 + 8 * K + 15) // 16 * 16
        overhead = len(data) - hb - single
        assert 0 < overhead <= K * (64 * 4 + 2) + 0.005 * single


# ---------------------------------------------------------------------------
# quantize / dequantize closed forms (CompressAI EntropyModel.quantize("symbols")
# = round(y - means).int(), dequantize = symbols.type_as(means) + means)
# ---------------------------------------------------------------------------

def test_quantize_matches_torch_round_half_even():
    med = np.array([0.0, 0.25, -1.5, 1e3], np.float32)
    base = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, -0.0, 0.49999997, 1e6 + 0.5,
                     8388607.5, -8388608.5, 3.0], np.float32)
    y = np.stack([base + m for m in med])[None]  # [1, 4, 12]
    ours = O.quantize(y, med)
    ref = torch.round(torch.from_numpy(y) - torch.from_numpy(med)[None, :, None]).int().numpy()
    assert (ours == ref).all()
    rng = np.random.default_rng(0)
    y = (rng.standard_normal((2, 4, 300)) * 50).astype(np.float32)
    ref = torch.round(torch.from_numpy(y) - torch.from_numpy(med)[None, :, None]).int().numpy()
    assert (O.quantize(y, med) == ref).all()


def test_dequantize_matches_torch_add():
    med = np.array([0.1, -3.3, 7.77], np.float32)
    s = np.array([[[0, 1, -1, 2**24 + 1, -(2**25) - 3], [5, 6, 7, 8, 9],
                   [-100, 100, 2**30, -(2**31), 2**31 - 1]]], np.int32)
    ref = (torch.from_numpy(s).float() + torch.from_numpy(med)[None, :, None]).numpy()
    assert np.array_equal(O.dequantize(s, med).view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------------------
# GaussianConditional build_indexes and elementwise quantize (restated)
# ---------------------------------------------------------------------------

SCALE_TABLE = np.exp(np.linspace(math.log(0.11), math.log(256.0), 64)).astype(np.float32)


def test_build_indexes_matches_searchsorted_on_sorted_tables():
    # for a sorted table, (L - 1) - #{k < L - 1 : lb <= t_k} = #{k < L - 1 : t_k < lb},
    # numpy's searchsorted(t[:-1], lb, 'left') computes the latter independently
    rng = np.random.default_rng(5)
    s = np.exp(rng.uniform(math.log(0.01), math.log(500.0), 20000)).astype(np.float32)
    s[:64] = SCALE_TABLE  # every table value itself
    s[64:128] = np.nextafter(SCALE_TABLE, np.float32(np.inf))
    s[128:192] = np.nextafter(SCALE_TABLE, np.float32(0))
    got = O.build_indexes(s, SCALE_TABLE, 0.11)
    lb = np.maximum(s, np.float32(0.11))
    want = np.searchsorted(SCALE_TABLE[:-1], lb, side="left")
    assert (got == want).all()
    assert (got[:63] == np.arange(63)).all() and got[63] == 63  # t_k -> k; the last -> L - 1


def test_build_indexes_edge_values():
    bound = np.float32(0.11)
    s = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, -5.0, bound,
                  np.nextafter(bound, np.float32(1)), 256.0, 1e30], np.float32)
    got = O.build_indexes(s, SCALE_TABLE, float(bound)).tolist()
    # NaN stays NaN through the lower bound, so no comparison holds: L - 1
    assert got[0] == 63 and got[1] == 63
    # everything at or below the bound maps to the first table entry (= bound)
    assert got[2:7] == [0, 0, 0, 0, 0]
    # 256 is the last table entry, which build_indexes never compares: L - 1
    assert got[7] == 1 and got[8] == 63 and got[9] == 63
    # a one-entry table: no comparisons, index 0
    assert O.build_indexes(s, SCALE_TABLE[:1], 0.11).tolist() == [0] * len(s)


def test_build_indexes_unsorted_table_is_the_literal_count():
    # the restatement assumes no order: count of table entries (but the last)
    # the lower-bounded scale does not exceed, subtracted from L - 1
    t = np.array([3.0, 1.0, 2.0, 0.5], np.float32)
    s = np.array([0.1, 1.5, 2.5, 5.0], np.float32)
    got = O.build_indexes(s, t, 0.11).tolist()
    assert got == [3 - 3, 3 - 2, 3 - 1, 3 - 0]


def test_quantize_elem_and_dequantize_elem_match_torch():
    rng = np.random.default_rng(6)
    y = rng.normal(0, 20, 5000).astype(np.float32)
    m = rng.normal(0, 2, 5000).astype(np.float32)
    y[:6] = m[:6] + np.array([0.5, -0.5, 1.5, -1.5, 2.5, -0.0], np.float32)
    ty, tm = torch.from_numpy(y), torch.from_numpy(m)
    want = torch.round(ty - tm).int().numpy()
    assert (O.quantize_elem(y, m) == want).all()
    assert (O.quantize_elem(y) == torch.round(ty).int().numpy()).all()
    yh = O.dequantize_elem(want, m)
    assert np.array_equal(yh.view(np.uint32), (torch.from_numpy(want).float() + tm).numpy().view(np.uint32))
    assert np.array_equal(O.dequantize_elem(want), want.astype(np.float32))
