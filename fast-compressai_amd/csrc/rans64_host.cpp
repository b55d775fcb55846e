// CompressAI Rans64 streams decoded on the host CPU: the product path for a
// batch of CompressAI strings too small to fill the GPU (one stream is one
// serial chain, so the GPU decoder k_rans64_decode gives one stream a lane and
// pays off only with many streams in flight).
//
// Stream format (CompressAI's RansEncoder / RansDecoder, rans64.h and
// rans_interface.cpp, Apache-2.0; the reference calls it at
// src/fast_compressai/coders/compressai_ans.py:51-87): 64-bit state x,
// L = 2^31, 32-bit renormalisation words, 16-bit CDF precision.  The first
// two words are the final state (low word first).  A symbol of a table with
// S CDF entries: cum = x mod 2^16, s = the entry with cdf[s] <= cum <
// cdf[s + 1], x = freq (x >> 16) + cum - cdf[s], then one word in when x < L.
// s = S - 2 is the escape bin: 4-bit groups taken from the low bits of x
// (each followed by the same renormalisation) give a count n (groups summed
// while a group is 15) and then the n nibbles of raw, least significant
// first; raw odd -> -(raw >> 1) - 1, even -> (raw >> 1) + S - 2, plus the
// table offset.
//
// Written for this library from the format above; the oracle's restatement
// (oracle/gaans_oracle.c) is the checker of this code, not part of it.

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "gaans_common.h"
#include "gaans_w64.h"

using namespace gaans;

namespace {

constexpr uint64_t kR64Low = 1ull << 31;
constexpr int kFirstBits = 8;  // a 256-value bucket index per table
constexpr int kMaxRawNibbles = 8;

// Per table: the symbol holding the first cum value of each 256-value
// bucket (the scan from there meets at most the symbols starting inside the
// bucket).
struct HostTables {
  const int32_t* cdfs;
  int32_t Lmax, M;
  const int32_t* sizes;
  const int32_t* offsets;
  std::vector<uint16_t> first;  // M x 256
};

int build_host_tables(const int32_t* cdfs, const int32_t* sizes, const int32_t* offsets,
                      int32_t M, int32_t Lmax, HostTables* T) {
  if (M < 1 || M > 65536 || Lmax < 2)
    return fail(GAANS_EINVAL, "need 1 <= M <= 65536 tables of Lmax >= 2 entries (got M=%d)", M);
  T->cdfs = cdfs;
  T->Lmax = Lmax;
  T->M = M;
  T->sizes = sizes;
  T->offsets = offsets;
  try {
    T->first.assign((size_t)M << kFirstBits, 0);
  } catch (...) {
    return fail(GAANS_EINVAL, "no host memory for the lookups of %d tables", M);
  }
  for (int32_t t = 0; t < M; ++t) {
    const int32_t S = sizes[t];
    const int32_t* c = cdfs + (int64_t)t * Lmax;
    if (S < 2 || S > Lmax || S > 65536)
      return fail(GAANS_ETABLE, "table %d: cdf size %d outside [2, %d]", t, S,
                  Lmax < 65536 ? Lmax : 65536);
    if (c[0] != 0 || c[S - 1] != 65536)
      return fail(GAANS_ETABLE, "table %d: CDF must start at 0 and end at 65536", t);
    for (int32_t j = 0; j + 1 < S; ++j)
      if (c[j + 1] <= c[j])
        return fail(GAANS_ETABLE, "table %d: CDF is not strictly increasing at entry %d", t, j);
    uint16_t* f = T->first.data() + ((size_t)t << kFirstBits);
    int32_t s = 0;
    for (int32_t b = 0; b < (1 << kFirstBits); ++b) {
      const int32_t lo = b << (16 - kFirstBits);
      while (c[s + 1] <= lo) ++s;  // c[S - 1] = 65536 > lo ends the scan
      f[b] = (uint16_t)s;
    }
  }
  return GAANS_OK;
}

// The word stream of one CompressAI string (little-endian u32, any alignment).
struct Words {
  const uint8_t* p;
  const uint8_t* end;
  bool short_read = false;
  uint32_t next() {
    if (end - p < 4) {
      short_read = true;
      return 0;
    }
    uint32_t w;
    memcpy(&w, p, 4);
    p += 4;
    return w;
  }
};

// 4 bits of the state (a bypass group), with the state's renormalisation.
inline uint32_t take_nibble(uint64_t& x, Words& in) {
  const uint32_t v = (uint32_t)x & 15u;
  x >>= 4;
  if (x < kR64Low) x = (x << 32) | in.next();
  return v;
}

// Decode one stream of n symbols into out; status bits (GAANS_ST_*).
uint32_t decode_one(const HostTables& T, const uint8_t* bytes, int64_t nbytes,
                    const int32_t* idx, int64_t hw, int64_t n, int32_t* out) {
  if (n == 0) return 0;
  if (nbytes < 8 || (nbytes & 3)) return GAANS_ST_CORRUPT;
  Words in{bytes, bytes + nbytes};
  uint64_t x = in.next();
  x |= (uint64_t)in.next() << 32;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t tb = idx ? (int64_t)idx[i] : i / hw;
    if (tb < 0 || tb >= T.M) return GAANS_ST_INDEX;
    const int32_t S = T.sizes[tb];
    const int32_t* c = T.cdfs + tb * (int64_t)T.Lmax;
    const uint32_t cum = (uint32_t)x & 0xffffu;
    int32_t s = T.first[((size_t)tb << kFirstBits) + (cum >> (16 - kFirstBits))];
    while ((uint32_t)c[s + 1] <= cum) ++s;
    const uint32_t start = (uint32_t)c[s];
    x = (uint64_t)((uint32_t)c[s + 1] - start) * (x >> 16) + cum - start;
    if (x < kR64Low) x = (x << 32) | in.next();
    int64_t value = s;
    if (s == S - 2) {  // bypass-coded escape
      uint32_t g = take_nibble(x, in);
      uint32_t count = g;
      while (g == 15u && count <= (uint32_t)kMaxRawNibbles) {
        g = take_nibble(x, in);
        count += g;
      }
      if (count > (uint32_t)kMaxRawNibbles) return GAANS_ST_CORRUPT;
      uint32_t raw = 0;
      for (uint32_t j = 0; j < count; ++j) raw |= take_nibble(x, in) << (4u * j);
      value = (raw & 1u) ? -(int64_t)(raw >> 1) - 1 : (int64_t)(raw >> 1) + (S - 2);
    }
    value += T.offsets[tb];
    if (value < INT32_MIN || value > INT32_MAX) return GAANS_ST_CORRUPT;
    out[i] = (int32_t)value;
    if (in.short_read) return GAANS_ST_CORRUPT;
  }
  return 0;
}

}  // namespace

extern "C" int gaans_rans64_decode_host(const uint8_t* streams, const int64_t* stream_offsets,
                                        const int32_t* indexes, const int32_t* cdfs,
                                        const int32_t* cdf_sizes, const int32_t* offsets,
                                        int32_t M, int32_t Lmax, int64_t B, int64_t N, int64_t C,
                                        int32_t threads, int32_t* out, uint32_t* status) {
  if (!stream_offsets || !cdfs || !cdf_sizes || !offsets || !out || !status)
    return fail(GAANS_EINVAL, "NULL argument");
  if (B < 1 || N < 1 || C < 1 || N % C != 0)
    return fail(GAANS_EINVAL, "need B, N, C >= 1 and N %% C == 0 (B=%lld N=%lld C=%lld)",
                (long long)B, (long long)N, (long long)C);
  if (!indexes && C > M)
    return fail(GAANS_EINVAL, "table = channel needs a table per channel (C=%lld > M=%d)",
                (long long)C, M);
  for (int64_t b = 0; b < B; ++b)
    if (stream_offsets[b] < 0 || stream_offsets[b + 1] < stream_offsets[b])
      return fail(GAANS_EINVAL, "stream offsets must be non-negative and non-decreasing");
  if (!streams && stream_offsets[B] > 0) return fail(GAANS_EINVAL, "streams pointer is NULL");
  HostTables T;
  int rc = build_host_tables(cdfs, cdf_sizes, offsets, M, Lmax, &T);
  if (rc) return rc;
  const int64_t hw = N / C;
  int64_t nthreads = threads > 0 ? threads : (int64_t)std::thread::hardware_concurrency();
  nthreads = std::max<int64_t>(1, std::min<int64_t>(nthreads, B));
  std::atomic<int64_t> next{0};
  std::atomic<uint32_t> all{0};
  auto work = [&]() {
    for (int64_t b; (b = next.fetch_add(1)) < B;) {
      const uint32_t st = decode_one(T, streams + stream_offsets[b],
                                     stream_offsets[b + 1] - stream_offsets[b],
                                     indexes ? indexes + b * N : nullptr, hw, N, out + b * N);
      if (st) all.fetch_or(st);
    }
  };
  if (nthreads == 1) {
    work();
  } else {
    std::vector<std::thread> pool;
    try {
      pool.reserve((size_t)nthreads - 1);
      for (int64_t t = 1; t < nthreads; ++t) pool.emplace_back(work);
    } catch (...) {
      // fewer threads than asked for: the streams are shared out all the same
    }
    work();
    for (auto& th : pool) th.join();
  }
  *status = all.load();
  return GAANS_OK;
}
