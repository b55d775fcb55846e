// Internal definitions shared by the HIP kernels and launch code
// (gaans_w64.hip) and the host-only code (gaans_host.cpp): the payload and
// table-blob format constants, the blob's structs and section layout, the
// chunk / coding-unit layout, and the integer arithmetic that both sides
// compute identically (division by invariant integers, the encoder's
// division constants, the index hash term).  Host-only definitions
// (error text, layout and table preparation) live in gaans_host.cpp, which
// also builds without the HIP toolchain (for the sanitizer runs).
#ifndef GAANS_COMMON_H
#define GAANS_COMMON_H

#include <stdint.h>

#include "gaans_w64.h"

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define GAANS_HD __host__ __device__ __forceinline__
#define GAANS_HDI __host__ __device__ inline
#else
#define GAANS_HD inline
#define GAANS_HDI inline
#endif

namespace gaans {

constexpr int kLanes = 64;
constexpr uint32_t kStateLow = 1u << 16;  // rANS L
constexpr uint32_t kMagic = 0x31574147u;  // "GAW1"
constexpr uint32_t kVersion = 5u;
constexpr int kMaxSegments = 256;  // segments per chunk
constexpr uint32_t kParams = 0x00041040u;  // lanes 64 | precision 16 << 8 | bypass 4 << 16
constexpr int kFixedWords = 16;
constexpr uint32_t kTabMagic = 0x38425447u;  // "GTB8"
constexpr int kLutBits = 8;
constexpr int kLutSize = 1 << kLutBits;
constexpr int kSubBits = 4;                 // a sub-block: 16 entries of 16 or 1 values
constexpr int kSubSize = 1 << kSubBits;
constexpr int kSubBytes = 8 * kSubSize;
// wide decode lookups: 2048 buckets of 32 values per table, a dense bucket
// (two or more symbols starting after its first value) resolved by one
// sub-block of 16 two-value ranges (never dense); built for blobs of at most
// kWideMaxTables tables (16 KB of lookups per table)
constexpr int kWideBits = 11;
constexpr int kWideSize = 1 << kWideBits;
constexpr int kWideSubShift = 16 - kWideBits - kSubBits;  // a sub-range: 2 values
constexpr int kWideMaxTables = 4096;
constexpr uint32_t kHashMul = 0x9E3779B9u;
constexpr int kMaxEscNibbles = 9;  // escape count + 8 nibbles of raw

// Records `code`'s message for gaans_last_error() (thread-local) and
// returns code.
int fail(int code, const char* fmt, ...);

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// ---- prepared table blob ---------------------------------------------------
// [TabHdr 64 B][TabMeta x M][entries: 2 x u32 per symbol][lut: u64 x 256 x M]
// [sub-blocks: u64 x 16 each]
// entry of symbol v (encoder): word 0 = start | (freq - 1) << 16;
//                              word 1 = division magic of freq (enc_magic).
// Decode lookup entries (u64) cover a range of cum values: 256 (the table's
// lookup, bucket j = [j << 8, (j << 8) + 255]), 16 (second level) or 1 (third
// level).  With s the symbol containing the range's first value:
//   at most one other symbol starts in the range:
//     low word = start(s) | (start(s + 1) - 1) << 16   (cum > that -> s + 1),
//     high word = s | (freq(s + 1) - 1) << 16
//   two or more (a dense range, 256 or 16 values wide):
//     low word = global index of a sub-block, high word = s | 0xffff << 16;
//     the sub-block's 16 entries cover the range's 16 sub-ranges (of 16 values
//     for a 256-value range, of one value for a 16-value range).
struct TabHdr {
  uint32_t magic, M, total_syms, lut_bits;
  uint32_t digest_lo, digest_hi;
  uint32_t meta_off, ent_off, lut_off;  // byte offsets
  uint32_t total_bytes;
  uint32_t max_nsym;
  uint32_t dense_off;    // byte offset of the sub-blocks
  uint32_t total_dense;  // sub-blocks over all tables
  uint32_t flags;        // kTabOffsetsSafe, kTabSearch, kTabWide
  uint32_t clut_off;    // byte offset of the search lookups (u32 per segment)
  uint32_t starts_off;  // byte offset of the symbol starts (u16 per symbol)
  uint32_t wide_off;    // byte offset of the wide lookups (u64 x kWideSize per table)
  uint32_t wdense_off;  // byte offset of the wide lookups' sub-blocks
  uint32_t wbase_off;   // byte offset of each table's first wide sub-block (u32 x (M + 1))
  uint32_t total_wide;  // wide sub-blocks over all tables
};
// every offset <= INT32_MAX - 65535: symbol index + offset cannot overflow
constexpr uint32_t kTabOffsetsSafe = 1u;
// the search lookups are filled: at most kSearchMaxSyms starts in all (the
// symbols and kStartsTablePad per table), every offset at least INT32_MIN +
// 65536 (offset - starts base cannot wrap)
constexpr uint32_t kTabSearch = 2u;
constexpr int64_t kSearchMaxSyms = 65535 - 8;
// Search lookup segments of a table: 32-value parts of its first and last
// kSearchFine 256-value buckets (entries 0-31: [0, 1024), 32-63: [64512,
// 65536), so a part's entry is (cum >> 5) & 63), then one entry per bucket
// (entry 64 + (cum >> 8); those of the 2 kSearchFine end buckets are filled
// but not read).
constexpr int kSearchFine = 4;
constexpr int kSearchFineBits = 5;
constexpr int kSearchParts = 2 * kSearchFine * (256 >> kSearchFineBits);
constexpr int kSearchEntries = kSearchParts + 256;
static_assert(kSearchParts == 64 && kSearchEntries % 4 == 0, "search segments");
constexpr int kStartsPad = 8;  // zero starts after the last symbol (sentinel, reads past it)
// Search lookups' starts: start - 1 (mod 2^16) of each symbol, table after
// table, each followed by kStartsTablePad entries 0xffff, then kStartsPad
// more (reads past the end).  A table's symbol v is at starts index
// ent_base + kStartsTablePad * table + v.
constexpr int kStartsTablePad = 3;
inline int64_t search_starts(int64_t M, int64_t total_syms) {
  return total_syms + kStartsTablePad * M + kStartsPad;
}
// the wide lookups are built (M <= kWideMaxTables)
constexpr uint32_t kTabWide = 4u;
static_assert(sizeof(TabHdr) == 80, "table header is 80 bytes");

struct TabMeta {
  uint32_t ent_base;    // first entry of the table
  uint32_t nsym;        // S - 1 symbols; the last one (nsym - 1) is the escape bin
  int32_t offset;
  uint32_t dense_base;  // first sub-block of the table
};

// Division by a wave-uniform divisor d in [1, 2^31) for numerators n < 2^31:
// q = (mulhi(n, m) + n) >> s with s = ceil(log2 d), m = floor(2^(32+s) / d) - 2^32 + 1
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up variant).
struct UDiv {
  uint32_t m, s;
};

GAANS_HDI uint32_t mulhi32(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umulhi(a, b);
#else
  return (uint32_t)(((uint64_t)a * b) >> 32);
#endif
}

GAANS_HDI uint32_t udiv(uint32_t n, UDiv d) {
  return (mulhi32(n, d.m) + n) >> d.s;
}

// Encoder division x / f for f in [1, 65536] and x < f 2^16 (the coder's
// state after renormalisation): l = ceil(log2 f) (enc_shift), M = 2^32 + m
// with m = floor(2^32 (2^l - f) / f) + 1 (enc_magic; 0 for f = 1), then
// q = floor(x M / 2^(32 + l)) (Granlund & Montgomery, PLDI 1994, theorem
// 4.2: 2^(32+l) < M f <= 2^(32+l) + 2^l, exact for every x < 2^32).  x M =
// x m + x 2^32, so its high word is mulhi(x, m) + x, which for x < f 2^16
// stays below 2^32 (x M < 2^(48+l) <= 2^64): two ops and a shift, and f = 1
// (m = 0, l = 0) needs no special case.
GAANS_HDI uint32_t enc_shift(uint32_t f) {  // l = ceil(log2 f): bits of f - 1
#if defined(__HIP_DEVICE_COMPILE__)
  return 32u - (uint32_t)__clz((int)(f - 1u));
#else
  uint32_t l = 0;
  while (((uint64_t)1 << l) < f) ++l;
  return l;
#endif
}

GAANS_HDI uint32_t enc_div(uint32_t x, uint32_t m, uint32_t l) {
  return (mulhi32(x, m) + x) >> (l & 31u);
}

// Index hash term of chunk position p with table tb: MurmurHash3's 32-bit
// finaliser (Appleby) of p * 0x9E3779B9 + tb + 1; a chunk's hash is the sum
// of its terms mod 2^32 (a bijective finaliser, so positions that trade
// tables change the sum except with probability about 2^-32).
GAANS_HD uint32_t index_term(uint32_t p, uint32_t tb) {
  uint32_t h = p * kHashMul + tb + 1u;
  h ^= h >> 16;
  h *= 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  h ^= h >> 16;
  return h;
}


// Host side of udiv (make_udiv) and of enc_div (enc_magic: m above).
UDiv make_udiv(uint32_t d);
uint32_t enc_magic(uint32_t f);

// Chunks and coding units.  Chunk k of a row covers the positions
// [k chunk_len, min((k + 1) chunk_len, N)) (P channels), Tc steps of 64
// positions; it is split into S interleaved segments, segment s holding the
// steps s, s + S, s + 2 S, ... (so every segment sees the chunk's channels in
// equal shares).  A segment is a coding unit, coded independently (own
// states, stream and escape section) by its own workgroup:
// unit g = (b K + k) S + s, U = B K S units.
struct Layout {
  int64_t B, N, C, P, S, HW, K, chunk_len, U, seg_cap, header_bytes, max_payload, cap_words,
      ws_bytes;
  int64_t o_words_cnt, o_status, o_hash, o_end, o_info, o_states, o_words, o_esc, o_esc_raw,
      o_look;
};
int make_layout(int64_t B, int64_t N, int64_t C, int64_t P, int64_t S, Layout* L);

// Coding unit g = (b K + k) S + s (see Layout): row offset b N, first
// position in the row, symbol count, and chunk k.
GAANS_HD void unit_range(int64_t g, int32_t K, int32_t S, int64_t N,
                                                    int32_t chunk_len, int64_t& row,
                                                    int32_t& start, int& len, int& k) {
  const int64_t per_row = (int64_t)K * S;
  const int64_t b = g / per_row;
  const int32_t r = (int32_t)(g - b * per_row);
  k = r / S;
  const int32_t s = r - k * S;
  row = b * N;
  const int32_t cs = k * chunk_len;
  const int32_t ce = (int64_t)cs + chunk_len < N ? cs + chunk_len : (int32_t)N;
  const int32_t tc = (ce - cs + kLanes - 1) / kLanes;
  // the unit's steps s, s + S, ..., s + S (T - 1) of the chunk; only the
  // chunk's last step (unit (tc - 1) mod S) may be partial
  const int32_t T = (tc - s + S - 1) / S;
  const int32_t last = s + S * (T - 1);
  start = cs + kLanes * s;
  len = kLanes * T - (last == tc - 1 ? kLanes * tc - (ce - cs) : 0);
}

// Row position of unit position p (lane p mod 64 of the unit's step p / 64)
// in a unit that starts at row position start, S segments per chunk.
GAANS_HD int32_t unit_pos(int32_t start, int32_t S, int32_t p) {
  return start + p + kLanes * (S - 1) * (p >> 6);
}

GAANS_HD int unit_len(int64_t g, int32_t K, int32_t S, int64_t N,
                                                 int32_t chunk_len) {
  int64_t row;
  int32_t start;
  int len, k;
  unit_range(g, K, S, N, chunk_len, row, start, len, k);
  return len;
}

// Tables of one chunk: a staged range [t_lo, t_lo + nt) in LDS, the rest in
// global memory.

// Blob sections: [header][metadata][entries][lookups][sub-blocks][search
// lookups][starts][wide lookups][wide sub-blocks][wide bases]; the offsets
// follow from the counts (the wide sections are empty unless `wide`).
struct BlobLayout {
  int64_t ent_off, lut_off, dense_off, clut_off, starts_off, wide_off, wdense_off, wbase_off,
      end;
};

inline BlobLayout blob_layout(int64_t M, int64_t total_syms, int64_t total_blocks, bool wide,
                              int64_t total_wide) {
  BlobLayout L;
  L.ent_off = align_up((int64_t)sizeof(TabHdr) + (int64_t)sizeof(TabMeta) * M, 8);
  L.lut_off = align_up(L.ent_off + 8 * total_syms, 16);
  L.dense_off = L.lut_off + 8ll * kLutSize * M;
  L.clut_off = L.dense_off + (int64_t)kSubBytes * total_blocks;
  L.starts_off = L.clut_off + 4ll * kSearchEntries * M;
  L.wide_off = L.starts_off + align_up(2 * search_starts(M, total_syms), 16);
  L.wdense_off = L.wide_off + (wide ? 8ll * kWideSize * M : 0);
  L.wbase_off = L.wdense_off + (wide ? (int64_t)kSubBytes * total_wide : 0);
  L.end = L.wbase_off + (wide ? align_up(4 * (M + 1), 16) : 0);
  return L;
}

}  // namespace gaans

#endif  // GAANS_COMMON_H
