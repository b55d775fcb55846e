// Host-only part of the GA-ANS library: error text, the chunk / coding-unit
// layout, the segment choice, preparation of the CDF table blob (validation,
// encoder entries, decode lookups and sub-blocks, search lookups, digest) and
// the host self test.  It uses no HIP API, so it also builds with g++ alone
// (the sanitizer tests build it that way); gaans_w64.hip holds the kernels
// and their launch code.
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>

#include "gaans_common.h"
#include "gaans_w64.h"

namespace gaans {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

UDiv make_udiv(uint32_t d) {
  uint32_t s = 0;
  while (((uint64_t)1 << s) < d) ++s;
  uint64_t m = (((uint64_t)1 << (32 + s)) / d) - ((uint64_t)1 << 32) + 1;
  return UDiv{(uint32_t)m, s};
}

uint32_t enc_magic(uint32_t f) {
  if (f < 2) return 0;
  uint32_t l = 0;
  while (((uint64_t)1 << l) < f) ++l;
  return (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - f)) / f + 1);
}

int make_layout(int64_t B, int64_t N, int64_t C, int64_t P, int64_t S, Layout* L) {
  if (B < 1 || N < 1 || C < 1 || P < 1)
    return fail(GAANS_EINVAL, "B, N, C and P must be >= 1 (got %lld, %lld, %lld, %lld)",
                (long long)B, (long long)N, (long long)C, (long long)P);
  if (N % C != 0)
    return fail(GAANS_EINVAL, "symbols per row N=%lld is not a multiple of channels C=%lld",
                (long long)N, (long long)C);
  if (P > C) return fail(GAANS_EINVAL, "P=%lld exceeds channels C=%lld", (long long)P, (long long)C);
  if (N >= ((int64_t)1 << 31) || B >= ((int64_t)1 << 31))
    return fail(GAANS_EINVAL, "B and N must be < 2^31");
  L->B = B; L->N = N; L->C = C; L->P = P; L->S = S;
  L->HW = N / C;
  L->K = (C + P - 1) / P;
  L->chunk_len = P * L->HW;
  // every segment holds at least one step: S <= the steps of the last
  // (shortest) chunk of a row
  const int64_t t_last = (N - (L->K - 1) * L->chunk_len + kLanes - 1) / kLanes;
  if (S < 1 || S > kMaxSegments || S > t_last)
    return fail(GAANS_EINVAL,
                "segments per chunk must be in [1, %lld] for this shape (got %lld)",
                (long long)(t_last < kMaxSegments ? t_last : kMaxSegments), (long long)S);
  L->U = B * L->K * S;
  // the encoder's completion counter holds the unit count in 24 bits
  if (L->U >= ((int64_t)1 << 24))
    return fail(GAANS_EINVAL, "too many coding units (%lld, at most 2^24 - 1)", (long long)L->U);
  if ((int64_t)kMaxEscNibbles * L->chunk_len + 8 >= ((int64_t)1 << 31))
    return fail(GAANS_EINVAL, "chunk of %lld symbols is too large", (long long)L->chunk_len);
  // the longest unit: ceil(Tc / S) steps of the longest chunk
  const int64_t tc = (L->chunk_len + kLanes - 1) / kLanes;
  L->seg_cap = std::min<int64_t>(L->chunk_len, kLanes * ((tc + S - 1) / S));
  L->header_bytes = align_up(4 * kFixedWords + 8 * L->U, 16);
  // per symbol at most one stream word and 9 escape nibbles; per unit the
  // states, a pad word and a partly used escape word
  L->max_payload = L->header_bytes + B * N * 7 + L->U * (4 * kLanes + 8);
  // ... and the payload body in 36 bits of u32 words
  if (L->max_payload >= ((int64_t)1 << 38))
    return fail(GAANS_EINVAL, "shape too large (worst-case payload of %lld bytes)",
                (long long)L->max_payload);
  // whole 16-byte chunks, so that every unit's staging slot is 16-byte
  // aligned (the fused encode copies it to LDS in 16-byte pieces)
  L->cap_words = align_up(L->seg_cap + 2, 8);
  int64_t o = 0;
  // the fused encode's look-back words first: their place does not depend
  // on the shape, so one zeroing serves every shape that uses the workspace
  L->o_look = o;      o = align_up(o + 8 * L->U, 256);
  L->o_words_cnt = o; o = align_up(o + 4 * L->U, 256);
  L->o_status = o;    o = align_up(o + 4 * L->U, 256);
  L->o_hash = o;      o = align_up(o + 4 * L->U, 256);
  L->o_end = o;       o = align_up(o + 4 * L->U, 256);
  L->o_info = o;      o = align_up(o + 32, 256);
  L->o_states = o;    o = align_up(o + 4 * kLanes * L->U, 256);
  L->o_words = o;     o = align_up(o + 2 * L->cap_words * L->U, 256);
  L->o_esc = o;       o = align_up(o + 8 * L->U, 256);
  L->o_esc_raw = o;   o = align_up(o + 4 * L->seg_cap * L->U, 256);
  L->ws_bytes = o;
  return GAANS_OK;
}

}  // namespace gaans

namespace {

using namespace gaans;

uint64_t fnv_u32(uint64_t h, uint32_t v) {
  for (int i = 0; i < 4; ++i) {
    h ^= (v >> (8 * i)) & 0xffu;
    h *= 0x100000001b3ull;
  }
  return h;
}

int64_t tables_size(int32_t M, int64_t total_syms, int64_t total_blocks, int64_t total_wide) {
  return blob_layout(M, total_syms, total_blocks, M <= kWideMaxTables, total_wide).end;
}

// Search lookups of one table, whose symbol v has starts index pbase + v
// (see kStartsTablePad): starts[pbase + v] = cdf[v] - 1 mod 2^16 (0xffff for
// symbol 0), then kStartsTablePad entries 0xffff, so that "start - 1 < cum"
// holds for the symbols that start at or below cum and for no padding; and
// one u32 per segment of the cum range (kSearchEntries: 32-value parts of
// the first and the last kSearchFine buckets, then every 256-value bucket).
// With u = cum & 255, a fitted segment's entry m (bits 0-7), 0 (bits 8-15),
// G (bits 16-31) puts c = G + ((u * m) >> 8) at most three starts
// indexes below the symbol that contains cum and never above it, and never
// below the table's first symbol, so one read of starts c .. c + 4 resolves
// it.  A bucket's line starts at its first value's symbol g (G = g, the
// smallest m that meets both bounds); a part's may start anywhere (the first
// m, in increasing order, for which some G >= 0 meets them; G is then the
// largest).  A segment that no line fits gets G = g, m = 0 and in bits
// 8-15 n, the symbols that start inside it after g (4 to 255: m = 0 fits
// the segments with n <= 3); its lookup searches g .. g + n.
void build_search(const int32_t* c, uint32_t nsym, uint32_t pbase, uint32_t* clut,
                  uint16_t* starts) {
  for (uint32_t v = 0; v < nsym; ++v) starts[pbase + v] = (uint16_t)(c[v] - 1);
  for (int i = 0; i < kStartsTablePad; ++i) starts[pbase + nsym + (uint32_t)i] = 0xffffu;
  constexpr uint32_t kFineN = (uint32_t)kSearchParts / 2;  // parts at each end
  for (uint32_t j = 0; j < (uint32_t)kSearchEntries; ++j) {
    const bool part = j < (uint32_t)kSearchParts;
    const uint32_t w = part ? 1u << kSearchFineBits : 256u;
    const uint32_t lo = part ? (j < kFineN ? j * w : 65536u - kSearchFine * 256u + (j - kFineN) * w)
                             : (j - (uint32_t)kSearchParts) * 256u;
    // the symbol containing lo (c[0] = 0 <= lo), the symbol at each value
    const uint32_t s0 = (uint32_t)(std::upper_bound(c, c + nsym, (int32_t)lo) - c) - 1u;
    uint32_t sym[256];
    uint32_t n = 0;
    for (uint32_t o = 0; o < w; ++o) {
      while (s0 + n + 1 < nsym && (uint32_t)c[s0 + n + 1] <= lo + o) ++n;
      sym[o] = pbase + s0 + n;
    }
    const uint32_t u0 = lo & 255u, g = pbase + s0;
    uint32_t entry = (g << 16) | (n << 8);  // the search entry unless a line fits
    if (!part) {
      // c = g + floor(u m / 256): m >= ceil((d - 3) 256 / u), m <= ((d + 1) 256 - 1) / u
      uint32_t m_lo = 0, m_hi = 255;
      for (uint32_t o = 1; o < w; ++o) {
        const uint32_t d = sym[o] - g;
        if (d > 3u) {
          const uint32_t need = ((d - 3u) * 256u + o - 1u) / o;
          m_lo = need > m_lo ? need : m_lo;
        }
        const uint32_t cap = ((d + 1u) * 256u - 1u) / o;
        m_hi = cap < m_hi ? cap : m_hi;
      }
      if (m_lo <= m_hi) entry = (g << 16) | m_lo;
    } else {
      for (uint32_t m = 0; m < 256u; ++m) {
        int64_t g_lo = (int64_t)pbase - (int64_t)((u0 * m) >> 8), g_hi = INT64_MAX;
        g_lo = g_lo > 0 ? g_lo : 0;
        for (uint32_t o = 0; o < w; ++o) {
          const int64_t r = (int64_t)sym[o] - (int64_t)(((u0 + o) * m) >> 8);
          g_lo = r - 3 > g_lo ? r - 3 : g_lo;
          g_hi = r < g_hi ? r : g_hi;
        }
        if (g_lo <= g_hi) {
          entry = ((uint32_t)g_hi << 16) | m;
          break;
        }
      }
    }
    clut[j] = entry;
  }
}

// Decode lookup entry of the cum range [lo, lo + width) of a CDF with nsym
// symbols (cdf c) into *out; false when the range is dense (two or more
// symbols start after lo).  s is advanced to the symbol containing lo.
bool lookup_entry(const int32_t* c, uint32_t nsym, uint32_t lo, uint32_t width, uint32_t& s,
                  uint64_t* out) {
  while (s + 1 < nsym && (uint32_t)c[s + 1] <= lo) ++s;
  uint32_t e = s;
  while (e + 1 < nsym && (uint32_t)c[e + 1] <= lo + width - 1) ++e;
  if (e - s >= 2) return false;
  const uint32_t next = s + 1 < nsym ? (uint32_t)(c[s + 2] - c[s + 1] - 1) : 0u;
  const uint32_t lo_word = (uint32_t)c[s] | ((uint32_t)(c[s + 1] - 1) << 16);
  *out = (uint64_t)lo_word | ((uint64_t)(s | (next << 16)) << 32);
  return true;
}

// Sub-blocks of one CDF (S entries): one per dense 256-value bucket, one per
// dense 16-value sub-range of those.  Fills them when blocks is non-NULL
// (global indices from `first`) and the table's 256 lookup entries in lut.
int32_t build_lookup(const int32_t* c, int32_t S, uint64_t* lut, uint64_t* blocks,
                     uint32_t first) {
  const uint32_t nsym = (uint32_t)(S - 1);
  int32_t n = 0;
  uint32_t s = 0;
  for (int j = 0; j < kLutSize; ++j) {
    const uint32_t lo = (uint32_t)j << (16 - kLutBits);
    uint64_t e;
    if (lookup_entry(c, nsym, lo, 1u << (16 - kLutBits), s, &e)) {
      if (lut) lut[j] = e;
      continue;
    }
    const uint32_t b2 = (uint32_t)n++;
    if (lut) lut[j] = (uint64_t)(first + b2) | ((uint64_t)(s | (0xffffu << 16)) << 32);
    uint32_t s2 = s;
    for (int i = 0; i < kSubSize; ++i) {
      const uint32_t lo2 = lo + ((uint32_t)i << kSubBits);
      uint64_t e2;
      if (lookup_entry(c, nsym, lo2, kSubSize, s2, &e2)) {
        if (blocks) blocks[(size_t)b2 * kSubSize + i] = e2;
        continue;
      }
      const uint32_t b3 = (uint32_t)n++;
      if (blocks)
        blocks[(size_t)b2 * kSubSize + i] =
            (uint64_t)(first + b3) | ((uint64_t)(s2 | (0xffffu << 16)) << 32);
      uint32_t s3 = s2;
      for (int v = 0; v < kSubSize; ++v) {
        uint64_t e3 = 0;
        lookup_entry(c, nsym, lo2 + (uint32_t)v, 1u, s3, &e3);  // one value: never dense
        if (blocks) blocks[(size_t)b3 * kSubSize + v] = e3;
      }
    }
  }
  return n;
}

// Wide lookups of one CDF (S entries): kWideSize entries of 32-value
// buckets in lut and, for each dense bucket, a sub-block of 16 two-value
// ranges (global indices from `first`; filled when blocks is non-NULL).
// Returns the table's sub-blocks.
int32_t build_wide(const int32_t* c, int32_t S, uint64_t* lut, uint64_t* blocks,
                   uint32_t first) {
  const uint32_t nsym = (uint32_t)(S - 1);
  const uint32_t width = 1u << (16 - kWideBits);
  const uint32_t sub_width = 1u << kWideSubShift;
  int32_t n = 0;
  uint32_t s = 0;
  for (int j = 0; j < kWideSize; ++j) {
    const uint32_t lo = (uint32_t)j * width;
    uint64_t e;
    if (lookup_entry(c, nsym, lo, width, s, &e)) {
      if (lut) lut[j] = e;
      continue;
    }
    const uint32_t b2 = (uint32_t)n++;
    if (lut) lut[j] = (uint64_t)(first + b2) | ((uint64_t)(s | (0xffffu << 16)) << 32);
    uint32_t s2 = s;
    for (int i = 0; i < kSubSize; ++i) {
      uint64_t e2 = 0;
      // a two-value range holds at most one start after its first value
      lookup_entry(c, nsym, lo + (uint32_t)i * sub_width, sub_width, s2, &e2);
      if (blocks) blocks[(size_t)b2 * kSubSize + i] = e2;
    }
  }
  return n;
}

}  // namespace

using namespace gaans;

extern "C" {

int gaans_abi_version(void) { return GAANS_ABI_VERSION; }

const char* gaans_last_error(void) { return g_last_error.c_str(); }

int gaans_get_layout(int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                     gaans_layout* out) {
  if (!out) return fail(GAANS_EINVAL, "layout pointer is NULL");
  Layout L;
  int rc = make_layout(B, N, C, P, segments, &L);
  if (rc) return rc;
  out->B = L.B; out->N = L.N; out->C = L.C; out->P = L.P; out->S = L.S;
  out->HW = L.HW; out->K = L.K; out->chunk_len = L.chunk_len; out->U = L.U;
  out->header_bytes = L.header_bytes;
  out->max_payload_bytes = L.max_payload;
  out->cap_words = L.cap_words;
  out->workspace_bytes = L.ws_bytes;
  out->ws_chunk_words = L.o_words_cnt;
  out->ws_chunk_status = L.o_status;
  out->ws_index_hash = L.o_hash;
  out->ws_end_off = L.o_end;
  out->ws_info = L.o_info;
  out->ws_states = L.o_states;
  out->ws_words = L.o_words;
  out->ws_esc = L.o_esc;
  out->ws_esc_raw = L.o_esc_raw;
  out->ws_look = L.o_look;
  return GAANS_OK;
}

int gaans_choose_segments(const gaans_tables* tables, int64_t B, int64_t N, int64_t C,
                          int64_t P, double budget, int64_t target_units, int32_t* segments) {
  if (!tables || !segments) return fail(GAANS_EINVAL, "NULL argument");
  Layout L;
  int rc = make_layout(B, N, C, P, 1, &L);
  if (rc) return rc;
  if (!(budget >= 0.0) || !(tables->mean_bits >= 0.0f))
    return fail(GAANS_EINVAL, "budget and the tables' mean_bits must be non-negative numbers");
  // the most segments the shape allows: one step each in the shortest chunk
  const int64_t t_last = (N - (L.K - 1) * L.chunk_len + kLanes - 1) / kLanes;
  int64_t s = std::min<int64_t>(kMaxSegments, t_last);
  // enough units to fill target_units workgroups, no more
  if (target_units > 0) s = std::min<int64_t>(s, (target_units + L.U - 1) / L.U);
  // bytes an added unit costs, against the expected bytes of a full chunk:
  // its A final states (4 A) less what its fresh initial states absorb
  // before they emit, plus a pad and a partly used escape word; measured
  // 200-203 bytes per added unit of 64 lanes on every workload of the
  // benchmark (2160x3840 P=8, 512x768 P=4, hyperprior y P=16), so 3.125 A + 4
  const int64_t len = L.chunk_len < L.N ? L.chunk_len : L.N;
  const int64_t A = len < kLanes ? len : kLanes;
  const double expected = (double)len * tables->mean_bits / 8.0 + 4.0 * (double)A;
  const double per_seg = 3.125 * (double)A + 4.0;
  s = std::min<int64_t>(s, 1 + (int64_t)(budget * expected / per_seg));
  *segments = (int32_t)std::max<int64_t>(s, 1);
  return GAANS_OK;
}

int gaans_tables_bytes(const int32_t* cdfs, const int32_t* cdf_sizes, int32_t M, int32_t Lmax,
                       int64_t* bytes) {
  if (!cdfs || !cdf_sizes || !bytes) return fail(GAANS_EINVAL, "NULL argument");
  // decode records carry a table number and an escape symbol in 16 bits each
  if (M < 1 || M > 65536 || Lmax < 2)
    return fail(GAANS_EINVAL, "need 1 <= M <= 65536 tables of Lmax >= 2 entries (got M=%d)", M);
  int64_t total = 0, dense = 0, wide = 0;
  for (int32_t t = 0; t < M; ++t) {
    const int32_t S = cdf_sizes[t];
    if (S < 2 || S > Lmax || S > 65536)
      return fail(GAANS_ETABLE, "table %d: cdf size %d outside [2, %d]", t, S,
                  Lmax < 65536 ? Lmax : 65536);
    // a valid CDF before the lookups are sized (their construction assumes
    // one: 0 = c[0] < c[1] < ... < c[S-1] = 65536)
    const int32_t* c = cdfs + (int64_t)t * Lmax;
    if (c[0] != 0 || c[S - 1] != 65536)
      return fail(GAANS_ETABLE, "table %d: CDF must start at 0 and end at 65536", t);
    for (int32_t j = 0; j + 1 < S; ++j)
      if (c[j + 1] <= c[j])
        return fail(GAANS_ETABLE, "table %d: CDF is not strictly increasing at entry %d", t, j);
    total += S - 1;
    dense += build_lookup(c, S, nullptr, nullptr, 0u);
    if (M <= kWideMaxTables) wide += build_wide(c, S, nullptr, nullptr, 0u);
  }
  *bytes = tables_size(M, total, dense, wide);
  if (*bytes > 0xffffffffll) return fail(GAANS_ETABLE, "tables exceed 4 GiB");
  return GAANS_OK;
}

int gaans_tables_prepare(const int32_t* cdfs, const int32_t* cdf_sizes, const int32_t* offsets,
                         int32_t M, int32_t Lmax, void* out, int64_t out_bytes,
                         gaans_tables* desc) {
  if (!cdfs || !offsets || !out || !desc) return fail(GAANS_EINVAL, "NULL argument");
  int64_t need = 0;
  int rc = gaans_tables_bytes(cdfs, cdf_sizes, M, Lmax, &need);
  if (rc) return rc;
  if (out_bytes < need)
    return fail(GAANS_EINVAL, "table buffer too small (%lld < %lld)", (long long)out_bytes,
                (long long)need);
  uint8_t* o = static_cast<uint8_t*>(out);
  memset(o, 0, (size_t)need);
  TabHdr* h = reinterpret_cast<TabHdr*>(o);
  TabMeta* meta = reinterpret_cast<TabMeta*>(o + sizeof(TabHdr));
  const int64_t ent_off = align_up(sizeof(TabHdr) + (int64_t)sizeof(TabMeta) * M, 8);
  uint32_t* ent = reinterpret_cast<uint32_t*>(o + ent_off);
  const bool wide = M <= kWideMaxTables;
  int64_t total = 0, total_dense = 0, total_wide = 0;
  uint32_t max_nsym = 0;
  int32_t max_dense = 0, max_wide = 0;
  for (int32_t t = 0; t < M; ++t) {
    total += cdf_sizes[t] - 1;
    if ((uint32_t)(cdf_sizes[t] - 1) > max_nsym) max_nsym = (uint32_t)(cdf_sizes[t] - 1);
    const int32_t nd = build_lookup(cdfs + (int64_t)t * Lmax, cdf_sizes[t], nullptr, nullptr, 0u);
    total_dense += nd;
    if (nd > max_dense) max_dense = nd;
    if (wide) {
      const int32_t nw = build_wide(cdfs + (int64_t)t * Lmax, cdf_sizes[t], nullptr, nullptr, 0u);
      total_wide += nw;
      if (nw > max_wide) max_wide = nw;
    }
  }
  const BlobLayout BL = blob_layout(M, total, total_dense, wide, total_wide);
  uint64_t* wlut = reinterpret_cast<uint64_t*>(o + BL.wide_off);
  uint64_t* wblocks = reinterpret_cast<uint64_t*>(o + BL.wdense_off);
  uint32_t* wbase = reinterpret_cast<uint32_t*>(o + BL.wbase_off);
  uint32_t wblk = 0;
  const int64_t lut_off = BL.lut_off;
  uint64_t* lut = reinterpret_cast<uint64_t*>(o + lut_off);
  const int64_t dense_off = BL.dense_off;
  uint64_t* blocks = reinterpret_cast<uint64_t*>(o + dense_off);
  uint32_t* clut = reinterpret_cast<uint32_t*>(o + BL.clut_off);
  uint16_t* starts = reinterpret_cast<uint16_t*>(o + BL.starts_off);
  // the decoder's records carry a table's first segment in 16 bits
  bool search = total + (int64_t)kStartsTablePad * M <= kSearchMaxSyms &&
                (int64_t)M * kSearchEntries <= 65536;
  for (int32_t t = 0; t < M; ++t) search &= offsets[t] >= INT32_MIN + 65536;
  uint32_t dblk = 0;
  double bits = 0.0;  // sum over tables of the table's entropy
  uint64_t dg = 0xcbf29ce484222325ull;
  dg = fnv_u32(dg, (uint32_t)M);
  uint32_t base = 0;
  for (int32_t t = 0; t < M; ++t) {
    const int32_t S = cdf_sizes[t];
    const int32_t* c = cdfs + (int64_t)t * Lmax;
    dg = fnv_u32(dg, (uint32_t)S);
    dg = fnv_u32(dg, (uint32_t)offsets[t]);
    for (int32_t j = 0; j < S; ++j) dg = fnv_u32(dg, (uint32_t)c[j]);
    const uint32_t nsym = (uint32_t)(S - 1);
    meta[t].ent_base = base;
    meta[t].nsym = nsym;
    meta[t].offset = offsets[t];
    meta[t].dense_base = dblk;
    for (uint32_t v = 0; v < nsym; ++v) {
      const uint32_t f = (uint32_t)(c[v + 1] - c[v]);
      ent[2 * (base + v)] = (uint32_t)c[v] | ((f - 1u) << 16);
      ent[2 * (base + v) + 1] = enc_magic(f);
      const double pr = f / 65536.0;
      bits -= pr * log2(pr);
    }
    dblk += (uint32_t)build_lookup(c, S, lut + (int64_t)t * kLutSize,
                                   blocks + (size_t)dblk * kSubSize, dblk);
    if (wide) {
      wbase[t] = wblk;
      wblk += (uint32_t)build_wide(c, S, wlut + (int64_t)t * kWideSize,
                                   wblocks + (size_t)wblk * kSubSize, wblk);
    }
    if (search)
      build_search(c, nsym, base + (uint32_t)(kStartsTablePad * t),
                   clut + (int64_t)t * kSearchEntries, starts);
    base += nsym;
  }
  if (wide) wbase[M] = wblk;
  h->magic = kTabMagic;
  h->M = (uint32_t)M;
  h->total_syms = (uint32_t)total;
  h->lut_bits = kLutBits;
  h->digest_lo = (uint32_t)dg;
  h->digest_hi = (uint32_t)(dg >> 32);
  h->meta_off = sizeof(TabHdr);
  h->ent_off = (uint32_t)ent_off;
  h->lut_off = (uint32_t)lut_off;
  h->total_bytes = (uint32_t)need;
  h->max_nsym = max_nsym;
  h->dense_off = (uint32_t)dense_off;
  h->total_dense = (uint32_t)total_dense;
  h->clut_off = (uint32_t)BL.clut_off;
  h->starts_off = (uint32_t)BL.starts_off;
  h->wide_off = (uint32_t)BL.wide_off;
  h->wdense_off = (uint32_t)BL.wdense_off;
  h->wbase_off = (uint32_t)BL.wbase_off;
  h->total_wide = (uint32_t)total_wide;
  bool safe = true;
  for (int32_t t = 0; t < M; ++t) safe &= offsets[t] <= INT32_MAX - 65535;
  h->flags = (safe ? kTabOffsetsSafe : 0u) | (search ? kTabSearch : 0u) | (wide ? kTabWide : 0u);
  desc->dev = nullptr;
  desc->bytes = need;
  desc->flags = (search ? GAANS_TABLES_SEARCH : 0) | (wide ? GAANS_TABLES_WIDE : 0);
  desc->M = M;
  desc->max_nsym = (int32_t)max_nsym;
  desc->total_nsym = total;
  desc->digest = dg;
  desc->max_dense = max_dense;
  desc->total_dense = total_dense;
  desc->mean_bits = (float)(bits / M);
  desc->max_wide = max_wide;
  desc->total_wide = total_wide;
  return GAANS_OK;
}

int gaans_host_selftest(void) {
  // 1. magic division by the channel length: every divisor class against exact division
  const uint32_t ds[] = {1, 2, 3, 5, 7, 16, 48, 64, 96, 100, 255, 256, 1000, 1536, 4096,
                         32640, 65535, 65536, 65537, 1000003, (1u << 30) - 1, 1u << 30,
                         (1u << 31) - 1};
  uint64_t rng = 0x243F6A8885A308D3ull;
  for (uint32_t d : ds) {
    UDiv u = make_udiv(d);
    for (int i = 0; i < 20000; ++i) {
      rng = rng * 6364136223846793005ull + 1442695040888963407ull;
      uint32_t n = (uint32_t)(rng >> 33);  // < 2^31
      if (i < 64) n = (uint32_t)i;
      if (i >= 64 && i < 128) n = (uint32_t)((uint64_t)d * (uint64_t)(i - 63) - 1u);
      if (n >= (1u << 31)) continue;
      if (udiv(n, u) != n / d) return fail(1, "udiv selftest failed d=%u n=%u", d, n);
    }
    if (udiv((1u << 31) - 1u, u) != ((1u << 31) - 1u) / d)
      return fail(1, "udiv selftest failed at n=2^31-1, d=%u", d);
  }
  // 2. encoder division: the magic of every freq in [1, 65536] at quotient
  //    boundaries and at the ends of the coded range [0, f 2^16)
  for (uint32_t f = 1; f <= 65536; ++f) {
    const uint32_t m = enc_magic(f), sh = enc_shift(f);
    const uint32_t xmax = (uint32_t)(((uint64_t)f << 16) - 1u);
    const uint32_t xs[10] = {0u, 1u, f - 1u, f, f + 1u, xmax, xmax - 1u, xmax - f,
                             xmax / 2u, (uint32_t)(((uint64_t)xmax * 2654435761u) >> 32)};
    for (int k = 0; k < 10; ++k) {
      const uint32_t x = xs[k];
      if (enc_div(x, m, sh) != x / f)
        return fail(2, "encoder division selftest failed f=%u x=%u", f, x);
    }
    for (uint32_t qq = 1; qq < 65536u; qq = qq * 3u + 1u) {
      const uint64_t lo = (uint64_t)qq * f;
      if (lo > xmax) break;
      if (enc_div((uint32_t)lo, m, sh) != qq || enc_div((uint32_t)(lo - 1u), m, sh) != qq - 1u)
        return fail(2, "encoder division selftest failed f=%u q=%u", f, qq);
    }
  }
  return GAANS_OK;
}

}  // extern "C"
