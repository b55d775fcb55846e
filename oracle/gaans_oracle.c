/*
 * CPU oracle for the GA-ANS latent-coding path.  TEST INFRASTRUCTURE ONLY
 * (see gaans_oracle.h): the product path never links or calls this file.
 *
 * ===========================================================================
 * The wave64 GA-ANS payload format, "gaans-w64-v5"
 * ===========================================================================
 * Coding parameters: 16-bit CDF precision; one 32-bit rANS state per lane,
 * x in [2^16, 2^32), initial state 2^16; 16-bit renormalisation words;
 * 4-bit escape nibbles; 64 lanes per coding unit.
 *
 * Chunking.  A batch row holds N symbols, channel-major: C channels of
 * HW = N / C positions.  P channels form one chunk, K = ceil(C / P) chunks per
 * row, chunk_len = P * HW; chunk k of row b covers positions
 * [k*chunk_len, min((k+1)*chunk_len, N)), clen of them, Tc = ceil(clen / 64)
 * steps of 64 positions (step j: chunk positions [64 j, min(64 j + 64, clen))).
 * Each chunk is split into S interleaved segments ("segments per chunk",
 * 1 <= S <= min(256, Tc of every chunk)): segment s holds the steps
 * s, s + S, s + 2 S, ... of the chunk, T = ceil((Tc - s) / S) of them, so
 * the segments of a chunk see its channels in equal shares.  A segment is a
 * coding unit: unit g = (b K + k) S + s, U = B K S units, each coded on its
 * own (own states, own word stream, own escape section), so the units of a
 * chunk can be coded in parallel.  The unit's steps, in that order, give its
 * len positions: unit position p = l + 64 t (lane l of unit step t) is chunk
 * position 64 (s + S t) + l; len = 64 T, less the lanes the chunk's last
 * step lacks when that step is the unit's last (unit s = (Tc - 1) mod S).
 * In a unit A = min(64, len) lanes are active, so the 64 lanes of one step
 * read 64 consecutive positions.
 *
 * Symbol mapping (CompressAI's escape scheme; reference
 * warp_ans_kernel_v2.cu:139-169).  With table tb = index of the position,
 * S = cdf_sizes[tb], maxv = S - 2, v = symbol - offsets[tb] (64-bit):
 *   v <  0    -> escape, raw = -2 v - 1, v = maxv
 *   v >= maxv -> escape, raw = 2 (v - maxv), v = maxv
 * raw must be < 2^32.  An escape carries n = raw ? msb(raw) / 4 + 1 : 0
 * nibbles of raw (the 4-bit bypass values of CompressAI's coder).
 *
 * rANS stream.  Every symbol is one rANS op on its lane's state with
 * start = cdf[v], freq = cdf[v+1] - cdf[v] (an escape codes its bin maxv):
 *   encode: if (x >> 16) >= freq: emit x & 0xffff, x >>= 16;
 *           x = ((x / freq) << 16) + x % freq + start
 *   decode: cum = x & 0xffff; v = the symbol with cdf[v] <= cum < cdf[v+1];
 *           x = freq * (x >> 16) + cum - start;
 *           if x < 2^16: x = (x << 16) | next word
 * The encoder walks steps t = T-1 .. 0; the words emitted in one step form
 * a group, ordered by lane index, and each group is PREPENDED to the unit's
 * word stream.  The decoder reads the stream forwards: at step t the lanes
 * that need a refill take the next words in lane order.
 *
 * Escape section.  The escapes of a unit, in position order, form a nibble
 * sequence: for each escape its count n, then its n nibbles of raw, low
 * nibble first (the same 4 + 4n bits as CompressAI's bypass coding).
 * Nibble i of the sequence is bits 4 (i & 3) of escape word i >> 2; unused
 * nibbles of the last word are zero; Q = ceil(nibbles / 4) words.
 *
 * Unit bytes: the A final states (u32 LE, lane order), the W words of the
 * rANS stream (u16 LE), one zero u16 if W + Q is odd, then the Q escape
 * words in REVERSE order (escape word 0 is the last u16 of the unit), so a
 * decoder finds every escape from the unit's end without knowing W.  After
 * decoding, every active lane's state is back at 2^16, the stream, the pad
 * and the escape words have all been consumed, and every count is the
 * minimal one of its raw value (raw ? msb(raw) / 4 + 1 : 0, hence <= 8).
 *
 * Header (u32 LE words):
 *   0 magic 0x31574147 ("GAW1")   1 version (4)     2 B    3 N
 *   4 C    5 P    6 K    7 chunk_len    8 M (table count)
 *   9 params 0x00041040 (lanes 64 | precision 16 << 8 | bypass 4 << 16)
 *   10,11 table digest (FNV-1a 64, low word first)   12 segments S
 *   13..15 zero
 *   then U u32 unit end offsets (bytes, relative to the data start),
 *   then U u32 index hashes; zero padding to a multiple of 16 bytes.
 * Data start = header bytes; unit g spans [end[g-1], end[g]) of the data.
 * Index hash of a unit: sum over its positions p (0-based in the unit) of
 *   fmix32((p * 0x9E3779B9 + tb + 1) mod 2^32), mod 2^32, with fmix32 the
 *   finaliser of MurmurHash3 (Appleby): h ^= h >> 16; h *= 0x85EBCA6B;
 *   h ^= h >> 13; h *= 0xC2B2AE35; h ^= h >> 16 (mod 2^32).  The finaliser is
 *   a bijection with full avalanche, so two positions that trade table
 *   indexes change the sum except with probability about 2^-32.
 * Table digest: FNV-1a 64 over the little-endian bytes of u32 M, then for
 * every table: u32 S, i32 offset, u32 cdf[0..S-1].
 * ===========================================================================
 */
#include "gaans_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- shared helpers ------------------------------------------------------ */

static int check_tables(const int32_t* cdfs, int32_t M, int32_t Lmax,
                        const int32_t* sizes) {
  /* table numbers and escape symbols fit 16 bits in the GPU decoder */
  if (M <= 0 || M > 65536 || Lmax < 2) return GAANS_REF_EINVAL;
  for (int32_t t = 0; t < M; ++t) {
    int32_t S = sizes[t];
    const int32_t* c = cdfs + (int64_t)t * Lmax;
    if (S < 2 || S > Lmax || S > 65536) return GAANS_REF_ETABLE;
    if (c[0] != 0 || c[S - 1] != 65536) return GAANS_REF_ETABLE;
    for (int32_t j = 0; j + 1 < S; ++j)
      if (c[j + 1] <= c[j]) return GAANS_REF_ETABLE;
  }
  return GAANS_REF_OK;
}

/* escape mapping; returns 0 ok, GAANS_REF_ERANGE if raw >= 2^32 */
static int map_symbol(int32_t sym, int32_t S, int32_t offset, int32_t* v_out,
                      int* esc, uint32_t* raw) {
  int64_t maxv = (int64_t)S - 2;
  int64_t v = (int64_t)sym - (int64_t)offset;
  int64_t r = 0;
  *esc = 0;
  if (v < 0) {
    r = -2 * v - 1;
    v = maxv;
    *esc = 1;
  } else if (v >= maxv) {
    r = 2 * (v - maxv);
    v = maxv;
    *esc = 1;
  }
  if (r >= ((int64_t)1 << 32)) return GAANS_REF_ERANGE;
  *v_out = (int32_t)v;
  *raw = (uint32_t)r;
  return GAANS_REF_OK;
}

static int nibble_count(uint32_t raw) {
  int n = 0;
  while (n < 8 && (((uint64_t)raw) >> (4 * n)) != 0) ++n;
  return n;
}

/* symbol v of table c (S entries) containing cum; plain linear scan */
static int32_t find_symbol(const int32_t* c, int32_t S, uint32_t cum) {
  int32_t v = 0;
  while (v + 1 < S - 1 && (uint32_t)c[v + 1] <= cum) ++v;
  return v;
}

static int unmap_escape(uint32_t raw, int32_t S, int32_t offset, int32_t* sym) {
  int64_t maxv = (int64_t)S - 2;
  int64_t v = (raw & 1u) ? -(int64_t)(raw >> 1) - 1 : (int64_t)(raw >> 1) + maxv;
  int64_t s = v + offset;
  if (s < INT32_MIN || s > INT32_MAX) return GAANS_REF_ECORRUPT;
  *sym = (int32_t)s;
  return GAANS_REF_OK;
}

/* ===========================================================================
 * 1. CompressAI-equivalent Rans64 (64-bit state, L = 2^31, 32-bit words)
 * ======================================================================== */

#define R64_L ((uint64_t)1 << 31)

typedef struct {
  uint32_t start, freq; /* freq may be 65536 for a one-entry alphabet */
  int bypass;           /* 1: 4-bit raw value in start */
} r64_op;

/* reference rans64_gpu.cuh:21-32 */
static void r64_put(uint64_t* r, uint32_t** pptr, uint32_t start, uint32_t freq) {
  uint64_t x = *r;
  uint64_t x_max = ((R64_L >> 16) << 32) * (uint64_t)freq;
  if (x >= x_max) {
    *pptr -= 1;
    **pptr = (uint32_t)x;
    x >>= 32;
  }
  *r = ((x / freq) << 16) + (x % freq) + start;
}

/* reference rans64_gpu.cuh:42-55 with nbits = 4 */
static void r64_put_bits(uint64_t* r, uint32_t** pptr, uint32_t val) {
  uint64_t x = *r;
  uint64_t x_max = ((R64_L >> 16) << 32) * (uint64_t)(1u << 12);
  if (x >= x_max) {
    *pptr -= 1;
    **pptr = (uint32_t)x;
    x >>= 32;
  }
  *r = (x << 4) | val;
}

int rans64_ref_encode(const int32_t* symbols, const int32_t* indexes, int64_t n,
                      const int32_t* cdfs, int32_t M, int32_t Lmax,
                      const int32_t* cdf_sizes, const int32_t* offsets,
                      uint32_t* out_words, int64_t cap_words, int64_t* n_words) {
  int rc = check_tables(cdfs, M, Lmax, cdf_sizes);
  if (rc) return rc;
  if (n < 0) return GAANS_REF_EINVAL;
  /* push ops in CompressAI order (main, count nibbles, raw nibbles j=0..) */
  int64_t cap_ops = n * 11 + 1;
  r64_op* ops = (r64_op*)malloc(sizeof(r64_op) * (size_t)cap_ops);
  if (!ops) return GAANS_REF_ESPACE;
  int64_t nops = 0;
  for (int64_t i = 0; i < n; ++i) {
    int32_t tb = indexes[i];
    if (tb < 0 || tb >= M) { free(ops); return GAANS_REF_EINDEX; }
    const int32_t* c = cdfs + (int64_t)tb * Lmax;
    int32_t v; int esc; uint32_t raw;
    rc = map_symbol(symbols[i], cdf_sizes[tb], offsets[tb], &v, &esc, &raw);
    if (rc) { free(ops); return rc; }
    ops[nops].start = (uint32_t)c[v];
    ops[nops].freq = (uint32_t)(c[v + 1] - c[v]);
    ops[nops].bypass = 0;
    ++nops;
    if (esc) {
      int nb = nibble_count(raw);
      int32_t val = nb;
      while (val >= 15) {
        ops[nops].start = 15; ops[nops].freq = 16; ops[nops].bypass = 1; ++nops;
        val -= 15;
      }
      ops[nops].start = (uint32_t)val; ops[nops].freq = 16; ops[nops].bypass = 1; ++nops;
      for (int j = 0; j < nb; ++j) {
        ops[nops].start = (raw >> (4 * j)) & 15u; ops[nops].freq = 16; ops[nops].bypass = 1;
        ++nops;
      }
    }
  }
  /* BufferedRansEncoder::flush: encode in reverse into a backward buffer */
  int64_t cap = nops * 2 + 2; /* <= 1 word per op + 2 flush words */
  uint32_t* buf = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)cap);
  if (!buf) { free(ops); return GAANS_REF_ESPACE; }
  uint32_t* end = buf + cap;
  uint32_t* ptr = end;
  uint64_t x = R64_L;
  for (int64_t k = nops - 1; k >= 0; --k) {
    if (ops[k].bypass) r64_put_bits(&x, &ptr, ops[k].start);
    else r64_put(&x, &ptr, ops[k].start, ops[k].freq);
  }
  ptr -= 2; /* rans64_gpu.cuh:34-39 */
  ptr[0] = (uint32_t)(x >> 0);
  ptr[1] = (uint32_t)(x >> 32);
  int64_t used = end - ptr;
  free(ops);
  if (used > cap_words) { free(buf); return GAANS_REF_ESPACE; }
  memcpy(out_words, ptr, sizeof(uint32_t) * (size_t)used);
  *n_words = used;
  free(buf);
  return GAANS_REF_OK;
}

typedef struct {
  uint64_t x;
  const uint32_t* p;
  const uint32_t* end;
  int bad;
} r64_dec;

static uint32_t r64_next(r64_dec* d) {
  if (d->p >= d->end) { d->bad = 1; return 0; }
  return *d->p++;
}

/* reference rans64dec_gpu.cuh:35-48 with n_bits = 4 */
static uint32_t r64_get_bits(r64_dec* d) {
  uint32_t val = (uint32_t)(d->x & 15u);
  d->x >>= 4;
  if (d->x < R64_L) d->x = (d->x << 32) | (uint64_t)r64_next(d);
  return val;
}

int rans64_ref_decode(const uint32_t* words, int64_t n_words,
                      const int32_t* indexes, int64_t n,
                      const int32_t* cdfs, int32_t M, int32_t Lmax,
                      const int32_t* cdf_sizes, const int32_t* offsets,
                      int32_t* out_symbols) {
  int rc = check_tables(cdfs, M, Lmax, cdf_sizes);
  if (rc) return rc;
  if (n == 0) return GAANS_REF_OK;
  if (n_words < 2) return GAANS_REF_ECORRUPT;
  r64_dec d;
  d.x = (uint64_t)words[0] | ((uint64_t)words[1] << 32); /* rans64dec_gpu.cuh:8-14 */
  d.p = words + 2;
  d.end = words + n_words;
  d.bad = 0;
  for (int64_t i = 0; i < n; ++i) {
    int32_t tb = indexes[i];
    if (tb < 0 || tb >= M) return GAANS_REF_EINDEX;
    const int32_t* c = cdfs + (int64_t)tb * Lmax;
    int32_t S = cdf_sizes[tb];
    uint32_t cum = (uint32_t)(d.x & 0xffffu);
    int32_t v = find_symbol(c, S, cum);
    uint32_t start = (uint32_t)c[v], freq = (uint32_t)(c[v + 1] - c[v]);
    /* rans64dec_gpu.cuh:20-32 */
    d.x = (uint64_t)freq * (d.x >> 16) + (d.x & 0xffffu) - start;
    if (d.x < R64_L) d.x = (d.x << 32) | (uint64_t)r64_next(&d);
    if (v == S - 2) {
      int32_t val = (int32_t)r64_get_bits(&d);
      int32_t nb = val;
      while (val == 15 && !d.bad) {
        val = (int32_t)r64_get_bits(&d);
        nb += val;
      }
      if (nb > 8) return GAANS_REF_ECORRUPT;
      uint32_t raw = 0;
      for (int j = 0; j < nb; ++j) raw |= r64_get_bits(&d) << (4 * j);
      rc = unmap_escape(raw, S, offsets[tb], &out_symbols[i]);
      if (rc) return rc;
    } else {
      out_symbols[i] = v + offsets[tb];
    }
    if (d.bad) return GAANS_REF_ECORRUPT;
  }
  return GAANS_REF_OK;
}

/* ===========================================================================
 * 2. wave64 GA-ANS format
 * ======================================================================== */

#define W_LANES 64
#define W_L ((uint32_t)1 << 16)
#define W_MAGIC 0x31574147u
#define W_VERSION 5u
#define W_PARAMS 0x00041040u
#define W_FIXED_WORDS 16

#define W_MAX_SEGMENTS 256

typedef struct {
  int32_t N, K, chunk_len, HW, S;
  int64_t U, header_bytes;
} w_layout;

static int w_layout_of(int32_t B, int32_t N, int32_t C, int32_t P, int32_t S, w_layout* L) {
  if (B <= 0 || N <= 0 || C <= 0 || P <= 0 || P > C || N % C != 0)
    return GAANS_REF_EINVAL;
  L->N = N;
  L->HW = N / C;
  L->K = (C + P - 1) / P;
  if ((int64_t)P * L->HW > INT32_MAX) return GAANS_REF_EINVAL;
  L->chunk_len = P * L->HW;
  /* every segment holds at least one step: S <= the steps of the last
   * (shortest) chunk of a row */
  int64_t last = (int64_t)N - (int64_t)(L->K - 1) * L->chunk_len;
  if (S < 1 || S > W_MAX_SEGMENTS || S > (last + W_LANES - 1) / W_LANES) return GAANS_REF_EINVAL;
  L->S = S;
  L->U = (int64_t)B * L->K * S;
  L->header_bytes = ((4 * W_FIXED_WORDS + 8 * L->U) + 15) / 16 * 16;
  return GAANS_REF_OK;
}

/* row b, the row position *start of unit g's first symbol and its symbol
 * count *len (see w_pos for the others) */
static void w_unit(const w_layout* L, int64_t g, int64_t* b, int64_t* start, int32_t* len) {
  int64_t per_row = (int64_t)L->K * L->S;
  *b = g / per_row;
  int64_t r = g % per_row, k = r / L->S, s = r % L->S;
  int64_t cs = k * (int64_t)L->chunk_len;
  int64_t ce = cs + L->chunk_len < L->N ? cs + L->chunk_len : L->N;
  int64_t Tc = (ce - cs + W_LANES - 1) / W_LANES;
  int64_t T = (Tc - s + L->S - 1) / L->S;  /* steps s, s + S, ..., s + S (T - 1) */
  int64_t last = s + L->S * (T - 1);      /* the unit's last step */
  *start = cs + W_LANES * s;
  *len = (int32_t)(W_LANES * T - (last == Tc - 1 ? W_LANES * Tc - (ce - cs) : 0));
}

/* row position of unit position p (lane p mod 64 of unit step p / 64) in a
 * unit that starts at row position start, S segments per chunk */
static int64_t w_pos(int64_t start, int32_t S, int64_t p) {
  return start + p + (int64_t)W_LANES * (S - 1) * (p / W_LANES);
}

int64_t gaans_ref_max_payload_bytes(int32_t B, int32_t N, int32_t C, int32_t P, int32_t S) {
  w_layout L;
  if (w_layout_of(B, N, C, P, S, &L)) return -1;
  /* per symbol at most one word and 9 escape nibbles; per unit 64 states,
   * a pad word and a partly used escape word */
  return L.header_bytes + (int64_t)B * N * 7 + L.U * (4 * W_LANES + 8);
}

/* MurmurHash3's 32-bit finaliser (Austin Appleby, public domain) */
static uint32_t fmix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  h ^= h >> 16;
  return h;
}

/* index hash term of unit position p with table tb */
static uint32_t index_term(int64_t p, int32_t tb) {
  return fmix32((uint32_t)p * 0x9E3779B9u + (uint32_t)tb + 1u);
}

uint32_t gaans_ref_index_term(int64_t p, int32_t tb) { return index_term(p, tb); }

static uint64_t fnv_bytes(uint64_t h, const void* p, size_t n) {
  const uint8_t* b = (const uint8_t*)p;
  for (size_t i = 0; i < n; ++i) {
    h ^= b[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

static uint64_t fnv_u32(uint64_t h, uint32_t v) {
  uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
  return fnv_bytes(h, b, 4);
}

uint64_t gaans_ref_table_digest(const int32_t* cdfs, int32_t M, int32_t Lmax,
                                const int32_t* cdf_sizes, const int32_t* offsets) {
  uint64_t h = 0xcbf29ce484222325ull;
  h = fnv_u32(h, (uint32_t)M);
  for (int32_t t = 0; t < M; ++t) {
    h = fnv_u32(h, (uint32_t)cdf_sizes[t]);
    h = fnv_u32(h, (uint32_t)offsets[t]);
    for (int32_t j = 0; j < cdf_sizes[t]; ++j)
      h = fnv_u32(h, (uint32_t)cdfs[(int64_t)t * Lmax + j]);
  }
  return h;
}

static void put_u32(uint8_t* p, uint32_t v) {
  p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24);
}
static uint32_t get_u32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* nibble sequence of a unit's escape section (grows as needed) */
typedef struct {
  uint8_t* nib;
  int64_t n, cap;
} w_nibs;

static int w_nibs_push(w_nibs* z, uint32_t v) {
  if (z->n == z->cap) {
    int64_t cap = z->cap ? 2 * z->cap : 64;
    uint8_t* p = (uint8_t*)realloc(z->nib, (size_t)cap);
    if (!p) return GAANS_REF_ESPACE;
    z->nib = p;
    z->cap = cap;
  }
  z->nib[z->n++] = (uint8_t)(v & 15u);
  return GAANS_REF_OK;
}

static int w_encode_unit(const int32_t* sym, const int32_t* idx_row, int64_t start,
                          int32_t len, int32_t S_seg, int32_t HW, const int32_t* cdfs, int32_t M,
                          int32_t Lmax, const int32_t* sizes, const int32_t* offsets,
                          uint8_t** out, int64_t* out_bytes, uint32_t* hash_out) {
  int A = len < W_LANES ? len : W_LANES;
  int T = (len + W_LANES - 1) / W_LANES;
  uint32_t* st_ = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(2 * (int64_t)len + 1));
  int64_t cap = (int64_t)len + 2;
  uint16_t* buf = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)cap);
  w_nibs z = {NULL, 0, 0};
  int rc = GAANS_REF_OK;
  if (!st_ || !buf) { rc = GAANS_REF_ESPACE; goto fail; }
  uint32_t* starts = st_;
  uint32_t* freqs = st_ + len;
  uint32_t hash = 0;
  /* pass 1, position order: rANS op of every symbol and the escape section */
  for (int32_t p = 0; p < len; ++p) {
    int64_t i = w_pos(start, S_seg, p);
    int32_t tb = idx_row ? idx_row[i] : (int32_t)(i / HW);
    if (tb < 0 || tb >= M) { rc = GAANS_REF_EINDEX; goto fail; }
    hash += index_term(p, tb);
    const int32_t* c = cdfs + (int64_t)tb * Lmax;
    int32_t v; int esc; uint32_t raw;
    rc = map_symbol(sym[i], sizes[tb], offsets[tb], &v, &esc, &raw);
    if (rc) goto fail;
    starts[p] = (uint32_t)c[v];
    freqs[p] = (uint32_t)(c[v + 1] - c[v]);
    if (esc) {
      int n = nibble_count(raw);
      rc = w_nibs_push(&z, (uint32_t)n);
      for (int j = 0; !rc && j < n; ++j) rc = w_nibs_push(&z, raw >> (4 * j));
      if (rc) goto fail;
    }
  }
  /* pass 2: rANS, steps last to first, one word group per step */
  uint32_t x[W_LANES];
  for (int l = 0; l < W_LANES; ++l) x[l] = W_L;
  int64_t wp = cap;
  for (int t = T - 1; t >= 0; --t) {
    int emit[W_LANES];
    int cnt = 0;
    for (int l = 0; l < W_LANES; ++l) {
      int64_t p = l + (int64_t)W_LANES * t;
      emit[l] = p < len && (x[l] >> 16) >= freqs[p];
      cnt += emit[l];
    }
    wp -= cnt;
    int64_t r = wp;
    for (int l = 0; l < W_LANES; ++l) {
      int64_t p = l + (int64_t)W_LANES * t;
      if (p >= len) continue;
      if (emit[l]) {
        buf[r++] = (uint16_t)(x[l] & 0xffffu);
        x[l] >>= 16;
      }
      uint32_t f = freqs[p];
      x[l] = ((x[l] / f) << 16) + (x[l] % f) + starts[p];
    }
  }
  {
    int64_t W = cap - wp;
    int64_t Q = (z.n + 3) / 4;
    int64_t pad = (W + Q) & 1;
    int64_t U = W + pad + Q;
    int64_t bytes = 4 * (int64_t)A + 2 * U;
    uint8_t* o = (uint8_t*)calloc((size_t)bytes, 1);
    if (!o) { rc = GAANS_REF_ESPACE; goto fail; }
    for (int l = 0; l < A; ++l) put_u32(o + 4 * l, x[l]);
    uint8_t* w16 = o + 4 * (int64_t)A;
    for (int64_t k = 0; k < W; ++k) {
      w16[2 * k] = (uint8_t)buf[wp + k];
      w16[2 * k + 1] = (uint8_t)(buf[wp + k] >> 8);
    }
    for (int64_t j = 0; j < Q; ++j) {
      uint32_t e = 0;
      for (int q = 0; q < 4 && 4 * j + q < z.n; ++q) e |= (uint32_t)z.nib[4 * j + q] << (4 * q);
      int64_t pos = U - 1 - j; /* escape word j, counted from the unit end */
      w16[2 * pos] = (uint8_t)e;
      w16[2 * pos + 1] = (uint8_t)(e >> 8);
    }
    *out = o;
    *out_bytes = bytes;
    *hash_out = hash;
  }
fail:
  free(st_);
  free(buf);
  free(z.nib);
  return rc;
}

int gaans_ref_encode(const int32_t* symbols, const int32_t* indexes,
                     int32_t B, int32_t N, int32_t C, int32_t P, int32_t S,
                     const int32_t* cdfs, int32_t M, int32_t Lmax,
                     const int32_t* cdf_sizes, const int32_t* offsets,
                     uint8_t* out, int64_t out_cap, int64_t* out_len) {
  w_layout L;
  int rc = w_layout_of(B, N, C, P, S, &L);
  if (rc) return rc;
  rc = check_tables(cdfs, M, Lmax, cdf_sizes);
  if (rc) return rc;
  uint8_t** units = (uint8_t**)calloc((size_t)L.U, sizeof(uint8_t*));
  int64_t* cbytes = (int64_t*)calloc((size_t)L.U, sizeof(int64_t));
  uint32_t* hashes = (uint32_t*)calloc((size_t)L.U, sizeof(uint32_t));
  if (!units || !cbytes || !hashes) { rc = GAANS_REF_ESPACE; goto done; }
  for (int64_t g = 0; g < L.U; ++g) {
    int64_t b, start;
    int32_t len;
    w_unit(&L, g, &b, &start, &len);
    rc = w_encode_unit(symbols + b * (int64_t)N, indexes ? indexes + b * (int64_t)N : NULL,
                       start, len, L.S, L.HW, cdfs, M, Lmax, cdf_sizes, offsets, &units[g],
                       &cbytes[g], &hashes[g]);
    if (rc) goto done;
  }
  {
    int64_t total = L.header_bytes;
    for (int64_t g = 0; g < L.U; ++g) total += cbytes[g];
    if (total - L.header_bytes > (int64_t)UINT32_MAX) { rc = GAANS_REF_ESPACE; goto done; }
    if (total > out_cap) { rc = GAANS_REF_ESPACE; goto done; }
    memset(out, 0, (size_t)L.header_bytes);
    uint64_t digest = gaans_ref_table_digest(cdfs, M, Lmax, cdf_sizes, offsets);
    uint32_t hw[W_FIXED_WORDS] = {W_MAGIC, W_VERSION, (uint32_t)B, (uint32_t)N,
                                  (uint32_t)C, (uint32_t)P, (uint32_t)L.K,
                                  (uint32_t)L.chunk_len, (uint32_t)M, W_PARAMS,
                                  (uint32_t)digest, (uint32_t)(digest >> 32), (uint32_t)S,
                                  0, 0, 0};
    for (int w = 0; w < W_FIXED_WORDS; ++w) put_u32(out + 4 * w, hw[w]);
    int64_t pos = 0;
    for (int64_t g = 0; g < L.U; ++g) {
      memcpy(out + L.header_bytes + pos, units[g], (size_t)cbytes[g]);
      pos += cbytes[g];
      put_u32(out + 4 * W_FIXED_WORDS + 4 * g, (uint32_t)pos);
      put_u32(out + 4 * W_FIXED_WORDS + 4 * L.U + 4 * g, hashes[g]);
    }
    *out_len = total;
  }
done:
  if (units)
    for (int64_t g = 0; g < L.U; ++g) free(units[g]);
  free(units);
  free(cbytes);
  free(hashes);
  return rc;
}

int gaans_ref_decode(const uint8_t* payload, int64_t payload_len,
                     const int32_t* indexes,
                     int32_t B, int32_t N, int32_t C, int32_t P, int32_t S,
                     const int32_t* cdfs, int32_t M, int32_t Lmax,
                     const int32_t* cdf_sizes, const int32_t* offsets,
                     int32_t* out_symbols) {
  w_layout L;
  int rc = w_layout_of(B, N, C, P, S, &L);
  if (rc) return rc;
  rc = check_tables(cdfs, M, Lmax, cdf_sizes);
  if (rc) return rc;
  if (payload_len < L.header_bytes) return GAANS_REF_ECORRUPT;
  uint64_t digest = gaans_ref_table_digest(cdfs, M, Lmax, cdf_sizes, offsets);
  uint32_t want[13] = {W_MAGIC, W_VERSION, (uint32_t)B, (uint32_t)N, (uint32_t)C,
                       (uint32_t)P, (uint32_t)L.K, (uint32_t)L.chunk_len, (uint32_t)M,
                       W_PARAMS, (uint32_t)digest, (uint32_t)(digest >> 32), (uint32_t)S};
  for (int w = 0; w < 10; ++w)
    if (get_u32(payload + 4 * w) != want[w]) return GAANS_REF_ECORRUPT;
  for (int w = 10; w < 12; ++w)
    if (get_u32(payload + 4 * w) != want[w]) return GAANS_REF_EMISMATCH;
  if (get_u32(payload + 4 * 12) != want[12]) return GAANS_REF_ECORRUPT;
  const uint8_t* data = payload + L.header_bytes;
  int64_t data_len = payload_len - L.header_bytes;
  uint32_t prev = 0;
  for (int64_t g = 0; g < L.U; ++g) {
    uint32_t endo = get_u32(payload + 4 * W_FIXED_WORDS + 4 * g);
    uint32_t want_hash = get_u32(payload + 4 * W_FIXED_WORDS + 4 * L.U + 4 * g);
    if (endo < prev || (int64_t)endo > data_len) return GAANS_REF_ECORRUPT;
    int64_t b, start;
    int32_t len;
    w_unit(&L, g, &b, &start, &len);
    int A = len < W_LANES ? len : W_LANES;
    int T = (len + W_LANES - 1) / W_LANES;
    int64_t nst = A;
    const uint8_t* cp = data + prev;
    int64_t cbytes = (int64_t)endo - prev;
    if (cbytes < 4 * nst || ((cbytes - 4 * nst) & 3)) return GAANS_REF_ECORRUPT;
    int64_t U = (cbytes - 4 * nst) / 2; /* u16 words: stream, pad, escapes */
    const uint8_t* wbase = cp + 4 * nst;
    int64_t rp = 0;  /* stream words read */
    int64_t eq = 0;  /* escape nibbles read */
    uint32_t x[W_LANES];
    for (int l = 0; l < W_LANES; ++l) x[l] = l < A ? get_u32(cp + 4 * (int64_t)l) : W_L;
    const int32_t* idx_row = indexes ? indexes + b * (int64_t)N : NULL;
    int32_t* orow = out_symbols + b * (int64_t)N;
    uint32_t hash = 0;
    for (int t = 0; t < T; ++t) {
      int need[W_LANES];
      for (int l = 0; l < W_LANES; ++l) {
        int64_t p = l + (int64_t)W_LANES * t;
        need[l] = 0;
        if (p >= len) continue;
        int64_t i = w_pos(start, L.S, p);
        int32_t tb = idx_row ? idx_row[i] : (int32_t)(i / L.HW);
        if (tb < 0 || tb >= M) return GAANS_REF_EINDEX;
        hash += index_term(p, tb);
        const int32_t* c = cdfs + (int64_t)tb * Lmax;
        int32_t S = cdf_sizes[tb];
        uint32_t cum = x[l] & 0xffffu;
        int32_t v = find_symbol(c, S, cum);
        uint32_t st = (uint32_t)c[v], f = (uint32_t)(c[v + 1] - c[v]);
        x[l] = f * (x[l] >> 16) + cum - st;
        need[l] = x[l] < W_L;
        if (v == S - 2) { /* escape: the next entry of the escape section */
          uint32_t nib[9];
          for (int j = 0; j < 9; ++j) nib[j] = 0;
          int n = 0;
          for (int j = 0; j <= n; ++j) {
            int64_t wi = (eq + j) >> 2; /* escape word, from the unit end */
            if (wi >= U) return GAANS_REF_ECORRUPT;
            int64_t pos = U - 1 - wi;
            uint32_t e = (uint32_t)wbase[2 * pos] | ((uint32_t)wbase[2 * pos + 1] << 8);
            nib[j] = (e >> (4 * ((eq + j) & 3))) & 15u;
            if (j == 0) {
              n = (int)nib[0];
              if (n > 8) return GAANS_REF_ECORRUPT;
            }
          }
          uint32_t raw = 0;
          for (int j = 0; j < n; ++j) raw |= nib[1 + j] << (4 * j);
          if (n != nibble_count(raw)) return GAANS_REF_ECORRUPT; /* not minimal */
          eq += 1 + n;
          rc = unmap_escape(raw, S, offsets[tb], &orow[i]);
          if (rc) return rc;
        } else {
          orow[i] = v + offsets[tb];
        }
      }
      for (int l = 0; l < W_LANES; ++l) {
        if (!need[l]) continue;
        if (rp >= U) return GAANS_REF_ECORRUPT;
        uint32_t w = (uint32_t)wbase[2 * rp] | ((uint32_t)wbase[2 * rp + 1] << 8);
        ++rp;
        x[l] = (x[l] << 16) | w;
      }
    }
    for (int l = 0; l < A; ++l)
      if (x[l] != W_L) return GAANS_REF_ECORRUPT;
    {
      int64_t Q = (eq + 3) / 4;
      int64_t pad = (rp + Q) & 1;
      if (rp + pad + Q != U) return GAANS_REF_ECORRUPT;
      if (pad && (wbase[2 * rp] | wbase[2 * rp + 1])) return GAANS_REF_ECORRUPT;
      if (eq & 3) { /* unused nibbles of the last escape word */
        int64_t pos = U - Q;
        uint32_t e = (uint32_t)wbase[2 * pos] | ((uint32_t)wbase[2 * pos + 1] << 8);
        if (e >> (4 * (eq & 3))) return GAANS_REF_ECORRUPT;
      }
    }
    if (hash != want_hash) return GAANS_REF_EMISMATCH;
    prev = endo;
  }
  if ((int64_t)prev != data_len) return GAANS_REF_ECORRUPT;
  return GAANS_REF_OK;
}

/* ---- quantize / dequantize closed forms ----------------------------------- */

void gaans_ref_quantize(const float* y, const float* medians, int32_t B, int32_t C,
                        int64_t HW, int32_t* symbols) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t p = 0; p < HW; ++p) {
        int64_t i = (b * C + c) * HW + p;
        volatile float d = y[i] - medians[c]; /* one fp32 rounding, no contraction */
        float r = rintf(d);                   /* round half to even */
        symbols[i] = (int32_t)r;              /* callers keep |r| < 2^31 */
      }
}

void gaans_ref_dequantize(const int32_t* symbols, const float* medians, int32_t B,
                          int32_t C, int64_t HW, float* y_hat) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t p = 0; p < HW; ++p) {
        int64_t i = (b * C + c) * HW + p;
        volatile float f = (float)symbols[i];
        y_hat[i] = f + medians[c];
      }
}

/* ---- GaussianConditional indexes and per-element quantize ------------------ */

/* CompressAI GaussianConditional.build_indexes (third-party; the algorithm,
 * restated): lb = max(scale, bound) elementwise with NaN propagated (torch.max),
 * index = (L - 1) - #{k < L - 1 : lb <= table[k]}, as its loop over
 * scale_table[:-1] subtracting (scales <= s) computes it.  No assumption on the
 * order of the table. */
void gaans_ref_build_indexes(const float* scales, int64_t n, const float* table, int32_t L,
                             float bound, int32_t* indexes) {
  for (int64_t i = 0; i < n; ++i) {
    float s = scales[i];
    float lb = (s != s) ? s : (s < bound ? bound : s);
    int32_t idx = L - 1;
    for (int32_t k = 0; k + 1 < L; ++k) idx -= (lb <= table[k]) ? 1 : 0;
    indexes[i] = idx;
  }
}

/* quantize(y, "symbols", means) with per-element means (NULL: none) and
 * dequantize(symbols, means) of CompressAI's EntropyModel, elementwise. */
void gaans_ref_quantize_elem(const float* y, const float* means, int64_t n, int32_t* symbols) {
  for (int64_t i = 0; i < n; ++i) {
    volatile float d = means ? y[i] - means[i] : y[i];
    symbols[i] = (int32_t)rintf(d);
  }
}

void gaans_ref_dequantize_elem(const int32_t* symbols, const float* means, int64_t n,
                               float* y_hat) {
  for (int64_t i = 0; i < n; ++i) {
    volatile float f = (float)symbols[i];
    y_hat[i] = means ? f + means[i] : f;
  }
}
