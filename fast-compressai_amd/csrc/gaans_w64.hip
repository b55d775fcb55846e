// GA-ANS wave64 latent coder for MI355X (gfx950): HIP kernels + C ABI.
//
// One wave64 codes one chunk of P latent channels.  Each lane carries one
// 32-bit rANS state (x in [2^16, 2^32), 16-bit renormalisation words, 16-bit
// CDF precision).  Lane l of a chunk owns positions l + 64 t, so a wave reads
// 64 consecutive symbols per step.  The renormalisation words a step emits
// are compacted in lane order with a wave ballot + mbcnt prefix count; the
// decoder hands refill words out in the same order.
//
// Per chunk (one 64-thread workgroup):
//  - the CDF tables of the chunk's channels (or all tables, when they fit)
//    are staged in LDS: packed (start, freq-1) entries, and for decode a
//    256-bucket lookup per table; tables that are not staged are read
//    through L1/L2;
//  - symbols / indexes / latents are prefetched kSB steps ahead in registers
//    (coalesced 256-byte loads per step);
//  - encode: emitted words go to an LDS ring that is flushed to a per-chunk
//    staging slot when it fills; decode: the word stream is prefetched from
//    HBM into registers and copied into an LDS ring ahead of use;
//  - the last workgroup of a launch (device-scope counter in a caller-owned
//    control block) scans the chunk sizes into payload offsets (encode) or
//    reduces the status words (decode) and writes them to caller memory.
//
// Payload format "gaans-w64-v1" (the bytes are defined by the CPU oracle,
// oracle/gaans_oracle.c): header, then per chunk the final lane states (u32)
// and the word stream (u16, decode order).
//
// Reference path replaced: src/fast_compressai/coders/cuda/warp_ans_kernel_v2.cu:71-306
// (encode), warp_ans_kernel.cu:178-369 and :477-544 (pack, header, decode),
// rans64_gpu.cuh / rans64dec_gpu.cuh / warp_rans.cuh (per-lane arithmetic).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "gaans_w64.h"

namespace {

constexpr int kLanes = 64;
constexpr uint32_t kStateLow = 1u << 16;   // rANS L
constexpr uint32_t kBitsEmit = 1u << 28;   // renorm bound of a 4-bit bypass op
constexpr uint32_t kMagic = 0x31574147u;   // "GAW1"
constexpr uint32_t kVersion = 1u;
constexpr uint32_t kParams = 0x00041040u;  // lanes 64 | precision 16 << 8 | bypass 4 << 16
constexpr int kFixedWords = 16;
constexpr uint32_t kTabMagic = 0x31425447u;  // "GTB1"
constexpr int kLutBits = 8;
constexpr int kLutSize = 1 << kLutBits;
constexpr uint32_t kHashMul = 0x9E3779B9u;
constexpr int kMaxOpsPerSymbol = 10;  // main + count + 8 nibbles

#ifndef GAANS_PREFETCH_STEPS
#define GAANS_PREFETCH_STEPS 8
#endif
constexpr int kSB = GAANS_PREFETCH_STEPS;  // steps per register prefetch block
constexpr int kRingWords = 4096;    // encoder LDS output ring (u16 words)
constexpr int kStreamRing = 2048;   // decoder LDS stream ring (u16 words)
constexpr int kPfU32 = 4;           // decoder stream prefetch: u32 per lane (512 words)
constexpr int kPfWords = 2 * kPfU32 * kLanes;
constexpr int64_t kEncTableBudget = 32 * 1024;
constexpr int64_t kDecTableBudget = 48 * 1024;
// control block (u32 words); encoder and decoder fields on separate 64-byte lines
constexpr int kCtrlEncDone = 0;
constexpr int kCtrlDecDone = 16;
constexpr int kCtrlDecStatus = 17;

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

int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// ---- prepared table blob ---------------------------------------------------
// [TabHdr 64 B][TabMeta x M][u32 entries: start | (freq-1) << 16][u64 lut: M x 256]
// lut entry of bucket j (cum in [j << 8, (j << 8) + 255]):
//   low word  = entry of the symbol s containing cum = j << 8
//   high word = s | next << 16: next = freq(s + 1) - 1 if the bucket holds at
//               most one symbol boundary, else 0xffff (search the entries)
struct TabHdr {
  uint32_t magic, M, total_syms, lut_bits;
  uint32_t digest_lo, digest_hi;
  uint32_t meta_off, ent_off, lut_off;  // byte offsets
  uint32_t total_bytes;
  uint32_t max_nsym;
  uint32_t reserved[5];
};
static_assert(sizeof(TabHdr) == 64, "table header is 64 bytes");

struct TabMeta {
  uint32_t ent_base;  // first entry of the table
  uint32_t nsym;      // S - 1 symbols; the last one (nsym - 1) is the escape bin
  int32_t offset;
  uint32_t lut_base;  // first lut entry of the table
};

// Division by a wave-uniform divisor d in [1, 2^31) for numerators n < 2^31:
// q = (mulhi(n, m) + n) >> s with s = ceil(log2 d), m = floor(2^(32+s) / d) - 2^32 + 1
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up variant).
struct UDiv {
  uint32_t m, s;
};

__host__ __device__ inline uint32_t udiv(uint32_t n, UDiv d) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint32_t t = __umulhi(n, d.m);
#else
  uint32_t t = (uint32_t)(((uint64_t)n * d.m) >> 32);
#endif
  return (t + n) >> d.s;
}

UDiv make_udiv(uint32_t d) {
  uint32_t s = 0;
  while (((uint64_t)1 << s) < d) ++s;
  uint64_t m = (((uint64_t)1 << (32 + s)) / d) - ((uint64_t)1 << 32) + 1;
  return UDiv{(uint32_t)m, s};
}

struct Layout {
  int64_t B, N, C, P, HW, K, chunk_len, BK, header_bytes, max_payload, cap_words, ws_bytes;
  int64_t o_words_cnt, o_status, o_hash, o_end, o_info, o_states, o_words;
};

int make_layout(int64_t B, int64_t N, int64_t C, int64_t P, Layout* L) {
  if (B < 1 || N < 1 || C < 1 || P < 1)
    return fail(GAANS_EINVAL, "B, N, C and P must be >= 1 (got %lld, %lld, %lld, %lld)",
                (long long)B, (long long)N, (long long)C, (long long)P);
  if (N % C != 0)
    return fail(GAANS_EINVAL, "symbols per row N=%lld is not a multiple of channels C=%lld",
                (long long)N, (long long)C);
  if (P > C) return fail(GAANS_EINVAL, "P=%lld exceeds channels C=%lld", (long long)P, (long long)C);
  if (N >= ((int64_t)1 << 31) || B >= ((int64_t)1 << 31))
    return fail(GAANS_EINVAL, "B and N must be < 2^31");
  L->B = B; L->N = N; L->C = C; L->P = P;
  L->HW = N / C;
  L->K = (C + P - 1) / P;
  L->chunk_len = P * L->HW;
  L->BK = B * L->K;
  if (L->BK >= ((int64_t)1 << 31)) return fail(GAANS_EINVAL, "too many chunks");
  L->header_bytes = align_up(4 * kFixedWords + 8 * L->BK, 16);
  L->max_payload = L->header_bytes + B * N * 2 * kMaxOpsPerSymbol + L->BK * (4 * kLanes + 4);
  L->cap_words = align_up((int64_t)kMaxOpsPerSymbol * L->chunk_len + 2, 2);
  int64_t o = 0;
  L->o_words_cnt = o; o = align_up(o + 4 * L->BK, 256);
  L->o_status = o;    o = align_up(o + 4 * L->BK, 256);
  L->o_hash = o;      o = align_up(o + 4 * L->BK, 256);
  L->o_end = o;       o = align_up(o + 4 * L->BK, 256);
  L->o_info = o;      o = align_up(o + 32, 256);
  L->o_states = o;    o = align_up(o + 4 * kLanes * L->BK, 256);
  L->o_words = o;     o = align_up(o + 2 * L->cap_words * L->BK, 256);
  L->ws_bytes = o;
  return GAANS_OK;
}

// ---- wave helpers -----------------------------------------------------------

__device__ __forceinline__ uint32_t lane_rank(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
  for (int off = 32; off > 0; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off, 64);
  return v;
}

__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
  for (int off = 32; off > 0; off >>= 1) v |= (uint32_t)__shfl_xor((int)v, off, 64);
  return v;
}

__device__ __forceinline__ int wave_max(int v) {
  for (int off = 32; off > 0; off >>= 1) {
    int o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ uint64_t wave_incl_scan(uint64_t v, int lane) {
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, off, 64);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(v >> 32), off, 64);
    if (lane >= off) v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// Encoder main op on a renormalised state x < freq << 16:
// x' = ((x / freq) << 16) + x % freq + start.  The quotient comes from a fp32
// reciprocal (error < 2^-6 because x / freq < 2^16) and one signed correction,
// written without branches.
__device__ __forceinline__ uint32_t enc_main(uint32_t x, uint32_t start, uint32_t freq,
                                             float rcp) {
  uint32_t q = (uint32_t)((float)x * rcp);
  uint32_t r = x - q * freq;                       // in (-freq, 2 freq) as a signed value
  const uint32_t neg = (uint32_t)((int32_t)r >> 31);  // all ones when r < 0
  q += neg;
  r += freq & neg;
  const uint32_t over = r >= freq ? 0xffffffffu : 0u;
  q -= over;
  r -= freq & over;
  return (q << 16) + r + start;
}

// Keep a wave-uniform value in a scalar register.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ bool tables_ok(const uint8_t* tables, uint32_t M, uint32_t bytes) {
  const TabHdr* h = reinterpret_cast<const TabHdr*>(tables);
  return h->magic == kTabMagic && h->M == M && h->total_bytes == bytes &&
         h->lut_bits == (uint32_t)kLutBits;
}

__device__ __forceinline__ int chunk_len_of(int64_t g, int32_t K, int32_t chunk_len, int64_t N) {
  const int64_t k = g % K;
  const int64_t s = k * chunk_len;
  const int64_t e = s + chunk_len < N ? s + chunk_len : N;
  return (int)(e - s);
}

// Tables of one chunk: a staged range [t_lo, t_lo + nt) in LDS, the rest in
// global memory.
struct Tabs {
  const TabMeta* __restrict__ gmeta;
  const uint32_t* __restrict__ gent;
  const uint64_t* __restrict__ glut;
  const uint4* lmeta;     // {ent_base (LDS-local), nsym, offset, 0}
  const uint32_t* lent;
  const uint64_t* llut;   // nt x 256
  int t_lo, nt;
};

// Stage tables [t_lo, t_hi) of the blob into LDS (one wave).
__device__ void stage_tables(Tabs& T, uint4* lmeta, uint32_t* lent, uint64_t* llut, int t_lo,
                             int t_hi, int lane) {
  T.t_lo = t_lo;
  T.nt = t_hi > t_lo ? t_hi - t_lo : 0;
  if (T.nt == 0) return;
  const uint32_t base0 = T.gmeta[t_lo].ent_base;
  const TabMeta last = T.gmeta[t_hi - 1];
  const uint32_t n_ent = last.ent_base + last.nsym - base0;
  for (int i = lane; i < T.nt; i += kLanes) {
    const TabMeta m = T.gmeta[t_lo + i];
    lmeta[i] = make_uint4(m.ent_base - base0, m.nsym, (uint32_t)m.offset, 0u);
  }
  for (uint32_t i = lane; i < n_ent; i += kLanes) lent[i] = T.gent[base0 + i];
  if (llut) {
    const uint64_t* src = T.glut + T.gmeta[t_lo].lut_base;  // tables' luts are contiguous
    for (int i = lane; i < T.nt * kLutSize; i += kLanes) llut[i] = src[i];
  }
  __syncthreads();
}

// ============================================================================
// Encoder
// ============================================================================

struct EncArgs {
  const int32_t* __restrict__ symbols;
  const float* __restrict__ y;
  const float* __restrict__ medians;
  const int32_t* __restrict__ indexes;
  const uint8_t* __restrict__ tables;
  uint32_t M, tables_bytes;
  int64_t N;
  int32_t K, P, C, chunk_len;
  UDiv div_hw;
  int32_t cap_words;
  int64_t BK, header_bytes;
  int32_t nt_cap, stage_all;
  uint32_t* __restrict__ chunk_words;
  uint32_t* __restrict__ chunk_status;
  uint32_t* __restrict__ index_hash;
  uint32_t* __restrict__ end_off;
  uint64_t* __restrict__ ws_info;
  uint32_t* __restrict__ states;
  uint16_t* __restrict__ words;
  uint32_t* __restrict__ ctrl;
  uint64_t* __restrict__ info_out;
};

// One symbol ready for the rANS update.  Inactive lanes carry the identity op
// (start 0, freq 65536: no word, x unchanged).  The escape split is finished
// only in steps where some lane escapes (enc_escape_ops).
struct EncSym {
  uint32_t st, fr;
  float rcp;
  int32_t v, maxv, sym;  // v = sym - offset (wrapped), maxv = escape bin
  bool esc, ovf;         // ovf: sym - offset does not fit int32
};

// last workgroup of an encode launch: chunk offsets + payload size + status
__device__ void encode_finish(const EncArgs& a, int lane) {
  uint64_t carry = 0;
  uint32_t st = 0;
  for (int64_t base = 0; base < a.BK; base += kLanes) {
    const int64_t g = base + lane;
    uint64_t v = 0;
    if (g < a.BK) {
      const int len = chunk_len_of(g, a.K, a.chunk_len, a.N);
      const uint32_t A = len < kLanes ? (uint32_t)len : (uint32_t)kLanes;
      const uint32_t W = __hip_atomic_load(&a.chunk_words[g], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
      v = 4ull * A + 2ull * (W + (W & 1u));
      st |= __hip_atomic_load(&a.chunk_status[g], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint64_t incl = wave_incl_scan(v, lane) + carry;
    if (g < a.BK) {
      a.end_off[g] = (uint32_t)incl;
      if (incl > 0xffffffffull) st |= GAANS_ST_SIZE;
    }
    carry = (uint64_t)__shfl((long long)incl, 63, 64);
  }
  st = wave_or(st);
  if (lane == 0) {
    const uint64_t total = (uint64_t)a.header_bytes + carry;
    a.ws_info[0] = total;
    a.ws_info[1] = st;
    if (a.info_out) {
      a.info_out[0] = total;
      a.info_out[1] = st;
    }
    __threadfence_system();
    __hip_atomic_store(&a.ctrl[kCtrlEncDone], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Branch-free mapping of one symbol: table (LDS or global), escape flag,
// entry lookup and index hash.  Reports bad indexes / non-finite latents in
// `status`.
template <bool kLatents, bool kImplicit, bool kLds>
__device__ __forceinline__ EncSym enc_map(const EncArgs& a, const Tabs& tb, int lane, int t,
                                          int len, int32_t start, int32_t in_a, int32_t in_b,
                                          float in_m, uint32_t& hash, uint32_t& status) {
  const int p = lane + kLanes * t;
  const bool act = p < len;
  int32_t tbi = kImplicit ? (int32_t)udiv((uint32_t)(start + p), a.div_hw) : in_b;
  const bool bad = act & ((uint32_t)tbi >= a.M);
  const bool ok = act & !bad;
  status |= bad ? GAANS_ST_INDEX : 0u;
  tbi = ok ? tbi : (kLds ? tb.t_lo : 0);
  hash += ok ? ((uint32_t)(tbi + 1) ^ ((uint32_t)p * kHashMul)) : 0u;
  int32_t sym;
  if (kLatents) {
    const float r = rintf(__fsub_rn(__int_as_float(in_a), in_m));
    const bool rng = !(fabsf(r) < 2147483648.0f);
    status |= (ok & rng) ? GAANS_ST_RANGE : 0u;
    sym = (int32_t)(rng ? 0.0f : r);
  } else {
    sym = in_a;
  }
  uint32_t ebase, nsym;
  int32_t offset;
  if (kLds) {
    const uint4 m = tb.lmeta[tbi - tb.t_lo];
    ebase = m.x;
    nsym = m.y;
    offset = (int32_t)m.z;
  } else {
    const TabMeta m = tb.gmeta[tbi];
    ebase = m.ent_base;
    nsym = m.nsym;
    offset = m.offset;
  }
  EncSym s;
  s.sym = sym;
  s.v = (int32_t)((uint32_t)sym - (uint32_t)offset);
  s.maxv = (int32_t)nsym - 1;
  s.ovf = ok & (((sym ^ offset) & (sym ^ s.v)) < 0);
  const bool out = ((uint32_t)s.v >= (uint32_t)s.maxv) | s.ovf;  // v < 0 or v >= maxv
  s.esc = ok & out;
  const int32_t vv = out ? s.maxv : s.v;
  const uint32_t e = kLds ? tb.lent[ebase + (uint32_t)vv] : tb.gent[ebase + (uint32_t)vv];
  s.st = ok ? (e & 0xffffu) : 0u;
  s.fr = ok ? ((e >> 16) + 1u) : 65536u;
  s.rcp = __builtin_amdgcn_rcpf((float)s.fr);
  return s;
}

// Escape details of one symbol (CompressAI's split, reference
// warp_ans_kernel_v2.cu:139-164): raw value and the op count in decode
// order (1, or nibbles + 2).  v is the wrapped 32-bit sym - offset; when it
// overflowed, the sign of sym tells the side, and raw = 2 (v - maxv) is
// exact whenever the true raw is < 2^32 (else the symbol is uncodable).
__device__ __forceinline__ void enc_escape_split(const EncSym& s, uint32_t& raw,
                                                 uint32_t& nops, uint32_t& status) {
  const uint32_t d = (uint32_t)s.v - (uint32_t)s.maxv;
  const bool lo = s.ovf ? (s.sym < 0) : (s.v < 0);
  const bool uncodable = s.ovf & (lo | (d >= 0x80000000u));
  status |= uncodable ? GAANS_ST_RANGE : 0u;
  const uint32_t r = lo ? ~((uint32_t)s.v << 1) : (d << 1);
  raw = s.esc ? r : 0u;
  const uint32_t nn = raw ? ((31u - (uint32_t)__clz((int)raw)) >> 2) + 1u : 0u;
  nops = s.esc ? nn + 2u : 1u;
}

// Encoder LDS ring: kRingWords words + one spare slot per lane, which lanes
// that emit nothing write to (so the store needs no branch).
__device__ __forceinline__ void ring_flush(uint16_t* __restrict__ wbuf,
                                           const uint16_t* ring, int wp, int fl, int lane) {
  __syncthreads();
  for (int pos = wp + lane; pos < fl; pos += kLanes) wbuf[pos] = ring[pos & (kRingWords - 1)];
}

__device__ __forceinline__ void emit_words(bool emit, uint32_t& x, uint16_t* ring,
                                           uint16_t* __restrict__ wbuf, int& wp, int& fl,
                                           int lane) {
  const uint64_t m = __ballot(emit);
  const int c = __popcll(m);
  if (fl - wp + c > kRingWords) {
    ring_flush(wbuf, ring, wp, fl, lane);
    fl = uni(wp);
  }
  wp = uni(wp - c);
  const uint32_t slot =
      emit ? ((uint32_t)(wp + (int)lane_rank(m)) & (kRingWords - 1)) : (uint32_t)(kRingWords + lane);
  ring[slot] = (uint16_t)x;
  x = emit ? (x >> 16) : x;
}

template <bool kLatents, bool kImplicit>
__global__ __launch_bounds__(64) void k_encode(EncArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* ring = reinterpret_cast<uint16_t*>(smem);
  constexpr int kRingBytes = 2 * (kRingWords + kLanes);
  uint4* lmeta = reinterpret_cast<uint4*>(smem + kRingBytes);
  uint32_t* lent = reinterpret_cast<uint32_t*>(smem + kRingBytes + 16 * a.nt_cap);

  const int g = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t b = g / a.K;
  const int k = g - (int)(b * a.K);
  const int64_t row = b * a.N;
  const int32_t start = k * a.chunk_len;
  const int32_t endp = (int64_t)start + a.chunk_len < a.N ? start + a.chunk_len : (int32_t)a.N;
  const int len = endp - start;
  const int T = (len + kLanes - 1) / kLanes;
  const int A = len < kLanes ? len : kLanes;
  uint16_t* __restrict__ wbuf = a.words + (int64_t)g * a.cap_words;
  int wp = a.cap_words;  // wave-uniform write cursor (backwards)
  int fl = a.cap_words;  // words at [fl, cap) are already in wbuf
  uint32_t x = kStateLow;
  uint32_t hash = 0, status = 0;

  if (tables_ok(a.tables, a.M, a.tables_bytes)) {
    const TabHdr* th = reinterpret_cast<const TabHdr*>(a.tables);
    Tabs tb;
    tb.gmeta = reinterpret_cast<const TabMeta*>(a.tables + th->meta_off);
    tb.gent = reinterpret_cast<const uint32_t*>(a.tables + th->ent_off);
    tb.glut = nullptr;
    tb.lmeta = lmeta;
    tb.lent = lent;
    tb.llut = nullptr;
    int t_lo = 0, t_hi = 0;
    if (a.nt_cap > 0) {
      if (a.stage_all) {
        t_hi = (int)a.M;
      } else {
        t_lo = k * a.P;
        t_hi = t_lo + a.P < (int)a.M ? t_lo + a.P : (int)a.M;
      }
    }
    stage_tables(tb, lmeta, lent, nullptr, t_lo, t_hi, lane);

    int32_t ca[kSB], cb[kSB], na[kSB], nb[kSB];
    float cm[kSB], nm[kSB];
    // loads are issued for every lane (inactive lanes read the chunk's last
    // position) so that no branch separates them from their use one block later
    auto load_block = [&](int j, int32_t* ia, int32_t* ib, float* im) {
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        int p = lane + kLanes * (j * kSB + u);
        p = p < len ? p : len - 1;
        const int64_t i = row + start + p;
        if (kLatents) {
          ia[u] = __float_as_int(a.y[i]);
          im[u] = a.medians[udiv((uint32_t)(start + p), a.div_hw)];
        } else {
          ia[u] = a.symbols[i];
          im[u] = 0.0f;
        }
        ib[u] = kImplicit ? 0 : a.indexes[i];
      }
    };

    const int nblk = (T + kSB - 1) / kSB;
    if (nblk > 0) load_block(nblk - 1, ca, cb, cm);
    for (int j = nblk - 1; j >= 0; --j) {
      if (j > 0) load_block(j - 1, na, nb, nm);
      bool lds = tb.nt > 0;
      if (!kImplicit && lds) {
        bool in = true;
#pragma unroll
        for (int u = 0; u < kSB; ++u)
          in = in && (lane + kLanes * (j * kSB + u) >= len ||
                      (uint32_t)(cb[u] - tb.t_lo) < (uint32_t)tb.nt);
        lds = __ballot(!in) == 0;
      }
      EncSym s[kSB];
      if (lds) {
#pragma unroll
        for (int u = 0; u < kSB; ++u)
          s[u] = enc_map<kLatents, kImplicit, true>(a, tb, lane, j * kSB + u, len, start, ca[u],
                                                    cb[u], cm[u], hash, status);
      } else {
#pragma unroll
        for (int u = 0; u < kSB; ++u)
          s[u] = enc_map<kLatents, kImplicit, false>(a, tb, lane, j * kSB + u, len, start, ca[u],
                                                     cb[u], cm[u], hash, status);
      }
#pragma unroll
      for (int u = kSB - 1; u >= 0; --u) {
        if (j * kSB + u >= T) continue;
        const EncSym& e = s[u];
        if (__ballot(e.esc) == 0) {
          emit_words((x >> 16) >= e.fr, x, ring, wbuf, wp, fl, lane);
          x = enc_main(x, e.st, e.fr, e.rcp);
        } else {
          // escape sub-rounds, decode order d = 0 (main), 1 (count), 2.. (nibbles);
          // encoded from the last op to the first
          uint32_t raw, nops;
          enc_escape_split(e, raw, nops, status);
          const int Mt = uni(wave_max((int)nops));
          for (int d = Mt - 1; d >= 0; --d) {
            const bool part = (uint32_t)d < nops;
            const bool want = d == 0 ? (x >> 16) >= e.fr : x >= kBitsEmit;
            const uint32_t x0 = x;
            emit_words(part & want, x, ring, wbuf, wp, fl, lane);
            uint32_t xn;
            if (d == 0) {
              xn = enc_main(x, e.st, e.fr, e.rcp);
            } else {
              const uint32_t val = d == 1 ? nops - 2u : (raw >> (4 * (d - 2))) & 15u;
              xn = (x << 4) | val;
            }
            x = part ? xn : x0;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        ca[u] = na[u];
        cb[u] = nb[u];
        cm[u] = nm[u];
      }
    }
    if (fl > wp) ring_flush(wbuf, ring, wp, fl, lane);
  } else {
    status |= GAANS_ST_TABLES;
  }

  if (lane < A) a.states[(int64_t)g * kLanes + lane] = x;
  hash = wave_sum(hash);
  status = wave_or(status);
  if (lane == 0) {
    a.chunk_words[g] = (uint32_t)(a.cap_words - wp);
    a.chunk_status[g] = status;
    a.index_hash[g] = hash;
  }
  __threadfence();
  __syncthreads();
  uint32_t done = 0;
  if (lane == 0)
    done = __hip_atomic_fetch_add(&a.ctrl[kCtrlEncDone], 1u, __ATOMIC_ACQ_REL,
                                  __HIP_MEMORY_SCOPE_AGENT);
  done = (uint32_t)__shfl((int)done, 0, 64);
  if (done == (uint32_t)(a.BK - 1)) {
    __threadfence();
    encode_finish(a, lane);
  }
}

// ============================================================================
// Pack
// ============================================================================

struct PackArgs {
  const uint32_t* __restrict__ chunk_words;
  const uint32_t* __restrict__ index_hash;
  const uint32_t* __restrict__ end_off;
  const uint32_t* __restrict__ states;
  const uint16_t* __restrict__ words;
  const uint8_t* __restrict__ tables;
  uint8_t* __restrict__ out;
  int64_t out_bytes, header_bytes, cap_words, BK, N;
  uint32_t B, N32, C, P, K, chunk_len, M;
};

__global__ __launch_bounds__(256) void k_pack(PackArgs a) {
  const int64_t g = blockIdx.x;
  const int tid = threadIdx.x;
  const uint32_t beg = g ? a.end_off[g - 1] : 0u;
  const uint32_t endo = a.end_off[g];
  uint32_t* __restrict__ hdr = reinterpret_cast<uint32_t*>(a.out);
  if (tid == 0) {
    hdr[kFixedWords + g] = endo;
    hdr[kFixedWords + a.BK + g] = a.index_hash[g];
  }
  if (g == 0) {
    const TabHdr* th = reinterpret_cast<const TabHdr*>(a.tables);
    if (tid < kFixedWords) {
      uint32_t w = 0;
      switch (tid) {
        case 0: w = kMagic; break;
        case 1: w = kVersion; break;
        case 2: w = a.B; break;
        case 3: w = a.N32; break;
        case 4: w = a.C; break;
        case 5: w = a.P; break;
        case 6: w = a.K; break;
        case 7: w = a.chunk_len; break;
        case 8: w = a.M; break;
        case 9: w = kParams; break;
        case 10: w = th->digest_lo; break;
        case 11: w = th->digest_hi; break;
        default: w = 0; break;
      }
      hdr[tid] = w;
    }
    for (int64_t j = kFixedWords + 2 * a.BK + tid; j < a.header_bytes / 4; j += 256) hdr[j] = 0;
  }
  if ((int64_t)a.header_bytes + endo > a.out_bytes || endo < beg) return;
  const int len = chunk_len_of(g, (int32_t)a.K, (int32_t)a.chunk_len, a.N);
  const int A = len < kLanes ? len : kLanes;
  const int64_t W = a.chunk_words[g];
  uint8_t* dst = a.out + a.header_bytes + beg;
  uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
  for (int j = tid; j < A; j += 256) d32[j] = a.states[g * kLanes + j];
  const uint16_t* src = a.words + g * a.cap_words + (a.cap_words - W);
  uint32_t* w32 = reinterpret_cast<uint32_t*>(dst + 4 * A);
  const int64_t n32 = (W + 1) / 2;
  for (int64_t j = tid; j < n32; j += 256) {
    const uint32_t lo = src[2 * j];
    const uint32_t hi = (2 * j + 1 < W) ? src[2 * j + 1] : 0u;
    w32[j] = lo | (hi << 16);
  }
}

// ============================================================================
// Decoder
// ============================================================================

struct DecArgs {
  const uint8_t* __restrict__ payload;
  int64_t payload_bytes;
  const int32_t* __restrict__ indexes;
  const uint8_t* __restrict__ tables;
  uint32_t M, tables_bytes;
  const float* __restrict__ medians;
  int32_t* __restrict__ out_sym;
  float* __restrict__ out_y;
  int64_t N, header_bytes, BK;
  uint32_t B, C, P, K, chunk_len;
  UDiv div_hw;
  int32_t nt_cap, ne_cap, stage_all;
  uint32_t* __restrict__ ctrl;
  uint32_t* __restrict__ status_out;
};

struct DecMeta {
  uint32_t lbase, ebase, nsym;
  int32_t offset;
};

// Per-step table metadata (branch-free), index hash and index checks.
template <bool kImplicit, bool kLds>
__device__ __forceinline__ DecMeta dec_map(const DecArgs& a, const Tabs& tb, int lane, int t,
                                           int len, int32_t start, int32_t in_b,
                                           uint32_t& hash, uint32_t& status) {
  const int p = lane + kLanes * t;
  const bool act = p < len;
  int32_t tbi = kImplicit ? (int32_t)udiv((uint32_t)(start + p), a.div_hw) : in_b;
  const bool bad = act & ((uint32_t)tbi >= a.M);
  const bool ok = act & !bad;
  status |= bad ? GAANS_ST_INDEX : 0u;
  tbi = ok ? tbi : (kLds ? tb.t_lo : 0);
  hash += ok ? ((uint32_t)(tbi + 1) ^ ((uint32_t)p * kHashMul)) : 0u;
  DecMeta m;
  if (kLds) {
    const uint4 lm = tb.lmeta[tbi - tb.t_lo];
    m.ebase = lm.x;
    m.nsym = lm.y;
    m.offset = (int32_t)lm.z;
    m.lbase = (uint32_t)(tbi - tb.t_lo) * kLutSize;
  } else {
    const TabMeta gm = tb.gmeta[tbi];
    m.ebase = gm.ent_base;
    m.nsym = gm.nsym;
    m.offset = gm.offset;
    m.lbase = gm.lut_base;
  }
  return m;
}

// cum -> (symbol, start, freq).  One lookup resolves every bucket with at most
// one symbol boundary; buckets with more (the marker 0xffff) are searched.
template <bool kLds>
__device__ __forceinline__ void dec_lookup(const Tabs& tb, const DecMeta& m, uint32_t cum,
                                           bool act, uint32_t& s, uint32_t& st, uint32_t& fr) {
  const uint64_t e = kLds ? tb.llut[m.lbase + (cum >> (16 - kLutBits))]
                          : tb.glut[m.lbase + (cum >> (16 - kLutBits))];
  const uint32_t lo = (uint32_t)e, hi = (uint32_t)(e >> 32);
  const uint32_t s0 = hi & 0xffffu, nxt = hi >> 16;
  const uint32_t st0 = lo & 0xffffu, fr0 = (lo >> 16) + 1u;
  const bool up = cum >= st0 + fr0;
  s = up ? s0 + 1u : s0;
  st = up ? st0 + fr0 : st0;
  fr = up ? nxt + 1u : fr0;
  const bool slow = act & (nxt == 0xffffu);
  if (__ballot(slow)) {
    if (slow) {
      // largest s' in [s0, s0 + 256] with start(s') <= cum (a bucket spans 256 values)
      uint32_t a0 = s0, b0 = s0 + (1u << (16 - kLutBits));
      if (b0 > m.nsym - 1u) b0 = m.nsym - 1u;
      while (a0 < b0) {
        const uint32_t mid = (a0 + b0 + 1u) >> 1;
        const uint32_t en = kLds ? tb.lent[m.ebase + mid] : tb.gent[m.ebase + mid];
        if ((en & 0xffffu) <= cum) a0 = mid;
        else b0 = mid - 1u;
      }
      const uint32_t en = kLds ? tb.lent[m.ebase + a0] : tb.gent[m.ebase + a0];
      s = a0;
      st = en & 0xffffu;
      fr = (en >> 16) + 1u;
    }
  }
}

// Word stream of one chunk: prefetched from HBM into registers (kPfWords words
// ahead) and copied into an LDS ring that refills read from.
struct Stream {
  const uint32_t* __restrict__ s32;
  const uint32_t* __restrict__ safe;  // an in-bounds word of the chunk
  int q, q32, rp, filled;
  uint32_t pf[kPfU32];
};

// Words past the stream end read the chunk's first state word instead (always
// in bounds) and are replaced by zero, so the loads need no branch.
__device__ __forceinline__ void stream_fetch(Stream& S, int lane) {
#pragma unroll
  for (int kk = 0; kk < kPfU32; ++kk) {
    const int i32 = (S.filled >> 1) + kk * kLanes + lane;
    const bool in = i32 < S.q32;
    const uint32_t w = *(in ? S.s32 + i32 : S.safe);
    S.pf[kk] = in ? w : 0u;
  }
}

__device__ __forceinline__ void stream_commit(Stream& S, uint32_t* ring32, int lane) {
#pragma unroll
  for (int kk = 0; kk < kPfU32; ++kk)
    ring32[((S.filled >> 1) + kk * kLanes + lane) & (kStreamRing / 2 - 1)] = S.pf[kk];
  S.filled = uni(S.filled + kPfWords);
  stream_fetch(S, lane);
}

__device__ __forceinline__ void dec_refill(bool need, uint32_t& x, Stream& S,
                                           const uint16_t* ring, uint32_t* ring32,
                                           uint32_t& status, int lane) {
  if (S.filled - S.rp < kLanes && S.filled < S.q) stream_commit(S, ring32, lane);
  const uint64_t m = __ballot(need);
  const int r = S.rp + (int)lane_rank(m);
  const uint32_t w = ring[r & (kStreamRing - 1)];
  status |= (need & (r >= S.q)) ? GAANS_ST_CORRUPT : 0u;
  x = need ? ((x << 16) | w) : x;
  S.rp = uni(S.rp + __popcll(m));
}

template <bool kLatents, bool kLds>
__device__ __forceinline__ void dec_step(const DecArgs& a, const Tabs& tb, const DecMeta& m,
                                         int lane, int t, int len, int64_t row, int32_t start,
                                         float med, uint32_t& x, Stream& S, const uint16_t* ring,
                                         uint32_t* ring32, uint32_t& status) {
  const int p = lane + kLanes * t;
  const bool act = p < len;
  const uint32_t cum = x & 0xffffu;
  uint32_t s, st, fr;
  dec_lookup<kLds>(tb, m, cum, act, s, st, fr);
  const uint32_t xn = __umul24(fr, x >> 16) + cum - st;
  x = act ? xn : x;
  dec_refill(act & (x < kStateLow), x, S, ring, ring32, status, lane);
  const bool esc = act & (s == m.nsym - 1u);
  int64_t value = (int64_t)s;
  if (__ballot(esc)) {
    uint32_t n = esc ? (x & 15u) : 0u;
    x = esc ? (x >> 4) : x;
    dec_refill(esc & (x < kStateLow), x, S, ring, ring32, status, lane);
    const bool badn = n > 8u;
    status |= (esc & badn) ? GAANS_ST_CORRUPT : 0u;
    n = badn ? 0u : n;
    uint32_t raw = 0;
    for (uint32_t jj = 0; jj < 8u; ++jj) {
      const bool part = esc & (jj < n);
      if (__ballot(part) == 0) break;
      raw |= part ? ((x & 15u) << (4 * jj)) : 0u;
      x = part ? (x >> 4) : x;
      dec_refill(part & (x < kStateLow), x, S, ring, ring32, status, lane);
    }
    const int64_t maxv = (int64_t)m.nsym - 1;
    const int64_t ev = (raw & 1u) ? -(int64_t)(raw >> 1) - 1 : (int64_t)(raw >> 1) + maxv;
    value = esc ? ev : value;
  }
  int64_t sv = value + m.offset;
  const bool oob = act & ((sv < INT32_MIN) | (sv > INT32_MAX));
  status |= oob ? GAANS_ST_CORRUPT : 0u;
  if (act) {
    const int64_t i = row + start + p;
    const int32_t o = oob ? 0 : (int32_t)sv;
    if (kLatents) a.out_y[i] = __fadd_rn((float)o, med);
    else a.out_sym[i] = o;
  }
}

template <bool kLatents, bool kImplicit>
__global__ __launch_bounds__(64) void k_decode(DecArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* sring = reinterpret_cast<uint16_t*>(smem);
  uint32_t* sring32 = reinterpret_cast<uint32_t*>(smem);
  uint64_t* llut = reinterpret_cast<uint64_t*>(smem + 2 * kStreamRing);
  uint4* lmeta = reinterpret_cast<uint4*>(smem + 2 * kStreamRing + 8 * kLutSize * a.nt_cap);
  uint32_t* lent = reinterpret_cast<uint32_t*>(smem + 2 * kStreamRing +
                                               (8 * kLutSize + 16) * a.nt_cap);

  const int64_t g = blockIdx.x;
  const int lane = threadIdx.x;
  uint32_t status = 0;
  const uint32_t* __restrict__ hdr = reinterpret_cast<const uint32_t*>(a.payload);
  const TabHdr* th = reinterpret_cast<const TabHdr*>(a.tables);
  bool ok = true;
  if (a.payload_bytes < a.header_bytes || hdr[0] != kMagic || hdr[1] != kVersion ||
      hdr[2] != a.B || hdr[3] != (uint32_t)a.N || hdr[4] != a.C || hdr[5] != a.P ||
      hdr[6] != a.K || hdr[7] != a.chunk_len || hdr[8] != a.M || hdr[9] != kParams) {
    status |= GAANS_ST_HEADER;
    ok = false;
  } else if (!tables_ok(a.tables, a.M, a.tables_bytes) || hdr[10] != th->digest_lo ||
             hdr[11] != th->digest_hi) {
    status |= GAANS_ST_TABLES;
    ok = false;
  }
  const int64_t b = g / a.K;
  const int k = (int)(g - b * a.K);
  const int64_t row = b * a.N;
  const int32_t start = k * (int32_t)a.chunk_len;
  const int32_t endp = (int64_t)start + a.chunk_len < a.N ? start + (int32_t)a.chunk_len
                                                            : (int32_t)a.N;
  const int len = endp - start;
  const int T = (len + kLanes - 1) / kLanes;
  const int A = len < kLanes ? len : kLanes;
  uint32_t beg = 0, endo = 0, want_hash = 0;
  int64_t cb = 0;
  if (ok) {
    beg = g ? hdr[kFixedWords + g - 1] : 0u;
    endo = hdr[kFixedWords + g];
    want_hash = hdr[kFixedWords + a.BK + g];
    cb = (int64_t)endo - (int64_t)beg;
    if (endo < beg || (int64_t)endo > a.payload_bytes - a.header_bytes || cb < 4 * A ||
        ((cb - 4 * A) & 3)) {
      status |= GAANS_ST_CORRUPT;
      ok = false;
    }
  }
  if (ok) {
    Tabs tb;
    tb.gmeta = reinterpret_cast<const TabMeta*>(a.tables + th->meta_off);
    tb.gent = reinterpret_cast<const uint32_t*>(a.tables + th->ent_off);
    tb.glut = reinterpret_cast<const uint64_t*>(a.tables + th->lut_off);
    tb.lmeta = lmeta;
    tb.lent = lent;
    tb.llut = llut;
    int t_lo = 0, t_hi = 0;
    if (a.nt_cap > 0) {
      if (a.stage_all) {
        t_hi = (int)a.M;
      } else {
        t_lo = k * (int)a.P;
        t_hi = t_lo + (int)a.P < (int)a.M ? t_lo + (int)a.P : (int)a.M;
      }
    }
    stage_tables(tb, lmeta, lent, llut, t_lo, t_hi, lane);

    const uint8_t* cdata = a.payload + a.header_bytes + beg;
    Stream S;
    S.s32 = reinterpret_cast<const uint32_t*>(cdata + 4 * A);
    S.safe = reinterpret_cast<const uint32_t*>(cdata);
    S.q = (int)((cb - 4 * A) / 2);  // stream words incl. pad (even)
    S.q32 = S.q / 2;
    S.rp = 0;
    S.filled = 0;
    stream_fetch(S, lane);
    stream_commit(S, sring32, lane);

    uint32_t x = lane < A ? reinterpret_cast<const uint32_t*>(cdata)[lane] : kStateLow;
    uint32_t hash = 0;

    int32_t cbx[kSB], nbx[kSB];
    float cm[kSB], nm[kSB];
    auto load_block = [&](int j, int32_t* ib, float* im) {
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        int p = lane + kLanes * (j * kSB + u);
        p = p < len ? p : len - 1;
        ib[u] = kImplicit ? 0 : a.indexes[row + start + p];
        im[u] = kLatents ? a.medians[udiv((uint32_t)(start + p), a.div_hw)] : 0.0f;
      }
    };
    const int nblk = (T + kSB - 1) / kSB;
    if (nblk > 0) load_block(0, cbx, cm);
    for (int j = 0; j < nblk; ++j) {
      if (j + 1 < nblk) load_block(j + 1, nbx, nm);
      bool lds = tb.nt > 0;
      if (!kImplicit && lds) {
        bool in = true;
#pragma unroll
        for (int u = 0; u < kSB; ++u)
          in = in && (lane + kLanes * (j * kSB + u) >= len ||
                      (uint32_t)(cbx[u] - tb.t_lo) < (uint32_t)tb.nt);
        lds = __ballot(!in) == 0;
      }
      DecMeta ms[kSB];
      if (lds) {
#pragma unroll
        for (int u = 0; u < kSB; ++u)
          ms[u] = dec_map<kImplicit, true>(a, tb, lane, j * kSB + u, len, start, cbx[u], hash,
                                           status);
#pragma unroll
        for (int u = 0; u < kSB; ++u)
          if (j * kSB + u < T)
            dec_step<kLatents, true>(a, tb, ms[u], lane, j * kSB + u, len, row, start, cm[u], x,
                                     S, sring, sring32, status);
      } else {
#pragma unroll
        for (int u = 0; u < kSB; ++u)
          ms[u] = dec_map<kImplicit, false>(a, tb, lane, j * kSB + u, len, start, cbx[u], hash,
                                            status);
#pragma unroll
        for (int u = 0; u < kSB; ++u)
          if (j * kSB + u < T)
            dec_step<kLatents, false>(a, tb, ms[u], lane, j * kSB + u, len, row, start, cm[u],
                                      x, S, sring, sring32, status);
      }
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        cbx[u] = nbx[u];
        cm[u] = nm[u];
      }
    }
    if (lane < A && x != kStateLow) status |= GAANS_ST_CORRUPT;
    if (!(S.rp == S.q || (S.rp == S.q - 1 && (S.q & 1) == 0))) status |= GAANS_ST_CORRUPT;
    hash = wave_sum(hash);
    if (hash != want_hash) status |= GAANS_ST_INDEXHASH;
  }
  status = wave_or(status);
  if (lane == 0 && status)
    __hip_atomic_fetch_or(&a.ctrl[kCtrlDecStatus], status, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  __threadfence();
  __syncthreads();
  uint32_t done = 0;
  if (lane == 0)
    done = __hip_atomic_fetch_add(&a.ctrl[kCtrlDecDone], 1u, __ATOMIC_ACQ_REL,
                                  __HIP_MEMORY_SCOPE_AGENT);
  done = (uint32_t)__shfl((int)done, 0, 64);
  if (done == (uint32_t)(a.BK - 1) && lane == 0) {
    const uint32_t st = __hip_atomic_exchange(&a.ctrl[kCtrlDecStatus], 0u, __ATOMIC_ACQ_REL,
                                              __HIP_MEMORY_SCOPE_AGENT);
    *a.status_out = st;
    __threadfence_system();
    __hip_atomic_store(&a.ctrl[kCtrlDecDone], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---- host helpers -------------------------------------------------------------

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(GAANS_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return GAANS_OK;
}

int check_tables_arg(const gaans_tables* t) {
  if (!t || !t->dev) return fail(GAANS_EINVAL, "tables descriptor or its device pointer is NULL");
  if (t->M < 1) return fail(GAANS_EINVAL, "table count M must be >= 1");
  if (t->bytes < (int64_t)sizeof(TabHdr) || t->bytes > 0xffffffffll)
    return fail(GAANS_EINVAL, "tables bytes %lld out of range", (long long)t->bytes);
  if (t->max_nsym < 1 || t->total_nsym < t->max_nsym)
    return fail(GAANS_EINVAL, "tables descriptor is inconsistent");
  return GAANS_OK;
}

// LDS staging plan: all tables if they fit the budget, else the chunk's
// channel range (P tables), else none.
struct Stage {
  int32_t nt_cap, ne_cap, stage_all;
};

Stage plan_stage(const gaans_tables* t, int64_t P, int64_t per_table, int64_t budget) {
  Stage s{0, 0, 0};
  const int64_t all = t->M * per_table + 4 * t->total_nsym;
  const int64_t range = P * per_table + 4 * P * (int64_t)t->max_nsym;
  if (all <= budget) {
    s.nt_cap = t->M;
    s.ne_cap = (int32_t)t->total_nsym;
    s.stage_all = 1;
  } else if (range <= budget) {
    s.nt_cap = (int32_t)P;
    s.ne_cap = (int32_t)(P * t->max_nsym);
  }
  return s;
}

int encode_stage1(bool latents, void* stream, const int32_t* symbols, const float* y,
                  const float* medians, const int32_t* indexes, const gaans_tables* tables,
                  int64_t B, int64_t N, int64_t C, int64_t P, void* ws, int64_t ws_bytes,
                  void* ctrl, uint64_t* info_out) {
  Layout L;
  int rc = make_layout(B, N, C, P, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables))) return rc;
  if (latents ? (!y || !medians) : !symbols) return fail(GAANS_EINVAL, "input pointer is NULL");
  if (!ctrl) return fail(GAANS_EINVAL, "control block pointer is NULL");
  if (!ws || ws_bytes < L.ws_bytes)
    return fail(GAANS_EINVAL, "workspace too small (%lld < %lld bytes)", (long long)ws_bytes,
                (long long)L.ws_bytes);
  uint8_t* w = static_cast<uint8_t*>(ws);
  const Stage st = plan_stage(tables, P, 16, kEncTableBudget);
  EncArgs a;
  a.symbols = symbols;
  a.y = y;
  a.medians = medians;
  a.indexes = indexes;
  a.tables = static_cast<const uint8_t*>(tables->dev);
  a.M = (uint32_t)tables->M;
  a.tables_bytes = (uint32_t)tables->bytes;
  a.N = N;
  a.K = (int32_t)L.K;
  a.P = (int32_t)P;
  a.C = (int32_t)C;
  a.chunk_len = (int32_t)L.chunk_len;
  a.div_hw = make_udiv((uint32_t)L.HW);
  a.cap_words = (int32_t)L.cap_words;
  a.BK = L.BK;
  a.header_bytes = L.header_bytes;
  a.nt_cap = st.nt_cap;
  a.stage_all = st.stage_all;
  a.chunk_words = reinterpret_cast<uint32_t*>(w + L.o_words_cnt);
  a.chunk_status = reinterpret_cast<uint32_t*>(w + L.o_status);
  a.index_hash = reinterpret_cast<uint32_t*>(w + L.o_hash);
  a.end_off = reinterpret_cast<uint32_t*>(w + L.o_end);
  a.ws_info = reinterpret_cast<uint64_t*>(w + L.o_info);
  a.states = reinterpret_cast<uint32_t*>(w + L.o_states);
  a.words = reinterpret_cast<uint16_t*>(w + L.o_words);
  a.ctrl = static_cast<uint32_t*>(ctrl);
  a.info_out = info_out;
  const size_t lds = 2 * (kRingWords + kLanes) + 16 * (size_t)st.nt_cap + 4 * (size_t)st.ne_cap;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((uint32_t)L.BK), block(kLanes);
  if (latents) {
    if (indexes) k_encode<true, false><<<grid, block, lds, s>>>(a);
    else k_encode<true, true><<<grid, block, lds, s>>>(a);
  } else {
    if (indexes) k_encode<false, false><<<grid, block, lds, s>>>(a);
    else k_encode<false, true><<<grid, block, lds, s>>>(a);
  }
  return check_launch("encode");
}

int decode_impl(bool latents, void* stream, const uint8_t* payload, int64_t payload_bytes,
                const int32_t* indexes, const gaans_tables* tables, const float* medians,
                int64_t B, int64_t N, int64_t C, int64_t P, int32_t* out_sym, float* out_y,
                void* ctrl, uint32_t* status_out) {
  Layout L;
  int rc = make_layout(B, N, C, P, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables))) return rc;
  if (!payload || !status_out || !ctrl || (latents ? (!out_y || !medians) : !out_sym))
    return fail(GAANS_EINVAL, "payload, output, control or status pointer is NULL");
  if (payload_bytes < L.header_bytes)
    return fail(GAANS_EINVAL, "payload (%lld bytes) is shorter than its header (%lld bytes)",
                (long long)payload_bytes, (long long)L.header_bytes);
  const Stage st = plan_stage(tables, P, 8 * kLutSize + 16, kDecTableBudget);
  DecArgs a;
  a.payload = payload;
  a.payload_bytes = payload_bytes;
  a.indexes = indexes;
  a.tables = static_cast<const uint8_t*>(tables->dev);
  a.M = (uint32_t)tables->M;
  a.tables_bytes = (uint32_t)tables->bytes;
  a.medians = medians;
  a.out_sym = out_sym;
  a.out_y = out_y;
  a.N = N;
  a.header_bytes = L.header_bytes;
  a.BK = L.BK;
  a.B = (uint32_t)B;
  a.C = (uint32_t)C;
  a.P = (uint32_t)P;
  a.K = (uint32_t)L.K;
  a.chunk_len = (uint32_t)L.chunk_len;
  a.div_hw = make_udiv((uint32_t)L.HW);
  a.nt_cap = st.nt_cap;
  a.ne_cap = st.ne_cap;
  a.stage_all = st.stage_all;
  a.ctrl = static_cast<uint32_t*>(ctrl);
  a.status_out = status_out;
  const size_t lds = 2 * kStreamRing + (8 * kLutSize + 16) * (size_t)st.nt_cap +
                     4 * (size_t)st.ne_cap;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((uint32_t)L.BK), block(kLanes);
  if (latents) {
    if (indexes) k_decode<true, false><<<grid, block, lds, s>>>(a);
    else k_decode<true, true><<<grid, block, lds, s>>>(a);
  } else {
    if (indexes) k_decode<false, false><<<grid, block, lds, s>>>(a);
    else k_decode<false, true><<<grid, block, lds, s>>>(a);
  }
  return check_launch("decode");
}

uint64_t fnv_u32(uint64_t h, uint32_t v) {
  for (int i = 0; i < 4; ++i) {
    h ^= (v >> (8 * i)) & 0xffu;
    h *= 0x100000001b3ull;
  }
  return h;
}

int64_t tables_size(int32_t M, int64_t total_syms) {
  int64_t o = sizeof(TabHdr);
  o += (int64_t)sizeof(TabMeta) * M;
  o = align_up(o + 4 * total_syms, 8);
  o += 8ll * kLutSize * M;
  return o;
}

}  // namespace

// =============================================================================
// C ABI
// =============================================================================

extern "C" {

int gaans_abi_version(void) { return GAANS_ABI_VERSION; }

const char* gaans_last_error(void) { return g_last_error.c_str(); }

int gaans_get_layout(int64_t B, int64_t N, int64_t C, int64_t P, gaans_layout* out) {
  if (!out) return fail(GAANS_EINVAL, "layout pointer is NULL");
  Layout L;
  int rc = make_layout(B, N, C, P, &L);
  if (rc) return rc;
  out->B = L.B; out->N = L.N; out->C = L.C; out->P = L.P;
  out->HW = L.HW; out->K = L.K; out->chunk_len = L.chunk_len; out->BK = L.BK;
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
  return GAANS_OK;
}

int gaans_tables_bytes(const int32_t* cdf_sizes, int32_t M, int32_t Lmax, int64_t* bytes) {
  if (!cdf_sizes || !bytes) return fail(GAANS_EINVAL, "NULL argument");
  if (M < 1 || Lmax < 2) return fail(GAANS_EINVAL, "need M >= 1 tables of Lmax >= 2 entries");
  int64_t total = 0;
  for (int32_t t = 0; t < M; ++t) {
    const int32_t S = cdf_sizes[t];
    if (S < 2 || S > Lmax || S > 65537)
      return fail(GAANS_ETABLE, "table %d: cdf size %d outside [2, %d]", t, S, Lmax);
    total += S - 1;
  }
  *bytes = tables_size(M, total);
  if (*bytes > 0xffffffffll) return fail(GAANS_ETABLE, "tables exceed 4 GiB");
  return GAANS_OK;
}

int gaans_tables_prepare(const int32_t* cdfs, const int32_t* cdf_sizes, const int32_t* offsets,
                         int32_t M, int32_t Lmax, void* out, int64_t out_bytes,
                         gaans_tables* desc) {
  if (!cdfs || !offsets || !out || !desc) return fail(GAANS_EINVAL, "NULL argument");
  int64_t need = 0;
  int rc = gaans_tables_bytes(cdf_sizes, M, Lmax, &need);
  if (rc) return rc;
  if (out_bytes < need)
    return fail(GAANS_EINVAL, "table buffer too small (%lld < %lld)", (long long)out_bytes,
                (long long)need);
  for (int32_t t = 0; t < M; ++t) {
    const int32_t S = cdf_sizes[t];
    const int32_t* c = cdfs + (int64_t)t * Lmax;
    if (c[0] != 0 || c[S - 1] != 65536)
      return fail(GAANS_ETABLE, "table %d: CDF must start at 0 and end at 65536", t);
    for (int32_t j = 0; j + 1 < S; ++j)
      if (c[j + 1] <= c[j])
        return fail(GAANS_ETABLE, "table %d: CDF is not strictly increasing at entry %d", t, j);
  }
  uint8_t* o = static_cast<uint8_t*>(out);
  memset(o, 0, (size_t)need);
  TabHdr* h = reinterpret_cast<TabHdr*>(o);
  TabMeta* meta = reinterpret_cast<TabMeta*>(o + sizeof(TabHdr));
  const int64_t ent_off = sizeof(TabHdr) + (int64_t)sizeof(TabMeta) * M;
  uint32_t* ent = reinterpret_cast<uint32_t*>(o + ent_off);
  int64_t total = 0;
  uint32_t max_nsym = 0;
  for (int32_t t = 0; t < M; ++t) {
    total += cdf_sizes[t] - 1;
    if ((uint32_t)(cdf_sizes[t] - 1) > max_nsym) max_nsym = (uint32_t)(cdf_sizes[t] - 1);
  }
  const int64_t lut_off = align_up(ent_off + 4 * total, 8);
  uint64_t* lut = reinterpret_cast<uint64_t*>(o + lut_off);
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
    meta[t].lut_base = (uint32_t)t * kLutSize;
    for (uint32_t v = 0; v < nsym; ++v)
      ent[base + v] = (uint32_t)c[v] | ((uint32_t)(c[v + 1] - c[v] - 1) << 16);
    // bucket j covers cum in [j << 8, (j << 8) + 255]; low word = entry of
    // the symbol s holding the bucket's first value; high word = s | next << 16,
    // next = freq(s + 1) - 1 when the bucket holds at most one boundary, else
    // the marker 0xffff (freq(s + 1) <= 65535, so next never equals it).
    uint32_t s = 0;
    for (int j = 0; j < kLutSize; ++j) {
      const uint32_t lo = (uint32_t)j << (16 - kLutBits);
      const uint32_t hi = lo + (1u << (16 - kLutBits)) - 1u;
      while (s + 1 < nsym && (uint32_t)c[s + 1] <= lo) ++s;
      uint32_t e = s;
      while (e + 1 < nsym && (uint32_t)c[e + 1] <= hi) ++e;
      uint32_t next = 0;
      if (e - s >= 2) next = 0xffffu;
      else if (s + 1 < nsym) next = (uint32_t)(c[s + 2] - c[s + 1] - 1);
      const uint32_t lo_word = (uint32_t)c[s] | ((uint32_t)(c[s + 1] - c[s] - 1) << 16);
      const uint32_t hi_word = s | (next << 16);
      lut[(int64_t)t * kLutSize + j] = (uint64_t)lo_word | ((uint64_t)hi_word << 32);
    }
    base += nsym;
  }
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
  desc->dev = nullptr;
  desc->bytes = need;
  desc->M = M;
  desc->max_nsym = (int32_t)max_nsym;
  desc->total_nsym = total;
  desc->digest = dg;
  return GAANS_OK;
}

int gaans_encode_symbols(void* stream, const int32_t* symbols_dev, const int32_t* indexes_dev,
                         const gaans_tables* tables, int64_t B, int64_t N, int64_t C, int64_t P,
                         void* workspace_dev, int64_t workspace_bytes, void* ctrl_dev,
                         uint64_t* info_out) {
  return encode_stage1(false, stream, symbols_dev, nullptr, nullptr, indexes_dev, tables, B, N,
                       C, P, workspace_dev, workspace_bytes, ctrl_dev, info_out);
}

int gaans_encode_latents(void* stream, const float* y_dev, const float* medians_dev,
                         const int32_t* indexes_dev, const gaans_tables* tables, int64_t B,
                         int64_t N, int64_t C, int64_t P, void* workspace_dev,
                         int64_t workspace_bytes, void* ctrl_dev, uint64_t* info_out) {
  return encode_stage1(true, stream, nullptr, y_dev, medians_dev, indexes_dev, tables, B, N, C,
                       P, workspace_dev, workspace_bytes, ctrl_dev, info_out);
}

int gaans_encode_pack(void* stream, const void* workspace_dev, int64_t workspace_bytes,
                      const gaans_tables* tables, int64_t B, int64_t N, int64_t C, int64_t P,
                      uint8_t* out_dev, int64_t out_bytes) {
  Layout L;
  int rc = make_layout(B, N, C, P, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables))) return rc;
  if (!workspace_dev || workspace_bytes < L.ws_bytes)
    return fail(GAANS_EINVAL, "workspace too small");
  if (!out_dev || out_bytes < L.header_bytes)
    return fail(GAANS_EINVAL, "output buffer smaller than the payload header");
  const uint8_t* w = static_cast<const uint8_t*>(workspace_dev);
  PackArgs a;
  a.chunk_words = reinterpret_cast<const uint32_t*>(w + L.o_words_cnt);
  a.index_hash = reinterpret_cast<const uint32_t*>(w + L.o_hash);
  a.end_off = reinterpret_cast<const uint32_t*>(w + L.o_end);
  a.states = reinterpret_cast<const uint32_t*>(w + L.o_states);
  a.words = reinterpret_cast<const uint16_t*>(w + L.o_words);
  a.tables = static_cast<const uint8_t*>(tables->dev);
  a.out = out_dev;
  a.out_bytes = out_bytes;
  a.header_bytes = L.header_bytes;
  a.cap_words = L.cap_words;
  a.BK = L.BK;
  a.N = N;
  a.B = (uint32_t)B;
  a.N32 = (uint32_t)N;
  a.C = (uint32_t)C;
  a.P = (uint32_t)P;
  a.K = (uint32_t)L.K;
  a.chunk_len = (uint32_t)L.chunk_len;
  a.M = (uint32_t)tables->M;
  k_pack<<<dim3((uint32_t)L.BK), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch("pack");
}

int gaans_decode_symbols(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                         const int32_t* indexes_dev, const gaans_tables* tables, int64_t B,
                         int64_t N, int64_t C, int64_t P, int32_t* out_dev, void* ctrl_dev,
                         uint32_t* status_out) {
  return decode_impl(false, stream, payload_dev, payload_bytes, indexes_dev, tables, nullptr, B,
                     N, C, P, out_dev, nullptr, ctrl_dev, status_out);
}

int gaans_decode_latents(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                         const int32_t* indexes_dev, const gaans_tables* tables,
                         const float* medians_dev, int64_t B, int64_t N, int64_t C, int64_t P,
                         float* y_hat_dev, void* ctrl_dev, uint32_t* status_out) {
  return decode_impl(true, stream, payload_dev, payload_bytes, indexes_dev, tables, medians_dev,
                     B, N, C, P, nullptr, y_hat_dev, ctrl_dev, status_out);
}

int gaans_host_selftest(void) {
  // 1. magic division: every divisor class against exact division
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
  // 2. encoder quotient: fp32 reciprocal (exact, and one ulp either side to
  //    cover v_rcp_f32's error) with one signed correction, for every freq
  for (uint32_t f = 1; f <= 65536; ++f) {
    const float r0 = 1.0f / (float)f;
    const float rs[3] = {r0, nextafterf(r0, 0.0f), nextafterf(r0, 1.0f)};
    const uint32_t xmax = (uint32_t)(((uint64_t)f << 16) - 1u);
    uint32_t xs[8] = {0u, 1u, f - 1u, f, xmax, xmax - 1u, xmax - f, xmax / 2u};
    for (int k = 0; k < 8; ++k) {
      const uint32_t x = xs[k];
      if ((uint64_t)x > xmax) continue;
      for (int j = 0; j < 3; ++j) {
        uint32_t q = (uint32_t)((float)x * rs[j]);
        int32_t r = (int32_t)(x - q * f);
        if (r < 0) { q -= 1u; r += (int32_t)f; }
        else if (r >= (int32_t)f) { q += 1u; r -= (int32_t)f; }
        if (q != x / f || (uint32_t)r != x % f)
          return fail(2, "division selftest failed f=%u x=%u", f, x);
      }
    }
  }
  return GAANS_OK;
}

}  // extern "C"
