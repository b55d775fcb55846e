// GA-ANS wave64 latent coder for MI355X (gfx950): HIP kernels + C ABI.
//
// One wave64 codes one chunk of P latent channels.  Each lane carries one
// 32-bit rANS state (x in [2^16, 2^32), 16-bit renormalisation words, 16-bit
// CDF precision).  Lane l of a chunk owns positions l + 64 t, so a wave reads
// 64 consecutive symbols per step.  The renormalisation words a step emits
// are compacted in lane order with a wave ballot + mbcnt prefix count and
// written backwards into a per-chunk staging slot; a one-block scan turns the
// per-chunk sizes into payload offsets and a pack kernel writes the payload.
// The decoder mirrors the schedule: refill words are handed out in lane order
// from the same ballot/mbcnt prefix.
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
struct TabHdr {
  uint32_t magic, M, total_syms, lut_bits;
  uint32_t digest_lo, digest_hi;
  uint32_t meta_off, ent_off, lut_off;  // byte offsets
  uint32_t total_bytes;
  uint32_t reserved[6];
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

// Encoder main op on a renormalised state x < freq << 16:
// x' = ((x / freq) << 16) + x % freq + start.  The quotient comes from a fp32
// reciprocal (error < 2^-6 because x / freq < 2^16) and one signed correction.
__device__ __forceinline__ uint32_t enc_main(uint32_t x, uint32_t start, uint32_t freq,
                                             float rcp) {
  uint32_t q = (uint32_t)((float)x * rcp);
  int32_t r = (int32_t)(x - q * freq);
  if (r < 0) {
    q -= 1u;
    r += (int32_t)freq;
  } else if (r >= (int32_t)freq) {
    q += 1u;
    r -= (int32_t)freq;
  }
  return (q << 16) + (uint32_t)r + start;
}

struct EncArgs {
  const int32_t* __restrict__ symbols;
  const float* __restrict__ y;
  const float* __restrict__ medians;
  const int32_t* __restrict__ indexes;
  const uint8_t* __restrict__ tables;
  uint32_t M;
  uint32_t tables_bytes;
  int64_t N;
  int32_t K, P, chunk_len, HW;
  UDiv div_hw;
  int64_t cap_words;
  uint32_t* __restrict__ chunk_words;
  uint32_t* __restrict__ chunk_status;
  uint32_t* __restrict__ index_hash;
  uint32_t* __restrict__ states;
  uint16_t* __restrict__ words;
};

__device__ __forceinline__ bool tables_ok(const uint8_t* tables, uint32_t M, uint32_t bytes) {
  const TabHdr* h = reinterpret_cast<const TabHdr*>(tables);
  return h->magic == kTabMagic && h->M == M && h->total_bytes == bytes &&
         h->lut_bits == (uint32_t)kLutBits;
}

// One wave64 per chunk.  kLatents: quantize y - median on the fly.
template <bool kLatents>
__global__ __launch_bounds__(64) void k_encode(EncArgs a) {
  const int g = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t b = g / a.K;
  const int k = g - (int)(b * a.K);
  const int64_t row = b * a.N;
  const int64_t start = (int64_t)k * a.chunk_len;
  const int64_t endp = start + a.chunk_len < a.N ? start + a.chunk_len : a.N;
  const int len = (int)(endp - start);
  const int T = (len + kLanes - 1) / kLanes;
  uint16_t* __restrict__ wbuf = a.words + (int64_t)g * a.cap_words;
  int64_t wp = a.cap_words;  // wave-uniform write cursor (backwards)
  uint32_t x = kStateLow;
  uint32_t hash = 0, status = 0;

  if (!tables_ok(a.tables, a.M, a.tables_bytes)) {
    if (lane == 0) {
      a.chunk_words[g] = 0;
      a.chunk_status[g] = GAANS_ST_TABLES;
      a.index_hash[g] = 0;
    }
    return;
  }
  const TabHdr* th = reinterpret_cast<const TabHdr*>(a.tables);
  const TabMeta* __restrict__ meta = reinterpret_cast<const TabMeta*>(a.tables + th->meta_off);
  const uint32_t* __restrict__ ent = reinterpret_cast<const uint32_t*>(a.tables + th->ent_off);

  // software prefetch of step t's inputs
  auto load_in = [&](int t, int32_t& sym_or_bits, int32_t& tb) {
    const int p = lane + kLanes * t;
    sym_or_bits = 0;
    tb = 0;
    if (p < len) {
      const int64_t i = start + p;
      if (a.indexes) tb = a.indexes[row + i];
      else tb = (int32_t)(udiv((uint32_t)i, a.div_hw));
      if (kLatents) sym_or_bits = __float_as_int(a.y[row + i]);
      else sym_or_bits = a.symbols[row + i];
    }
  };

  int32_t nx_sym = 0, nx_tb = 0;
  if (T > 0) load_in(T - 1, nx_sym, nx_tb);
  for (int t = T - 1; t >= 0; --t) {
    const int32_t in_sym = nx_sym, tb_raw = nx_tb;
    if (t > 0) load_in(t - 1, nx_sym, nx_tb);
    const int p = lane + kLanes * t;
    bool act = p < len;
    uint32_t st = 0, fr = 1, raw = 0;
    int nnib = 0;
    bool esc = false;
    if (act) {
      int32_t tb = tb_raw;
      if ((uint32_t)tb >= a.M) {
        status |= GAANS_ST_INDEX;
        act = false;
      } else {
        hash += (uint32_t)(tb + 1) ^ ((uint32_t)p * kHashMul);
        int64_t symv;
        if (kLatents) {
          const int64_t i = start + p;
          const uint32_t c = udiv((uint32_t)i, a.div_hw);
          const float d = __fsub_rn(__int_as_float(in_sym), a.medians[c]);
          const float r = rintf(d);
          if (!(fabsf(r) < 2147483648.0f)) {
            status |= GAANS_ST_RANGE;
            symv = 0;
          } else {
            symv = (int32_t)r;
          }
        } else {
          symv = in_sym;
        }
        const TabMeta m = meta[tb];
        const int64_t maxv = (int64_t)m.nsym - 1;
        int64_t v = symv - (int64_t)m.offset;
        int64_t rw = 0;
        if (v < 0) {
          rw = -2 * v - 1;
          v = maxv;
          esc = true;
        } else if (v >= maxv) {
          rw = 2 * (v - maxv);
          v = maxv;
          esc = true;
        }
        if (rw >= ((int64_t)1 << 32)) {
          status |= GAANS_ST_RANGE;
          rw = 0;
        }
        raw = (uint32_t)rw;
        nnib = raw ? ((31 - __clz((int)raw)) >> 2) + 1 : 0;
        const uint32_t e = ent[m.ent_base + (uint32_t)v];
        st = e & 0xffffu;
        fr = (e >> 16) + 1u;
      }
    }
    const float rcp = __builtin_amdgcn_rcpf((float)fr);
    const uint64_t escmask = __ballot(esc);
    if (escmask == 0) {
      const bool emit = act && (x >> 16) >= fr;
      const uint64_t m = __ballot(emit);
      wp -= __popcll(m);
      if (emit) {
        wbuf[wp + lane_rank(m)] = (uint16_t)x;
        x >>= 16;
      }
      if (act) x = enc_main(x, st, fr, rcp);
    } else {
      const int nops = act ? (esc ? nnib + 2 : 1) : 0;
      const int Mt = wave_max(nops);
      for (int d = Mt - 1; d >= 0; --d) {
        const bool part = d < nops;
        bool emit;
        if (d == 0) emit = part && (x >> 16) >= fr;
        else emit = part && x >= kBitsEmit;
        const uint64_t m = __ballot(emit);
        wp -= __popcll(m);
        if (emit) {
          wbuf[wp + lane_rank(m)] = (uint16_t)x;
          x >>= 16;
        }
        if (part) {
          if (d == 0) {
            x = enc_main(x, st, fr, rcp);
          } else {
            const uint32_t val = d == 1 ? (uint32_t)nnib : (raw >> (4 * (d - 2))) & 15u;
            x = (x << 4) | val;
          }
        }
      }
    }
  }
  const int A = len < kLanes ? len : kLanes;
  if (lane < A) a.states[(int64_t)g * kLanes + lane] = x;
  hash = wave_sum(hash);
  status = wave_or(status);
  if (lane == 0) {
    a.chunk_words[g] = (uint32_t)(a.cap_words - wp);
    a.chunk_status[g] = status;
    a.index_hash[g] = hash;
  }
}

struct ScanArgs {
  const uint32_t* __restrict__ chunk_words;
  const uint32_t* __restrict__ chunk_status;
  uint32_t* __restrict__ end_off;
  uint64_t* __restrict__ info;
  int64_t BK, N, header_bytes;
  int32_t K, chunk_len;
};

__device__ __forceinline__ int chunk_len_of(int64_t g, int32_t K, int32_t chunk_len, int64_t N) {
  const int64_t k = g % K;
  const int64_t s = k * chunk_len;
  const int64_t e = s + chunk_len < N ? s + chunk_len : N;
  return (int)(e - s);
}

// Device-wide exclusive scan of the chunk byte sizes (one block; B*K is at
// most a few ten thousand chunks), plus the OR of the chunk status words.
__global__ __launch_bounds__(1024) void k_scan(ScanArgs a) {
  __shared__ uint64_t wave_tot[16];
  __shared__ uint32_t st_sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  if (tid == 0) st_sh = 0;
  __syncthreads();
  uint64_t carry = 0;
  uint32_t st = 0;
  for (int64_t base = 0; base < a.BK; base += 1024) {
    const int64_t g = base + tid;
    uint64_t v = 0;
    if (g < a.BK) {
      const int len = chunk_len_of(g, a.K, a.chunk_len, a.N);
      const uint32_t A = len < kLanes ? (uint32_t)len : (uint32_t)kLanes;
      const uint32_t W = a.chunk_words[g];
      v = 4ull * A + 2ull * (W + (W & 1u));
      st |= a.chunk_status[g];
    }
    // inclusive wave scan
    uint64_t incl = v;
    for (int off = 1; off < 64; off <<= 1) {
      uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)incl, off, 64);
      uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(incl >> 32), off, 64);
      uint64_t o = ((uint64_t)hi << 32) | lo;
      if (lane >= off) incl += o;
    }
    if (lane == 63) wave_tot[wid] = incl;
    __syncthreads();
    uint64_t before = carry;
    for (int w = 0; w < wid; ++w) before += wave_tot[w];
    uint64_t tile_total = 0;
    for (int w = 0; w < 16; ++w) tile_total += wave_tot[w];
    if (g < a.BK) {
      const uint64_t e = before + incl;
      a.end_off[g] = (uint32_t)e;
      if (e > 0xffffffffull) st |= GAANS_ST_SIZE;
    }
    carry += tile_total;
    __syncthreads();
  }
  st = wave_or(st);
  if (lane == 0 && st) atomicOr(&st_sh, st);
  __syncthreads();
  if (tid == 0) {
    a.info[0] = (uint64_t)a.header_bytes + carry;
    a.info[1] = st_sh;
  }
}

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
  if ((int64_t)a.header_bytes + endo > a.out_bytes || endo < beg) return;
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

struct DecArgs {
  const uint8_t* __restrict__ payload;
  int64_t payload_bytes;
  const int32_t* __restrict__ indexes;
  const uint8_t* __restrict__ tables;
  uint32_t M, tables_bytes;
  const float* __restrict__ medians;
  int32_t* __restrict__ out_sym;
  float* __restrict__ out_y;
  uint32_t* __restrict__ status;
  int64_t N, header_bytes, BK;
  uint32_t B, C, P, K, chunk_len, HW;
  UDiv div_hw;
};

struct Sym {
  uint32_t v, start, freq;
};

__device__ __forceinline__ Sym dec_lookup(const uint64_t* __restrict__ lut,
                                          const uint32_t* __restrict__ ent, uint32_t cum) {
  const uint64_t e = lut[cum >> (16 - kLutBits)];
  const uint32_t lo = (uint32_t)e, hi = (uint32_t)(e >> 32);
  uint32_t s = hi & 0xffffu;
  const uint32_t span = hi >> 16;
  if (span == 0) return Sym{s, lo & 0xffffu, (lo >> 16) + 1u};
  uint32_t hi_s = s + span;  // answer in [s, hi_s]; start(s) <= cum
  while (s < hi_s) {
    const uint32_t mid = (s + hi_s + 1) >> 1;
    if ((ent[mid] & 0xffffu) <= cum) s = mid;
    else hi_s = mid - 1;
  }
  const uint32_t en = ent[s];
  return Sym{s, en & 0xffffu, (en >> 16) + 1u};
}

template <bool kLatents>
__global__ __launch_bounds__(64) void k_decode(DecArgs a) {
  const int64_t g = blockIdx.x;
  const int lane = threadIdx.x;
  uint32_t status = 0;
  const uint32_t* __restrict__ hdr = reinterpret_cast<const uint32_t*>(a.payload);
  // header checks (uniform)
  if (a.payload_bytes < a.header_bytes || hdr[0] != kMagic || hdr[1] != kVersion ||
      hdr[2] != a.B || hdr[3] != (uint32_t)a.N || hdr[4] != a.C || hdr[5] != a.P ||
      hdr[6] != a.K || hdr[7] != a.chunk_len || hdr[8] != a.M || hdr[9] != kParams) {
    if (lane == 0) atomicOr(a.status, GAANS_ST_HEADER);
    return;
  }
  if (!tables_ok(a.tables, a.M, a.tables_bytes)) {
    if (lane == 0) atomicOr(a.status, GAANS_ST_TABLES);
    return;
  }
  const TabHdr* th = reinterpret_cast<const TabHdr*>(a.tables);
  if (hdr[10] != th->digest_lo || hdr[11] != th->digest_hi) {
    if (lane == 0) atomicOr(a.status, GAANS_ST_TABLES);
    return;
  }
  const TabMeta* __restrict__ meta = reinterpret_cast<const TabMeta*>(a.tables + th->meta_off);
  const uint32_t* __restrict__ ent = reinterpret_cast<const uint32_t*>(a.tables + th->ent_off);
  const uint64_t* __restrict__ lutall = reinterpret_cast<const uint64_t*>(a.tables + th->lut_off);

  const int64_t b = g / a.K;
  const int k = (int)(g - b * a.K);
  const int64_t row = b * a.N;
  const int64_t start = (int64_t)k * a.chunk_len;
  const int64_t endp = start + a.chunk_len < a.N ? start + a.chunk_len : a.N;
  const int len = (int)(endp - start);
  const int T = (len + kLanes - 1) / kLanes;
  const int A = len < kLanes ? len : kLanes;
  const int64_t data_len = a.payload_bytes - a.header_bytes;
  const uint32_t beg = g ? hdr[kFixedWords + g - 1] : 0u;
  const uint32_t endo = hdr[kFixedWords + g];
  const uint32_t want_hash = hdr[kFixedWords + a.BK + g];
  const int64_t cb = (int64_t)endo - (int64_t)beg;
  if (endo < beg || (int64_t)endo > data_len || cb < 4 * A || ((cb - 4 * A) & 3)) {
    if (lane == 0) atomicOr(a.status, GAANS_ST_CORRUPT);
    return;
  }
  const uint8_t* cdata = a.payload + a.header_bytes + beg;
  const uint16_t* __restrict__ wstream = reinterpret_cast<const uint16_t*>(cdata + 4 * A);
  const int64_t q = (cb - 4 * A) / 2;
  int64_t rp = 0;  // wave-uniform read cursor
  uint32_t x = lane < A ? reinterpret_cast<const uint32_t*>(cdata)[lane] : kStateLow;
  uint32_t hash = 0;

  auto refill = [&](bool need) {
    const uint64_t m = __ballot(need);
    if (need) {
      const int64_t r = rp + lane_rank(m);
      uint32_t w = 0;
      if (r < q) w = wstream[r];
      else status |= GAANS_ST_CORRUPT;
      x = (x << 16) | w;
    }
    rp += __popcll(m);
  };

  for (int t = 0; t < T; ++t) {
    const int p = lane + kLanes * t;
    bool act = p < len;
    const int64_t i = start + p;
    int32_t tb = 0;
    if (act) {
      tb = a.indexes ? a.indexes[row + i] : (int32_t)udiv((uint32_t)i, a.div_hw);
      if ((uint32_t)tb >= a.M) {
        status |= GAANS_ST_INDEX;
        tb = 0;
      }
      hash += (uint32_t)(tb + 1) ^ ((uint32_t)p * kHashMul);
    }
    const TabMeta m = meta[tb];
    Sym s{0, 0, 1};
    if (act) {
      const uint32_t cum = x & 0xffffu;
      s = dec_lookup(lutall + m.lut_base, ent + m.ent_base, cum);
      x = s.freq * (x >> 16) + cum - s.start;
    }
    refill(act && x < kStateLow);
    const bool esc = act && s.v == m.nsym - 1;
    int64_t value = s.v;
    if (__ballot(esc)) {
      uint32_t n = 0;
      if (esc) {
        n = x & 15u;
        x >>= 4;
      }
      refill(esc && x < kStateLow);
      if (n > 8) {
        status |= GAANS_ST_CORRUPT;
        n = 0;
      }
      uint32_t raw = 0;
      for (uint32_t j = 0; __ballot(esc && j < n); ++j) {
        const bool part = esc && j < n;
        if (part) {
          raw |= (x & 15u) << (4 * j);
          x >>= 4;
        }
        refill(part && x < kStateLow);
      }
      if (esc) {
        const int64_t maxv = (int64_t)m.nsym - 1;
        value = (raw & 1u) ? -(int64_t)(raw >> 1) - 1 : (int64_t)(raw >> 1) + maxv;
      }
    }
    if (act) {
      int64_t sv = value + m.offset;
      if (sv < INT32_MIN || sv > INT32_MAX) {
        status |= GAANS_ST_CORRUPT;
        sv = 0;
      }
      if (kLatents) {
        const uint32_t c = udiv((uint32_t)i, a.div_hw);
        a.out_y[row + i] = __fadd_rn((float)(int32_t)sv, a.medians[c]);
      } else {
        a.out_sym[row + i] = (int32_t)sv;
      }
    }
  }
  if (lane < A && x != kStateLow) status |= GAANS_ST_CORRUPT;
  if (!(rp == q || (rp == q - 1 && (q & 1) == 0))) status |= GAANS_ST_CORRUPT;
  hash = wave_sum(hash);
  status = wave_or(status);
  if (hash != want_hash) status |= GAANS_ST_INDEXHASH;
  if (lane == 0 && status) atomicOr(a.status, status);
}

// ---- host helpers -------------------------------------------------------------

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(GAANS_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return GAANS_OK;
}

int check_tables_arg(const void* tables, int64_t tables_bytes, int32_t M) {
  if (!tables) return fail(GAANS_EINVAL, "tables pointer is NULL");
  if (M < 1) return fail(GAANS_EINVAL, "table count M must be >= 1");
  if (tables_bytes < (int64_t)sizeof(TabHdr) || tables_bytes > 0xffffffffll)
    return fail(GAANS_EINVAL, "tables_bytes %lld out of range", (long long)tables_bytes);
  return GAANS_OK;
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

int encode_stage1(bool latents, void* stream, const int32_t* symbols, const float* y,
                  const float* medians, const int32_t* indexes, const void* tables,
                  int64_t tables_bytes, int32_t M, int64_t B, int64_t N, int64_t C, int64_t P,
                  void* ws, int64_t ws_bytes) {
  Layout L;
  int rc = make_layout(B, N, C, P, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables, tables_bytes, M))) return rc;
  if (latents ? (!y || !medians) : !symbols) return fail(GAANS_EINVAL, "input pointer is NULL");
  if (!ws || ws_bytes < L.ws_bytes)
    return fail(GAANS_EINVAL, "workspace too small (%lld < %lld bytes)", (long long)ws_bytes,
                (long long)L.ws_bytes);
  uint8_t* w = static_cast<uint8_t*>(ws);
  EncArgs a;
  a.symbols = symbols;
  a.y = y;
  a.medians = medians;
  a.indexes = indexes;
  a.tables = static_cast<const uint8_t*>(tables);
  a.M = (uint32_t)M;
  a.tables_bytes = (uint32_t)tables_bytes;
  a.N = N;
  a.K = (int32_t)L.K;
  a.P = (int32_t)P;
  a.chunk_len = (int32_t)L.chunk_len;
  a.HW = (int32_t)L.HW;
  a.div_hw = make_udiv((uint32_t)L.HW);
  a.cap_words = L.cap_words;
  a.chunk_words = reinterpret_cast<uint32_t*>(w + L.o_words_cnt);
  a.chunk_status = reinterpret_cast<uint32_t*>(w + L.o_status);
  a.index_hash = reinterpret_cast<uint32_t*>(w + L.o_hash);
  a.states = reinterpret_cast<uint32_t*>(w + L.o_states);
  a.words = reinterpret_cast<uint16_t*>(w + L.o_words);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (latents) k_encode<true><<<dim3((uint32_t)L.BK), dim3(kLanes), 0, s>>>(a);
  else k_encode<false><<<dim3((uint32_t)L.BK), dim3(kLanes), 0, s>>>(a);
  if ((rc = check_launch("encode"))) return rc;
  ScanArgs sa;
  sa.chunk_words = a.chunk_words;
  sa.chunk_status = a.chunk_status;
  sa.end_off = reinterpret_cast<uint32_t*>(w + L.o_end);
  sa.info = reinterpret_cast<uint64_t*>(w + L.o_info);
  sa.BK = L.BK;
  sa.N = N;
  sa.header_bytes = L.header_bytes;
  sa.K = (int32_t)L.K;
  sa.chunk_len = (int32_t)L.chunk_len;
  k_scan<<<dim3(1), dim3(1024), 0, s>>>(sa);
  return check_launch("scan");
}

int decode_impl(bool latents, void* stream, const uint8_t* payload, int64_t payload_bytes,
                const int32_t* indexes, const void* tables, int64_t tables_bytes, int32_t M,
                const float* medians, int64_t B, int64_t N, int64_t C, int64_t P,
                int32_t* out_sym, float* out_y, uint32_t* status) {
  Layout L;
  int rc = make_layout(B, N, C, P, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables, tables_bytes, M))) return rc;
  if (!payload || !status || (latents ? (!out_y || !medians) : !out_sym))
    return fail(GAANS_EINVAL, "payload, output or status pointer is NULL");
  if (payload_bytes < L.header_bytes)
    return fail(GAANS_EINVAL, "payload (%lld bytes) is shorter than its header (%lld bytes)",
                (long long)payload_bytes, (long long)L.header_bytes);
  DecArgs a;
  a.payload = payload;
  a.payload_bytes = payload_bytes;
  a.indexes = indexes;
  a.tables = static_cast<const uint8_t*>(tables);
  a.M = (uint32_t)M;
  a.tables_bytes = (uint32_t)tables_bytes;
  a.medians = medians;
  a.out_sym = out_sym;
  a.out_y = out_y;
  a.status = status;
  a.N = N;
  a.header_bytes = L.header_bytes;
  a.BK = L.BK;
  a.B = (uint32_t)B;
  a.C = (uint32_t)C;
  a.P = (uint32_t)P;
  a.K = (uint32_t)L.K;
  a.chunk_len = (uint32_t)L.chunk_len;
  a.HW = (uint32_t)L.HW;
  a.div_hw = make_udiv((uint32_t)L.HW);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (latents) k_decode<true><<<dim3((uint32_t)L.BK), dim3(kLanes), 0, s>>>(a);
  else k_decode<false><<<dim3((uint32_t)L.BK), dim3(kLanes), 0, s>>>(a);
  return check_launch("decode");
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
                         uint64_t* digest) {
  if (!cdfs || !offsets || !out || !digest) return fail(GAANS_EINVAL, "NULL argument");
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
  for (int32_t t = 0; t < M; ++t) total += cdf_sizes[t] - 1;
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
    // bucket j covers cum in [j << 8, (j << 8) + 255]
    uint32_t s = 0;
    for (int j = 0; j < kLutSize; ++j) {
      const uint32_t lo = (uint32_t)j << (16 - kLutBits);
      const uint32_t hi = lo + (1u << (16 - kLutBits)) - 1u;
      while (s + 1 < nsym && (uint32_t)c[s + 1] <= lo) ++s;
      uint32_t e = s;
      while (e + 1 < nsym && (uint32_t)c[e + 1] <= hi) ++e;
      const uint32_t lo_word = (uint32_t)c[s] | ((uint32_t)(c[s + 1] - c[s] - 1) << 16);
      const uint32_t hi_word = s | ((e - s) << 16);
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
  *digest = dg;
  return GAANS_OK;
}

int gaans_encode_symbols(void* stream, const int32_t* symbols_dev, const int32_t* indexes_dev,
                         const void* tables_dev, int64_t tables_bytes, int32_t M, int64_t B,
                         int64_t N, int64_t C, int64_t P, void* workspace_dev,
                         int64_t workspace_bytes) {
  return encode_stage1(false, stream, symbols_dev, nullptr, nullptr, indexes_dev, tables_dev,
                       tables_bytes, M, B, N, C, P, workspace_dev, workspace_bytes);
}

int gaans_encode_latents(void* stream, const float* y_dev, const float* medians_dev,
                         const int32_t* indexes_dev, const void* tables_dev,
                         int64_t tables_bytes, int32_t M, int64_t B, int64_t N, int64_t C,
                         int64_t P, void* workspace_dev, int64_t workspace_bytes) {
  return encode_stage1(true, stream, nullptr, y_dev, medians_dev, indexes_dev, tables_dev,
                       tables_bytes, M, B, N, C, P, workspace_dev, workspace_bytes);
}

int gaans_encode_pack(void* stream, const void* workspace_dev, int64_t workspace_bytes,
                      const void* tables_dev, int64_t tables_bytes, int32_t M, int64_t B,
                      int64_t N, int64_t C, int64_t P, uint8_t* out_dev, int64_t out_bytes) {
  Layout L;
  int rc = make_layout(B, N, C, P, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables_dev, tables_bytes, M))) return rc;
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
  a.tables = static_cast<const uint8_t*>(tables_dev);
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
  a.M = (uint32_t)M;
  k_pack<<<dim3((uint32_t)L.BK), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch("pack");
}

int gaans_decode_symbols(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                         const int32_t* indexes_dev, const void* tables_dev,
                         int64_t tables_bytes, int32_t M, int64_t B, int64_t N, int64_t C,
                         int64_t P, int32_t* out_dev, uint32_t* status_dev) {
  return decode_impl(false, stream, payload_dev, payload_bytes, indexes_dev, tables_dev,
                     tables_bytes, M, nullptr, B, N, C, P, out_dev, nullptr, status_dev);
}

int gaans_decode_latents(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                         const int32_t* indexes_dev, const void* tables_dev,
                         int64_t tables_bytes, int32_t M, const float* medians_dev, int64_t B,
                         int64_t N, int64_t C, int64_t P, float* y_hat_dev,
                         uint32_t* status_dev) {
  return decode_impl(true, stream, payload_dev, payload_bytes, indexes_dev, tables_dev,
                     tables_bytes, M, medians_dev, B, N, C, P, nullptr, y_hat_dev, status_dev);
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
