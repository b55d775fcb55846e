// GA-ANS wave64 latent coder for MI355X (gfx950): HIP kernels + C ABI.
//
// Format: one chunk = P latent channels, split into S segments of whole
// 64-position steps; a segment is a coding unit with 64 lanes and one 32-bit
// rANS state per lane (x in [2^16, 2^32), 16-bit renormalisation words,
// 16-bit CDF precision); lane l owns positions l + 64 t of the unit.  The
// words a step emits are ordered by lane (wave ballot + mbcnt prefix); the
// decoder hands refill words out in the same order.  The bytes are defined
// by the CPU oracle (oracle/gaans_oracle.c).
//
// Work mapping: one workgroup per coding unit (a coder wave and mapper
// waves for encode; one more wave, the escape reader, for decode).  A chunk's
// S units run on S CUs, so S > 1 puts a launch of few long chunks on more of
// the chip.
//  - Wave 0 is the coder: it owns the 64 lane states and runs only the
//    serial part of every step (renormalisation, ballot compaction, state
//    update).
//  - The mappers: one block of steps ahead of the coder they load symbols /
//    indexes / latents from HBM (a block ahead again, so the loads are in
//    flight while the previous block is mapped), look the tables up, split
//    escapes, hash the indexes and write one op record per lane and step
//    into LDS (16 bytes for encode, 8 for decode); the decoder's mappers also
//    store the decoded values a block behind.
//  - The decoder's escape reader parses the chunk's escape section ahead of
//    the coder into an LDS FIFO, so an escape costs the coder one LDS read.
//  - The CDF tables of the chunk's channels (or all tables, when they are
//    few) are staged in LDS by the whole workgroup; others are read through
//    L1/L2.
//  - encode: emitted words go to an LDS ring, flushed to a per-chunk staging
//    slot when full; decode: the word stream is prefetched from HBM into
//    registers and copied into an LDS ring ahead of use.
//  - The last workgroup of a launch (device-scope counter in a caller-owned
//    control block) scans the chunk sizes into payload offsets (encode) or
//    reduces the status words (decode) and writes them to caller memory.
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

#include <algorithm>
#include <chrono>
#include <mutex>
#include <string>
#include <type_traits>

#include "gaans_common.h"
#include "gaans_w64.h"

using namespace gaans;

namespace {

#ifndef GAANS_MAPPERS
#define GAANS_MAPPERS 4
#endif
constexpr int kMappers = GAANS_MAPPERS;  // mapper waves per decode workgroup
// Encode workgroups: a coder wave and 4 mapper waves when several
// workgroups share a CU, 8 when each has a CU to itself (the mappers are the
// encoder's slower half: 8 take the 2160x3840 latent from 456 to 446 us and
// the hyperprior y at P=16 from 91 to 68 us, while at three workgroups per
// CU 8 cost more than they bring)
constexpr int kEncMaxWaves = 9;

// per-wave hash, status and escape nibbles, then the escape count, the unit's
// word count and the completion counter's value; the coder's final output
// ring cursors in the last two words
constexpr int kPartBytes = (12 * kEncMaxWaves + 12 + 15) / 16 * 16;
constexpr int kPartWp = kPartBytes / 4 - 2, kPartFl = kPartBytes / 4 - 1;
static_assert(kPartWp >= 3 * kEncMaxWaves + 3, "encoder LDS parts overlap");
constexpr int kRingWords = 4096;       // encoder LDS output ring (u16 words), the most a plan uses
constexpr int kPfU32Max = 8;  // decoder stream prefetch: u32 per lane (16-step blocks)
// word 3 of a raw buffer resource on gfx9 (32-bit data format; stride 0, so
// num_records counts bytes)
constexpr int kBufferFlags = 0x00020000;
constexpr int kMaxDevices = 64;

// Phase timestamps (measurement only; a library built with
// GAANS_PHASE_TIMES, see gaans_debug_phases).  The coder wave takes the
// constant-rate real-time counter (slots 0-11) or the shader clock (slots
// 12-15) into scalar registers at each point, and thread 0 stores its unit's
// slots once, after the unit's counter atomic, so the points add no vector
// registers to the coding loop.  In the default build every call is empty.
struct PhaseBuf {
  uint64_t* __restrict__ p;
  int64_t units;  // units that have slots
};
// The wave's HW_ID register: wave slot (bits 0-3), SIMD (4-5), CU (8-11),
// shader array (12), shader engine (13-14), thread-group slot on the CU
// (16-19).
__device__ __forceinline__ uint32_t hw_id() {
  uint32_t h;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(h));
  return h;
}

struct PhaseClock {
#ifdef GAANS_PHASE_TIMES
  uint64_t t[12] = {}, c12 = 0, c13 = 0, bw = 0, b0 = 0, hw = 0;
  __device__ __forceinline__ void mark(int i) {
    t[i] = __builtin_amdgcn_s_memrealtime();
    if (i == 0) {  // where the coder wave runs: XCC_ID << 32 | HW_ID (SIMD, CU, SE)
      const uint32_t h = hw_id();
      uint32_t xc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xc));
      hw = ((uint64_t)xc << 32) | h;
    }
  }
  __device__ __forceinline__ void cycles(int i) {
    (i == 12 ? c12 : c13) = __builtin_amdgcn_s_memtime();
  }
  // shader cycles the coder spends in its block barriers (slot 14)
  __device__ __forceinline__ void bar_in() { b0 = __builtin_amdgcn_s_memtime(); }
  __device__ __forceinline__ void bar_out() { bw += __builtin_amdgcn_s_memtime() - b0; }
  static constexpr int kPhaseSlots = GAANS_PHASE_SLOTS;
  // slots [lo, hi) of t (and, with lo == 0, the two shader-clock slots)
  __device__ __forceinline__ void store(const PhaseBuf& b, int64_t g, int lo, int hi) const {
    if (b.p != nullptr && g < b.units) {
      uint64_t* d = b.p + g * kPhaseSlots;
#pragma unroll
      for (int i = 0; i < 12; ++i)
        if (i >= lo && i < hi) d[i] = t[i];
      if (lo == 0) {
        d[12] = c12;
        d[13] = c13;
        d[14] = bw;
        d[15] = hw;
      }
    }
  }
  // the thread that wrote the completion word, just after
  __device__ __forceinline__ void store_done(const PhaseBuf& b, int64_t g) const {
    if (b.p != nullptr && g < b.units) b.p[g * kPhaseSlots + 7] = __builtin_amdgcn_s_memrealtime();
  }
  // after an atomic whose return marks the point: wait for it first
  __device__ __forceinline__ void mark_after_loads(int i) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    mark(i);
  }
#else
  __device__ __forceinline__ void mark(int) {}
  __device__ __forceinline__ void cycles(int) {}
  __device__ __forceinline__ void bar_in() {}
  __device__ __forceinline__ void bar_out() {}
  __device__ __forceinline__ void store(const PhaseBuf&, int64_t, int, int) const {}
  __device__ __forceinline__ void store_done(const PhaseBuf&, int64_t) const {}
  __device__ __forceinline__ void mark_after_loads(int) {}
#endif
};

// control block (u32 word indexes; the encoder's counter is a u64 at word 0);
// encoder and decoder fields on separate 64-byte lines
constexpr int kCtrlEncDone = 0;
constexpr int kCtrlEncFin = 8;      // fused encode: units past their look-back
constexpr int kCtrlDecDone = 16;    // u64: units done, status << 32
constexpr int kCtrlEncTicket = 32;  // fused encode: unit numbers handed out

// Look-back word of a unit (fused encode+pack), one u64 in the workspace:
// flag in bits 62-63 (0: nothing yet, 1: the unit's own size, 2: its
// inclusive prefix), status bits in 48-55, payload body u32 words in 0-39
// (the host keeps the worst-case body below 2^36 words).
constexpr uint64_t kLookAgg = 1ull << 62, kLookInc = 2ull << 62;
constexpr int kLookStShift = 48;
constexpr uint64_t kLookValMask = (1ull << 40) - 1;
// a look-back gives up after this many ticks of the 100 MHz real-time
// counter (10 s) and reports GAANS_ST_TIMEOUT: no kernel waits forever
constexpr uint64_t kLookSpinTicks = 1000000000ull;

// ---- wave helpers -----------------------------------------------------------

__device__ __forceinline__ uint32_t lane_rank(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
  for (int off = 32; off > 0; off >>= 1) v |= (uint32_t)__shfl_xor((int)v, off, 64);
  return v;
}

// Sum / OR over the wave's 64 lanes (all active), returned wave-uniform: a
// scan inside each 16-lane row by DPP row shifts (lanes shifted in from
// outside the row read 0), then the four rows' last lanes read out.  The
// cross-lane steps are VALU operations of a few cycles each, where the
// butterfly above waits for the LDS unit's permute six times.
template <bool kOr>
__device__ __forceinline__ uint32_t wave_fold_dpp(uint32_t v) {
  auto step = [&](uint32_t t) { v = kOr ? (v | t) : (v + t); };
  step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true));  // row_shr:1
  step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true));  // row_shr:2
  step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true));  // row_shr:4
  step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true));  // row_shr:8
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
  return kOr ? (r0 | r1 | r2 | r3) : (r0 + r1 + r2 + r3);
}

__device__ __forceinline__ uint64_t wave_incl_scan(uint64_t v, int lane) {
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, off, 64);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(v >> 32), off, 64);
    if (lane >= off) v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// Lanes (of the active ones) where pred holds, as a scalar mask.
__device__ __forceinline__ uint64_t ballot(bool pred) { return __builtin_amdgcn_ballot_w64(pred); }

// Keep a wave-uniform value in a scalar register.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// A buffer resource over the n 4-byte elements at base + 4 first (wave-uniform
// arguments, kept in scalar registers: a resource in vector registers makes
// the compiler loop over the lanes' values).  Loads at byte offsets >= 4 n
// return 0 without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t unit_rsrc(const void* base, int64_t first,
                                                            int64_t n) {
  const uint64_t p = reinterpret_cast<uint64_t>(base) + 4ull * (uint64_t)first;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  const uint64_t bytes = 4ull * (uint64_t)(n > 0 ? n : 0);
  const int nrec = (int)(uint32_t)(bytes < 0xffffffffull ? bytes : 0xffffffffull);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0,
                                           uni(nrec), kBufferFlags);
}

// Section offsets of a prepared table blob, derived on the host from the
// descriptor (M, symbols, sub-blocks), so the kernels address the sections
// without first reading the blob header.
struct BlobRef {
  uint32_t meta_off, ent_off, lut_off, dense_off, total_dense, clut_off, starts_off;
  uint32_t wide_off, wdense_off, wbase_off, total_wide;
};

// The blob header matches the call: magic, table count, size, lookup width
// and the section offsets.  Branch-free, so that the header's words load in
// one round trip.
__device__ __forceinline__ bool tables_ok(const TabHdr& h, uint32_t M, uint32_t bytes,
                                          const BlobRef& r) {
  return (h.magic == kTabMagic) & (h.M == M) & (h.total_bytes == bytes) &
         (h.lut_bits == (uint32_t)kLutBits) & (h.meta_off == r.meta_off) &
         (h.ent_off == r.ent_off) & (h.lut_off == r.lut_off) & (h.dense_off == r.dense_off) &
         (h.total_dense == r.total_dense) & (h.clut_off == r.clut_off) &
         (h.starts_off == r.starts_off) & (h.wide_off == r.wide_off) &
         (h.wdense_off == r.wdense_off) & (h.wbase_off == r.wbase_off) &
         (h.total_wide == r.total_wide);
}

// Blob header in registers (one 64-byte scalar load).
__device__ __forceinline__ TabHdr load_tab_hdr(const uint8_t* tables) {
  return *reinterpret_cast<const TabHdr*>(tables);
}

struct Tabs {
  const TabMeta* __restrict__ gmeta;
  const uint2* __restrict__ gent;
  const uint64_t* __restrict__ glut;
  const uint64_t* __restrict__ gsub;
  const uint4* lmeta;      // {ent_base (LDS-local), nsym, offset, ent_base (global)}
  const uint2* lent;       // encoder: both entry words
  const uint64_t* llut;    // decoder: nt x 256 (wide: nt x kWideSize) lookup entries
  const uint64_t* lsub;    // decoder: sub-blocks of the staged tables
  const uint32_t* lclut;   // decoder, search lookups: bucket entries of all tables
  const uint16_t* lstarts; // decoder, search lookups: symbol starts of all tables
  int t_lo, nt;
  uint32_t sub_first;      // first staged sub-block
  uint32_t sub_n;          // decoder: sub-blocks sub_first .. + sub_n - 1 are in LDS
};

// One pass over the staged metadata (nt), entries (ne) and sub-block 16-byte
// words (nd) with U loads of each kind in flight per thread before the
// stores.  Indexes past a count re-copy its last item, so nothing branches
// (the kinds are compile-time choices; counts are >= 1).
// Copy n 16-byte words global -> LDS with direct-to-LDS loads (gfx950
// global_load_lds_dwordx4: no registers, every load of the copy in flight at
// once): wave w of the NT threads issues the 64-word (1 KB) chunks w, w + W,
// ...; lane i of chunk c moves word 64 c + i to dst + 64 c + i (the LDS
// address is the chunk base, wave-uniform, plus 16 bytes per lane); lanes
// past n are masked off and write nothing.  The data is in LDS once the
// wave's vector-memory counter reaches zero: callers wait for it before the
// barrier that publishes the copy.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;
template <int NT>
__device__ __forceinline__ void copy16_dma(uint4* dst, const uint4* __restrict__ src, uint32_t n,
                                           int tid) {
  constexpr uint32_t W = NT / kLanes;
  const uint32_t lane = (uint32_t)tid & (kLanes - 1);
  for (uint32_t c = (uint32_t)__builtin_amdgcn_readfirstlane(tid >> 6); c * kLanes < n; c += W) {
    const uint32_t i = c * kLanes + lane;
    if (i < n)
      __builtin_amdgcn_global_load_lds((global_void_t*)(src + i), (lds_void_t*)(dst + c * kLanes),
                                       16, 0, 0);
  }
}

template <int NT, bool kEnt, bool kSub>
__device__ __forceinline__ void stage_pass(const Tabs& T, uint4* lmeta, uint2* lent, uint4* lsub,
                                           const uint4* __restrict__ ssrc, uint32_t nt,
                                           uint32_t ne, uint32_t nd, uint32_t base0, int t_lo,
                                           int tid) {
  // loads in flight per thread and kind (fewer for the decoder's larger
  // workgroup, whose waves keep more registers live across the staging)
  constexpr int U = NT >= 384 ? 3 : 4;
  uint32_t items = nt;
  if (kEnt) items = items > ne ? items : ne;
  if (kSub) items = items > nd ? items : nd;
  for (uint32_t b = tid; b < items; b += U * NT) {
    TabMeta mv[U];
    uint2 ev[U];
    uint4 dv[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const uint32_t i = b + k * NT;
      mv[k] = T.gmeta[t_lo + (i < nt ? i : nt - 1)];
      if (kEnt) ev[k] = T.gent[base0 + (i < ne ? i : ne - 1)];
      if (kSub) dv[k] = ssrc[i < nd ? i : nd - 1];
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const uint32_t i = b + k * NT;
      lmeta[i < nt ? i : nt - 1] =
          make_uint4(mv[k].ent_base - base0, mv[k].nsym, (uint32_t)mv[k].offset, mv[k].ent_base);
      if (kEnt) lent[i < ne ? i : ne - 1] = ev[k];
      if (kSub) lsub[i < nd ? i : nd - 1] = dv[k];
    }
  }
}

// Stage tables [t_lo, t_hi) of the blob into LDS (whole workgroup of NT
// threads): the encoder's metadata and entries (lent), or the lookups
// (llut), metadata and, when lsub is given, the tables' sub-blocks.  The
// entries and lookups are copied straight into LDS while the metadata loads
// are in flight; entries, lookups and sub-blocks are 16-byte aligned in the
// blob.
// Entry and sub-block ranges of the staged tables [t_lo, t_hi) (t_lo < M;
// t_lo == t_hi when nothing is staged), read from the blob's metadata.  Every
// load is unconditional, so a kernel can issue them with its other first
// loads.
struct StageBounds {
  uint32_t base0, ent_end, d0, d1;
};

__device__ __forceinline__ StageBounds stage_bounds(const TabMeta* __restrict__ gmeta, int t_lo,
                                                    int t_hi, uint32_t M,
                                                    uint32_t total_blocks) {
  const TabMeta lo = gmeta[t_lo];
  const TabMeta last = gmeta[t_hi > 0 ? t_hi - 1 : 0];
  const uint32_t next = gmeta[(uint32_t)t_hi < M ? t_hi : (int)M - 1].dense_base;
  StageBounds b;
  b.base0 = lo.ent_base;
  b.ent_end = last.ent_base + last.nsym;
  b.d0 = lo.dense_base;
  b.d1 = (uint32_t)t_hi < M ? next : total_blocks;
  return b;
}

// Wide-lookup sub-block range of the staged tables [t_lo, t_hi) from the
// blob's per-table bases (M + 1 of them, so t_hi = M is in range).
__device__ __forceinline__ StageBounds stage_bounds_wide(const uint32_t* __restrict__ wbase,
                                                         int t_lo, int t_hi) {
  StageBounds b;
  b.base0 = 0u;
  b.ent_end = 0u;
  b.d0 = wbase[t_lo];
  b.d1 = wbase[t_hi];
  return b;
}

// LB: lookup entries per table (kLutSize, or kWideSize for the wide lookups)
template <int NT, int LB = kLutSize>
__device__ void stage_tables(Tabs& T, uint4* lmeta, uint2* lent, uint64_t* llut, uint64_t* lsub,
                             const StageBounds& bd, int t_lo, int t_hi, int tid) {
  T.t_lo = t_lo;
  T.nt = t_hi > t_lo ? t_hi - t_lo : 0;
  T.sub_first = 0;
  T.sub_n = 0;
  if (T.nt > 0) {
    const uint32_t nt = (uint32_t)T.nt;
    const uint32_t base0 = bd.base0;
    if (lent) {
      // the entries straight into LDS from the even entry at or below the
      // range's first (16-byte aligned: the blob's entry section is), one
      // round trip however many there are; the metadata rows through
      // registers, their entry bases taken relative to that even entry
      const uint32_t b2 = base0 & ~1u;
      copy16_dma<NT>(reinterpret_cast<uint4*>(lent),
                     reinterpret_cast<const uint4*>(T.gent + b2), (bd.ent_end - b2 + 1u) / 2u,
                     tid);
      stage_pass<NT, false, false>(T, lmeta, nullptr, nullptr, nullptr, nt, 1u, 0u, b2, t_lo, tid);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct-to-LDS copies are in
    } else {
      // lookups and sub-blocks straight into LDS, the metadata rows through
      // registers (they are rewritten)
      const uint4* lut_src = reinterpret_cast<const uint4*>(T.glut + (int64_t)t_lo * LB);
      copy16_dma<NT>(reinterpret_cast<uint4*>(llut), lut_src, nt * (LB / 2), tid);
      const uint32_t d0 = bd.d0;
      const uint32_t d1 = bd.d1;
      if (lsub && d1 > d0) {
        T.sub_first = d0;
        T.sub_n = d1 - d0;
        copy16_dma<NT>(reinterpret_cast<uint4*>(lsub),
                       reinterpret_cast<const uint4*>(T.gsub + (size_t)d0 * kSubSize),
                       (d1 - d0) * (kSubBytes / 16), tid);
      }
      stage_pass<NT, false, false>(T, lmeta, nullptr, nullptr, nullptr, nt, 1u, 0u, base0, t_lo,
                                   tid);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct-to-LDS copies are in
    }
  }
  __syncthreads();
}

// Staged table range of chunk k: all tables, or the chunk's P channels.
__device__ __forceinline__ void stage_range(int nt_cap, int stage_all, int k, int P, int M,
                                            int& t_lo, int& t_hi) {
  t_lo = 0;
  t_hi = 0;
  if (nt_cap > 0) {
    if (stage_all) {
      t_hi = M;
    } else {
      t_lo = k * P;
      t_hi = t_lo + P < M ? t_lo + P : M;
    }
  }
}

// Input modes of the coding kernels.
constexpr int kModeSymbols = 0;   // int32 symbols; indexes given or table = channel
constexpr int kModeLatents = 1;   // fp32 latents, per-channel medians; indexes as above
constexpr int kModeGaussian = 2;  // fp32 latents, per-element means (optional) and scales
static_assert(kModeSymbols == GAANS_MODE_SYMBOLS && kModeLatents == GAANS_MODE_LATENTS &&
                  kModeGaussian == GAANS_MODE_GAUSSIAN,
              "plan modes are the kernel modes");

// Tables of at most kGaussFast + 1 scales are searched in two levels, one
// LDS read each instead of one per halving: the count c of the 8 values
// table[8i + 7] below lb (kept in registers, GaussCoarse; +inf for 8i + 7
// >= L - 1), then the count of table[8c .. 8c + 7] below lb, which is exact
// for a non-decreasing table.  The staged table is padded with +inf from
// entry L - 1 on (the search never reads entry L - 1) to L + 8, past the
// last entry the second level can read (8c + 7 <= L + 6).
constexpr int kGaussFast = 64;
constexpr int kGaussPad = 8;  // +inf entries staged after the table
struct GaussCoarse {
  float v[8];
};
__device__ __forceinline__ GaussCoarse gauss_coarse(const float* tab, int L) {
  GaussCoarse c;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    c.v[i] = L <= kGaussFast + 1 && 8 * i + 7 < L - 1 ? tab[8 * i + 7] : __builtin_inff();
  return c;
}
__device__ __forceinline__ int32_t gauss_index_fast(float lb, const float* tab,
                                                    const GaussCoarse& c) {
  int k = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) k += c.v[i] < lb ? 1 : 0;
  const float4 a = *reinterpret_cast<const float4*>(tab + 8 * k);
  const float4 b = *reinterpret_cast<const float4*>(tab + 8 * k + 4);
  return 8 * k + (a.x < lb) + (a.y < lb) + (a.z < lb) + (a.w < lb) + (b.x < lb) + (b.y < lb) +
         (b.z < lb) + (b.w < lb);
}

// CompressAI's GaussianConditional.build_indexes for one scale s (the
// third-party algorithm, restated in the oracle): lb = max(s, bound) (NaN
// propagates, as torch.max does), index =
// (L - 1) - #{k < L - 1 : lb <= table[k]}.  For a non-decreasing table that is
// #{k < L - 1 : table[k] < lb}, found by a fixed-step binary search over the
// table in LDS (pow2 = the largest power of two <= L - 1); NaN -> L - 1.
__device__ __forceinline__ int32_t gauss_index(float s, const float* tab, int L, int pow2,
                                               float bound, const GaussCoarse& gc) {
  const float lb = s < bound ? bound : s;
  if (L <= kGaussFast + 1) return lb != lb ? L - 1 : gauss_index_fast(lb, tab, gc);
  int pos = 0;
  for (int step = pow2; step > 0; step >>= 1) {
    const int i = pos + step - 1;
    const float t = tab[i < L - 2 ? i : L - 2];
    pos += (pos + step <= L - 1 && t < lb) ? step : 0;
  }
  return lb != lb ? L - 1 : pos;
}

// gauss_index of KP scales at once (in: the scales' bits, out: the
// indexes): the KP searches advance together, so each round's KP table
// reads are in flight at the same time.
template <int KP>
__device__ __forceinline__ void gauss_indexes(int32_t* io, const float* tab, int L, int pow2,
                                              float bound, const GaussCoarse& gc) {
  float lb[KP];
  int pos[KP];
#pragma unroll
  for (int e = 0; e < KP; ++e) {
    const float s = __int_as_float(io[e]);
    lb[e] = s < bound ? bound : s;
    pos[e] = 0;
  }
  if (L <= kGaussFast + 1) {  // uniform
#pragma unroll
    for (int e = 0; e < KP; ++e) pos[e] = gauss_index_fast(lb[e], tab, gc);
#pragma unroll
    for (int e = 0; e < KP; ++e) io[e] = lb[e] != lb[e] ? L - 1 : pos[e];
    return;
  }
  for (int step = pow2; step > 0; step >>= 1) {
#pragma unroll
    for (int e = 0; e < KP; ++e) {
      const int i = pos[e] + step - 1;
      const float t = tab[i < L - 2 ? i : L - 2];
      pos[e] += (pos[e] + step <= L - 1 && t < lb[e]) ? step : 0;
    }
  }
#pragma unroll
  for (int e = 0; e < KP; ++e) io[e] = lb[e] != lb[e] ? L - 1 : pos[e];
}

// Stage the scale table into LDS with the whole workgroup: entries 0 ..
// L - 2, then +inf up to L + kGaussPad (see gauss_index_fast); the caller's
// next barrier publishes it.
template <int NT>
__device__ __forceinline__ void stage_scales(float* dst, const float* __restrict__ src, int L,
                                             int tid) {
  for (int i = tid; i < L + kGaussPad; i += NT) dst[i] = i < L - 1 ? src[i] : __builtin_inff();
}

// ============================================================================
// Encoder
// ============================================================================

struct EncArgs {
  const int32_t* __restrict__ symbols;
  const float* __restrict__ y;
  const float* __restrict__ medians;
  const float* __restrict__ means;        // Gaussian: per element, or NULL
  const float* __restrict__ scales;       // Gaussian: per element
  const float* __restrict__ scale_table;  // Gaussian: L non-decreasing scales
  int32_t n_scales, scales_pow2;
  float scale_bound;
  uint32_t scales_lds;  // LDS byte offset of the staged scale table
  const int32_t* __restrict__ indexes;
  const uint8_t* __restrict__ tables;
  uint32_t M, tables_bytes;
  BlobRef blob;
  int64_t N;
  int32_t K, P, C, chunk_len;
  int32_t S;        // segments per chunk
  int32_t seg_cap;  // most symbols of a unit (escape list slots per unit)
  UDiv div_hw;
  int32_t cap_words;
  int64_t units, header_bytes;  // coding units (B K S)
  int32_t nt_cap, stage_all;
  uint32_t ring_mask;  // output ring words - 1 (a power of two, >= 2 SB kLanes)
  uint32_t* __restrict__ chunk_words;
  uint32_t* __restrict__ index_hash;
  uint32_t* __restrict__ end_off;
  uint64_t* __restrict__ ws_info;
  uint32_t* __restrict__ states;
  uint16_t* __restrict__ words;
  uint2* __restrict__ esc;          // per unit: escape count, escape nibbles
  uint32_t* __restrict__ esc_raw;   // per unit: seg_cap slots, filled from the end
  uint32_t* __restrict__ ctrl;
  uint64_t* __restrict__ info_out;
  // pack fused into the coding kernel (NULL: stage 1 only, k_pack follows):
  // the payload buffer (at least the layout's worst case) and the per-unit
  // look-back words (workspace, zero before the launch and left zero)
  uint8_t* __restrict__ out;
  int64_t out_bytes;
  uint64_t* __restrict__ look;
  uint32_t B;
  // fused: unit numbers from the control block's ticket counter (the grid
  // may not fit the device in one round), else the workgroup index
  uint32_t ticket;
  uint32_t lds_bytes;  // the launch's dynamic LDS
  // several workgroups share a CU: the coder role goes to a wave on the SIMD
  // numbered by the workgroup's slot on the CU
  uint32_t elect;
  PhaseBuf phase;
};

// Encoder LDS layout (bytes): the output ring of `ring` u16 words (a power
// of two chosen by the plan, at least two blocks' worst case) plus one spare
// slot per lane, then the geometry's records, flags and parts
constexpr int enc_ring_bytes(int ring) { return 2 * (ring + kLanes); }

// Encoder geometry for blocks of SB steps (the mappers' lead over the coder
// and the steps between two barriers).
template <int SB, int NM>
struct EncGeom {
  static constexpr int kWaves = NM + 1;  // the coder and NM mappers
  static constexpr int kThreads = kWaves * kLanes;
  // steps per mapper wave and block
  static constexpr int kPer = (SB + NM - 1) / NM;
  static constexpr int kRecBytes = 2 * SB * kLanes * 16;       // two blocks of op records
  static constexpr int kFlagBytes = 16;  // per block parity: steps with escapes (bit per step)
  // [ring][records][flags][parts]: the part after the ring
  static constexpr int kTail = kRecBytes + kFlagBytes + kPartBytes;
};

int enc_fixed_lds(int sb, int ring) {  // the same for either mapper count
  return enc_ring_bytes(ring) + (sb >= 16 ? EncGeom<16, 4>::kTail
                                          : (sb >= 8 ? EncGeom<8, 4>::kTail : EncGeom<4, 4>::kTail));
}

// Payload size of a unit in u32 words: A final states, then the stream's W
// u16 words and the escape section's Z nibbles (4 to a u16 word), padded to
// an even number of u16 words.
__device__ __forceinline__ uint32_t unit_quads(int A, uint32_t W, uint32_t Z) {
  const uint32_t U = W + (Z + 3u) / 4u;
  return (uint32_t)A + (U + (U & 1u)) / 2u;
}

// Encode completion counter: one u64 in the control block, units done in
// bits 0..23, payload body u32 words in bits 24..59, the OR of the units'
// status bits in bits 60..63.  A unit ORs in its status (rarely), waits for
// that and its count stores, then adds 1 | its words << 24; atomics on one
// address take effect in program order, so the unit whose add returns units - 1 done holds the
// payload size and status of the whole launch with no further memory round
// trip.  The host keeps units below 2^24 and the worst-case payload below
// 2^38 bytes, so no field carries into the next.
constexpr int kEncCountBits = 24, kEncStShift = 60;
constexpr uint64_t kEncCountMask = (1ull << kEncCountBits) - 1;
static_assert((GAANS_ST_RANGE | GAANS_ST_INDEX | GAANS_ST_TABLES) < 16,
              "encode status bits fit the completion counter");

// The unit that completed the launch (one thread): payload size and status
// to the workspace and the host's completion word (size and status in one
// 64-bit store, so the host can read it as soon as it lands: no system-wide
// cache write-back), then the counter back to zero for the next launch.
__device__ void encode_finish(const EncArgs& a, uint64_t word) {
  const uint64_t body = 4ull * ((word << (64 - kEncStShift)) >> (64 - kEncStShift + kEncCountBits));
  uint32_t st = (uint32_t)(word >> kEncStShift);
  if (body > 0xffffffffull) st |= GAANS_ST_SIZE;  // unit end offsets are u32
  const uint64_t total = (uint64_t)a.header_bytes + body;
  a.ws_info[0] = total;
  a.ws_info[1] = st;
  if (a.info_out) {
    a.info_out[0] = total;
    a.info_out[1] = st;
    __hip_atomic_store(&a.info_out[2], 1ull | ((uint64_t)st << 1) | (total << 16),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  __hip_atomic_store(reinterpret_cast<uint64_t*>(a.ctrl + kCtrlEncDone), 0ull, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Last workgroup of an encode launch (all threads), after the completion
// word is out: the unit end offsets (payload body bytes up to and including
// each unit) for the pack kernel, kThreads units at a time, the next tile's
// counts loaded before the current tile's scan.  A body past 4 GiB wraps
// here; the completion word carries GAANS_ST_SIZE then, and the pack kernel
// skips a unit whose offsets decrease.
template <int NT>
__device__ void unit_end_offsets(const EncArgs& a, int tid, uint64_t* sh) {
  constexpr int kThreads = NT, kWaves = NT / kLanes;
  const int lane = tid & (kLanes - 1), wv = tid >> 6;
  auto bytes = [&](int64_t g) -> uint64_t {
    const int len = unit_len(g, a.K, a.S, a.N, a.chunk_len);
    const uint32_t W = __hip_atomic_load(&a.chunk_words[g], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t Z = __hip_atomic_load(&a.esc[g].y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return 4ull * unit_quads(len < kLanes ? len : kLanes, W, Z);
  };
  uint64_t carry = 0;
  uint64_t v = tid < a.units ? bytes(tid) : 0ull;
  for (int64_t base = 0; base < a.units; base += kThreads) {
    const int64_t g = base + tid;
    const uint64_t vn = g + kThreads < a.units ? bytes(g + kThreads) : 0ull;
    uint64_t incl = wave_incl_scan(v, lane);
    if (lane == kLanes - 1) sh[wv] = incl;
    __syncthreads();
    uint64_t before = 0, tot = 0;
    for (int w = 0; w < kWaves; ++w) {
      before += w < wv ? sh[w] : 0ull;
      tot += sh[w];
    }
    __syncthreads();
    if (g < a.units) a.end_off[g] = (uint32_t)(incl + before + carry);
    carry += tot;
    v = vn;
  }
}

// Op record of one lane and step (16 bytes):
//   x: start | (65536 - freq) << 16      (identity op: 0)
//   y: division magic of freq            (enc_div)
//   z: shift (enc_shift) | escape << 8 | (freq - 1) << 16
//      (identity op: 15 | 0xffff << 16, so that it never emits)
//   w: escape raw value
// CompressAI's escape split (reference warp_ans_kernel_v2.cu:139-164):
// v = sym - offset; v < 0 -> raw = -2v - 1, v >= maxv -> raw = 2 (v - maxv),
// both coded as the escape bin maxv; raw goes to the escape section as
// n = raw ? msb(raw) / 4 + 1 : 0 nibbles after the count (1 + n nibbles,
// added to znib).  v is computed in 32-bit arithmetic; when sym - offset
// overflows int32 the sign of sym tells the side and raw = 2 (v - maxv)
// (wrapped) is exact whenever raw < 2^32, else the symbol is uncodable.
//
// A mapper wave builds the records of its KP steps of a block together
// (steps t0 + tstep e, e < nvalid; the others are inactive): the table
// numbers, symbols and index hash of all KP steps first, then their table
// metadata reads, then their entry reads, so that each kind of LDS (or L2)
// read is in flight for all KP steps at once rather than one step after the
// other.
template <int kMode, bool kImplicit, bool kLds, int KP>
__device__ __forceinline__ void enc_records(const EncArgs& a, const Tabs& tb, int lane, int t0,
                                            int tstep, int nvalid, int len, int32_t start,
                                            const int32_t* in_a, const int32_t* in_b,
                                            const float* in_m, uint32_t& hash, uint32_t& status,
                                            uint32_t& znib, uint4* rec) {
  bool ok[KP];
  int32_t sym[KP], offset[KP];
  uint32_t ebase[KP], nsym[KP];
#pragma unroll
  for (int e = 0; e < KP; ++e) {
    const int p = lane + kLanes * (t0 + tstep * e);
    const bool act = (e < nvalid) & (p < len);
    int32_t tbi =
        kImplicit ? (int32_t)udiv((uint32_t)unit_pos(start, a.S, p), a.div_hw) : in_b[e];
    const bool bad = act & ((uint32_t)tbi >= a.M);
    ok[e] = act & !bad;
    status |= bad ? GAANS_ST_INDEX : 0u;
    tbi = ok[e] ? tbi : (kLds ? tb.t_lo : 0);
    hash += ok[e] ? index_term((uint32_t)p, (uint32_t)tbi) : 0u;
    if (kMode != kModeSymbols) {
      const float r = rintf(__fsub_rn(__int_as_float(in_a[e]), in_m[e]));
      const bool rng = !(fabsf(r) < 2147483648.0f);
      status |= (ok[e] & rng) ? GAANS_ST_RANGE : 0u;
      sym[e] = (int32_t)(rng ? 0.0f : r);
    } else {
      sym[e] = in_a[e];
    }
    if (kLds) {
      const uint4 m = tb.lmeta[tbi - tb.t_lo];
      ebase[e] = m.x;
      nsym[e] = m.y;
      offset[e] = (int32_t)m.z;
    } else {
      const TabMeta m = tb.gmeta[tbi];
      ebase[e] = m.ent_base;
      nsym[e] = m.nsym;
      offset[e] = m.offset;
    }
  }
  int32_t v[KP];
  bool ovf[KP], esc[KP];
  uint2 ent[KP];
#pragma unroll
  for (int e = 0; e < KP; ++e) {
    v[e] = (int32_t)((uint32_t)sym[e] - (uint32_t)offset[e]);
    const int32_t maxv = (int32_t)nsym[e] - 1;
    ovf[e] = ((sym[e] ^ offset[e]) & (sym[e] ^ v[e])) < 0;
    const bool out = ((uint32_t)v[e] >= (uint32_t)maxv) | ovf[e];
    esc[e] = ok[e] & out;
    const uint32_t at = ebase[e] + (uint32_t)(out ? maxv : v[e]);
    ent[e] = kLds ? tb.lent[at] : tb.gent[at];
  }
#pragma unroll
  for (int e = 0; e < KP; ++e) {
    // escape split
    const uint32_t d = (uint32_t)v[e] - (nsym[e] - 1u);
    const bool lo = ovf[e] ? (sym[e] < 0) : (v[e] < 0);
    status |= (ok[e] & ovf[e] & (lo | (d >= 0x80000000u))) ? GAANS_ST_RANGE : 0u;
    // raw = esc ? (lo ? ~(v << 1) : d << 1) : 0, as bit selects (no branch)
    const uint32_t m_lo = 0u - (uint32_t)lo;
    const uint32_t raw = ((~((uint32_t)v[e] << 1) & m_lo) | ((d << 1) & ~m_lo)) &
                         (0u - (uint32_t)esc[e]);
    const uint32_t nn = raw ? ((31u - (uint32_t)__clz((int)raw)) >> 2) + 1u : 0u;
    znib += esc[e] ? nn + 1u : 0u;
    const uint32_t fr = (ent[e].x >> 16) + 1u;
    const uint32_t sh = enc_shift(fr);
    uint4 r;
    r.x = ok[e] ? ((ent[e].x & 0xffffu) | ((65536u - fr) << 16)) : 0u;
    r.y = ok[e] ? ent[e].y : 1u;
    r.z = (ok[e] ? sh | (ent[e].x & 0xffff0000u) : 0xffff000fu) | (esc[e] ? 256u : 0u);
    r.w = raw;
    rec[e] = r;
  }
}

// The records of a full block whose indexes and values are all in range,
// with the tables in LDS and every table offset at most INT32_MAX - 65535:
// the same records as enc_records, with the escape split computed only for
// the steps that have an escaping lane.  With such offsets, sym - offset
// wraps only to values of at least 65536, so (uint32)(sym - offset) <
// nsym - 1 tests "ordinary" alone.  Returns false, having changed nothing,
// when a lane of the block has an index outside the staged tables or a value
// outside int32 (the caller then maps the block with enc_records); else sets
// bit e of esc_steps for each step e with an escape.
//   x = start | (65535 - (freq - 1)) << 16 = entry word 0 ^ 0xffff0000
//   z = 31 - ffbh(freq - 1): the shift for freq >= 2, and 32 (the freq-1
//       flag) for freq = 1, where ffbh(0) = 0xffffffff; | 256 for an escape;
//       | (freq - 1) << 16 = entry word 0's high half
template <int kMode, bool kImplicit, int KP>
__device__ __forceinline__ bool enc_records_fast(const EncArgs& a, const Tabs& tb, int lane,
                                                 int t0, int tstep, int32_t start,
                                                 const int32_t* in_a, const int32_t* in_b,
                                                 const float* in_m, uint32_t& hash,
                                                 uint32_t& status, uint32_t& znib,
                                                 uint32_t& esc_steps, uint4* rec) {
  int32_t sym[KP];
  uint32_t tbl[KP];
  uint32_t h = 0;
  uint64_t bad = 0;  // lane masks (one compare per step, no bool arithmetic)
#pragma unroll
  for (int e = 0; e < KP; ++e) {
    const int p = lane + kLanes * (t0 + tstep * e);
    const int32_t tbi =
        kImplicit ? (int32_t)udiv((uint32_t)unit_pos(start, a.S, p), a.div_hw) : in_b[e];
    bad |= ballot((uint32_t)(tbi - tb.t_lo) >= (uint32_t)tb.nt);  // staged tables are below M
    tbl[e] = (uint32_t)tbi;
    h += index_term((uint32_t)p, (uint32_t)tbi);
    if (kMode != kModeSymbols) {
      const float r = rintf(__fsub_rn(__int_as_float(in_a[e]), in_m[e]));
      bad |= ballot(!(fabsf(r) < 2147483648.0f));
      sym[e] = (int32_t)r;
    } else {
      sym[e] = in_a[e];
    }
  }
  if (bad != 0ull) return false;
  uint32_t at[KP], v[KP], maxv[KP], off[KP];
  uint64_t om[KP];
#pragma unroll
  for (int e = 0; e < KP; ++e) {
    const uint4 m = tb.lmeta[tbl[e] - tb.t_lo];
    v[e] = (uint32_t)sym[e] - m.z;
    maxv[e] = m.y - 1u;
    off[e] = m.z;
    const bool out = v[e] >= maxv[e];
    om[e] = ballot(out);
    at[e] = m.x + (out ? maxv[e] : v[e]);
  }
  uint32_t es = 0;
#pragma unroll
  for (int e = 0; e < KP; ++e) {
    const uint2 ent = tb.lent[at[e]];
    // enc_shift: 31 - clz(2 (freq - 1) + 1) (never of zero), from the
    // entry's (freq - 1) << 16 | start
    uint32_t lz;
    asm("v_ffbh_u32 %0, %1" : "=v"(lz) : "v"((ent.x >> 15) | 1u));
    rec[e] = make_uint4(ent.x ^ 0xffff0000u, ent.y, (31u - lz) | (ent.x & 0xffff0000u), 0u);
    if (om[e] != 0ull) {
      // the escape split of enc_records for this step's escaping lanes
      const bool esc = (om[e] >> lane) & 1ull;
      const int32_t sv = sym[e], ov = (int32_t)off[e], vv = (int32_t)v[e];
      const bool ovf = ((sv ^ ov) & (sv ^ vv)) < 0;
      const uint32_t d = v[e] - maxv[e];
      const bool lo = ovf ? (sv < 0) : (vv < 0);
      status |= (esc & ovf & (lo | (d >= 0x80000000u))) ? GAANS_ST_RANGE : 0u;
      const uint32_t m_lo = 0u - (uint32_t)lo;
      const uint32_t raw = ((~(v[e] << 1) & m_lo) | ((d << 1) & ~m_lo)) & (0u - (uint32_t)esc);
      const uint32_t nn = raw ? ((31u - (uint32_t)__clz((int)raw)) >> 2) + 1u : 0u;
      znib += esc ? nn + 1u : 0u;
      rec[e].z |= esc ? 256u : 0u;
      rec[e].w = raw;
      es |= 1u << e;
    }
  }
  esc_steps = es;
  hash += h;
  return true;
}

// Encoder LDS ring: ring_mask + 1 words (a power of two) and one spare slot
// per lane (where a step's lanes that emit nothing store).
// Words [wp, fl) to the staging slot: the ones before the first multiple
// of 4 and after the last one word per lane, the rest 4 words (8 bytes) per
// lane (the ring's size is a multiple of 4 words, so such a group never
// straddles its wrap; the slot is 16-byte aligned).
__device__ __forceinline__ void ring_flush(uint16_t* __restrict__ wbuf, const uint16_t* ring,
                                           int wp, int fl, int lane, uint32_t ring_mask) {
  const int a0 = (wp + 3) & ~3, a1 = fl & ~3;
  if (a0 >= a1) {  // uniform: fewer than one aligned group
    for (int pos = wp + lane; pos < fl; pos += kLanes) wbuf[pos] = ring[pos & ring_mask];
    return;
  }
  if (lane < a0 - wp) wbuf[wp + lane] = ring[(wp + lane) & ring_mask];
  if (lane < fl - a1) wbuf[a1 + lane] = ring[(a1 + lane) & ring_mask];
  const uint2* r64 = reinterpret_cast<const uint2*>(ring);
  uint2* w64 = reinterpret_cast<uint2*>(wbuf);
  const uint32_t m64 = ring_mask >> 2;
  for (int i = (a0 >> 2) + lane; i < (a1 >> 2); i += kLanes) w64[i] = r64[(uint32_t)i & m64];
}

// The ring holds the words [wp, fl) (positions mod the ring size).  The coder
// flushes it at the start of a block when fewer than SB * kLanes slots are
// free (a step emits at most one word per lane), so the steps need no check.
// A lane emits when x >= freq << 16, i.e. (x >> 16) > freq - 1 (z's high
// half): one compare of the two high halves.  Every lane stores, the ones
// that emit nothing to their spare slot (spare = ring_mask + 1 + lane,
// computed once per wave): selects on the compare rather than an
// exec-masked branch, which costs three scalar instructions more per step
// and keeps consecutive steps from interleaving.  (With the spare slot
// computed here the compiler turned the selects back into a branch.)
__device__ __forceinline__ void emit_words(uint32_t z, uint32_t& x, uint16_t* ring, int& wp,
                                           uint32_t spare, uint32_t ring_mask) {
  const bool emit = (x >> 16) > (z >> 16);
  const uint64_t m = ballot(emit);
  wp = uni(wp - __popcll(m));
  // wp + the number of emitting lanes below this one
  const uint32_t pos = (uint32_t)__builtin_amdgcn_mbcnt_hi(
      (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)wp));
  ring[emit ? pos & ring_mask : spare] = (uint16_t)x;
  x = emit ? x >> 16 : x;
}

// main rANS op: x' = ((x / freq) << 16) + x % freq + start = x + start + q (65536 - freq)
// (for freq = 1 too: q = x < 2^16, x' = x 2^16 + start)
__device__ __forceinline__ uint32_t enc_apply(uint32_t x, uint4 r) {
  const uint32_t q = enc_div(x, r.y, r.z);
  return __umul24(q, r.x >> 16) + x + (r.x & 0xffffu);
}

// Escapes of one step into the unit's escape list: slots are taken from the
// end of the list, highest lane first, so that the list, read forwards, is in
// position order (the coder walks the steps last to first).
__device__ __forceinline__ void enc_escapes(uint32_t z, uint32_t raw, uint32_t* __restrict__ list,
                                            int& cnt, int lane) {
  const bool esc = (z & 256u) != 0u;
  const uint64_t em = ballot(esc);
  const int above = __popcll(lane < 63 ? em >> (lane + 1) : 0ull);
  if (esc) list[-1 - (cnt + above)] = raw;
  cnt = uni(cnt + __popcll(em));
}

// Escape section of a unit (NT threads of a workgroup): entry i (position
// order, raw value lst[i], E entries) is the count n then the n nibbles of
// raw, at nibble offset o_i = sum of (1 + n) over the entries before it.
// Escape word j is the u16 at U - 1 - j of the unit's U u16 words after its
// states (w32: those words as n32 = U / 2 u32), so the nibbles [8m, 8m + 8)
// (escape words 2m, 2m + 1) form the u32 at n32 - 1 - m with its halves
// swapped.  Entries share words: they are OR-ed into zeros, which the caller
// has stored (and waited for) before the barrier that precedes this call.
// wtot: NT / 64 u32 of LDS.
template <int NT>
__device__ void pack_escapes(const uint32_t* __restrict__ lst, uint32_t E, uint32_t* w32,
                             int64_t n32, int tid, uint32_t* wtot) {
  constexpr int kW = NT / kLanes;
  const int wv = tid >> 6, lane = tid & (kLanes - 1);
  uint32_t carry = 0;
  for (uint32_t i0 = 0; i0 < E; i0 += NT) {
    const uint32_t i = i0 + tid;
    const uint32_t raw = i < E ? lst[i] : 0u;
    const uint32_t n = raw ? ((31u - (uint32_t)__clz((int)raw)) >> 2) + 1u : 0u;
    const uint32_t c = i < E ? n + 1u : 0u;
    uint32_t incl = c;
    for (int off = 1; off < kLanes; off <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, off, kLanes);
      if (lane >= off) incl += o;
    }
    if (lane == kLanes - 1) wtot[wv] = incl;
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (int w = 0; w < kW; ++w) {
      before += w < wv ? wtot[w] : 0u;
      total += wtot[w];
    }
    __syncthreads();
    const uint32_t o = carry + before + incl - c;
    carry += total;
    const uint64_t v = ((uint64_t)n | ((uint64_t)raw << 4)) << (4 * (o & 7u));
    const int64_t m = o >> 3;
    const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    if (lo && m < n32)
      __hip_atomic_fetch_or(&w32[n32 - 1 - m], (lo >> 16) | (lo << 16), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    if (hi && m + 1 < n32)
      __hip_atomic_fetch_or(&w32[n32 - 2 - m], (hi >> 16) | (hi << 16), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The 16 fixed header words (thread i < 16 writes word i) and the zero
// padding after the unit tables (NT threads).
template <int NT>
__device__ __forceinline__ void write_fixed_header(uint32_t* hdr, int tid, uint32_t B,
                                                   uint32_t N, uint32_t C, uint32_t P,
                                                   uint32_t K, uint32_t chunk_len, uint32_t M,
                                                   uint32_t S, uint32_t dig_lo, uint32_t dig_hi,
                                                   int64_t units, int64_t header_bytes) {
  if (tid < kFixedWords) {
    uint32_t w = 0;
    switch (tid) {
      case 0: w = kMagic; break;
      case 1: w = kVersion; break;
      case 2: w = B; break;
      case 3: w = N; break;
      case 4: w = C; break;
      case 5: w = P; break;
      case 6: w = K; break;
      case 7: w = chunk_len; break;
      case 8: w = M; break;
      case 9: w = kParams; break;
      case 10: w = dig_lo; break;
      case 11: w = dig_hi; break;
      case 12: w = S; break;
      default: w = 0; break;
    }
    hdr[tid] = w;
  }
  for (int64_t j = kFixedWords + 2 * units + tid; j < header_bytes / 4; j += NT) hdr[j] = 0;
}

// Sum over the wave's 64 lanes of values below 2^40 (a 24-bit low part and
// the rest, each summed without overflow).
__device__ __forceinline__ uint64_t wave_sum40(uint64_t v) {
  const uint32_t lo = wave_fold_dpp<false>((uint32_t)v & 0xffffffu);
  const uint32_t hi = wave_fold_dpp<false>((uint32_t)(v >> 24));
  return (uint64_t)lo + ((uint64_t)hi << 24);
}

// Decoupled look-back of unit g (one whole wave): the exclusive prefix of
// the payload body (u32 words) and the OR of the status bits of units
// 0 .. g - 1.  Lane i of window r reads the look-back word of unit
// j - 64 r - i; kLookWindows windows are read per round trip (all the loads
// in flight together) and taken in order: a window counts when every unit up
// to the nearest one with an inclusive prefix has published its size (the
// prefix is then that inclusive value plus the sizes after it), or when all
// 64 have sizes and none a prefix (the next window follows).  A window with a
// unit that has published nothing is read again (with the ones behind it).
// The words are agent-scope atomics: only their own values are exchanged, so
// relaxed loads suffice.  After kLookSpinTicks the unit stops waiting and
// reports GAANS_ST_TIMEOUT (its prefix is then at most the true one, so its
// copy stays in bounds).
constexpr int kLookWindows = 4;
__device__ __forceinline__ uint64_t look_back(const uint64_t* look, int64_t g, int lane,
                                              uint32_t& st) {
  uint64_t excl = 0;
  int64_t j = g - 1;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  while (j >= 0) {
    uint64_t v[kLookWindows];
#pragma unroll
    for (int r = 0; r < kLookWindows; ++r) {
      const int64_t p = j - kLanes * r - lane;
      v[r] = kLookInc;  // before unit 0: an inclusive prefix of zero
      if (p >= 0) v[r] = __hip_atomic_load(&look[p], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    bool done = false, stalled = false;
#pragma unroll
    for (int r = 0; r < kLookWindows; ++r) {
      if (!done && !stalled) {  // uniform
        const uint32_t f = (uint32_t)(v[r] >> 62);
        const uint64_t inc = ballot(f == 2u), none = ballot(f == 0u);
        // lanes up to and including the nearest inclusive prefix (all without one)
        const uint64_t span = inc ? ((inc & (0ull - inc)) << 1) - 1ull : ~0ull;
        if ((none & span) == 0ull) {
          const uint64_t w = ((span >> lane) & 1ull) ? v[r] : 0ull;
          excl += wave_sum40(w & kLookValMask);
          st |= wave_fold_dpp<true>((uint32_t)(w >> kLookStShift) & 0xffu);
          if (inc) done = true;
          else j -= kLanes;
        } else {
          stalled = true;
        }
      }
    }
    if (done) break;
    if (stalled) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > kLookSpinTicks) {
        st |= GAANS_ST_TIMEOUT;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return excl;
}

// Completion of an encode launch (one thread): payload size and status to
// the workspace and, when given, the caller's info words, the completion
// word last (size and status in one 64-bit store, so the host can read it as
// soon as it lands: no system-wide cache write-back).
__device__ __forceinline__ void encode_complete(const EncArgs& a, uint64_t total, uint32_t st) {
  a.ws_info[0] = total;
  a.ws_info[1] = st;
  if (a.info_out) {
    a.info_out[0] = total;
    a.info_out[1] = st;
    __hip_atomic_store(&a.info_out[2], 1ull | ((uint64_t)st << 1) | (total << 16),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Pack fused into the coding kernel (all NT threads of unit g's workgroup,
// after the barrier that publishes the unit's parts): the first mapper wave
// publishes the unit's size, looks back for its offset and publishes its
// inclusive prefix; the unit with the last number writes the completion word
// right away, and the last unit past its look-back clears the look-back
// words and counters for the next launch.  Then the workgroup writes the
// unit's header entries (unit 0 also the fixed header), its final states
// (coder lanes), its words -- from the LDS ring, and from the staging slot
// for the part flushed earlier -- and its escape section.  Replaces the
// separate pack kernel (reference warp_ans_kernel_v2.cu:274-296).
template <int NT, int kWaves>
__device__ void fused_pack(const EncArgs& a, int64_t g, int tid, int lane, int wid, int A,
                           uint32_t x, const uint32_t* part, const uint16_t* ring,
                           uint32_t ring_mask, const uint16_t* __restrict__ wbuf, uint64_t* scr,
                           uint32_t dig_lo, uint32_t dig_hi, uint32_t* stg, uint32_t stg_bytes,
                           PhaseClock& pc) {
  uint32_t hs = 0, ss = 0, zs = 0;
  for (int w = 0; w < kWaves; ++w) {
    hs += part[w];
    ss |= part[kWaves + w];
    zs += part[2 * kWaves + w];
  }
  const uint32_t E = part[3 * kWaves];
  const uint32_t W = part[3 * kWaves + 1];
  const int wp = (int)part[kPartWp], fl = (int)part[kPartFl];
  const uint64_t q = unit_quads(A, W, zs);  // this unit's u32 words
  const int cap = a.cap_words;
  // The words flushed to the staging slot, [fl, cap), from the position f0
  // of a 16-byte boundary (the slot is 16-byte aligned and cap a multiple of
  // 8 words): copied straight into LDS by the other waves while the first
  // mapper wave looks back (most units wait there for the slowest unit
  // before them), every load of the copy in flight at once, so that after it
  // the copy only writes to HBM.  Read from the slot directly when they do
  // not fit.
  const int f0 = fl & ~7;
  const uint32_t n16 = (uint32_t)(cap - f0) >> 3;
  const bool staged = n16 * 16u <= stg_bytes;  // uniform
  if (wid != 1 && staged && n16 > 0) {
    // every wave but the first mapper wave, numbered densely
    const int t2 = tid < kLanes ? tid : tid - kLanes;
    copy16_dma<NT - kLanes>(reinterpret_cast<uint4*>(stg),
                            reinterpret_cast<const uint4*>(wbuf + f0), n16, t2);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // in LDS before the barrier
  }
  if (wid == 1) {
    pc.mark(5);
    if (g > 0 && lane == 0)
      __hip_atomic_store(&a.look[g], kLookAgg | ((uint64_t)ss << kLookStShift) | q,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t st = ss;
    const uint64_t excl = look_back(a.look, g, lane, st);
    pc.mark_after_loads(6);
    if (lane == 0) {
      __hip_atomic_store(&a.look[g], kLookInc | ((uint64_t)(st & 0xffu) << kLookStShift) |
                                         (excl + q),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      scr[0] = excl;
      pc.store(a.phase, g, 5, 7);
      if (g == a.units - 1) {
        const uint64_t body = 4ull * (excl + q);
        // unit end offsets are u32; a total past the buffer (look-back words
        // not zeroed, against the contract) is reported the same way
        if (body > 0xffffffffull || (uint64_t)a.header_bytes + body > (uint64_t)a.out_bytes)
          st |= GAANS_ST_SIZE;
        encode_complete(a, (uint64_t)a.header_bytes + body, st);
        pc.store_done(a.phase, g);
      }
    }
    // the last unit past its look-back: no unit reads look-back words any
    // more, so they and the counters are cleared for the next launch
    uint32_t fin = 0;
    if (lane == 0)
      fin = __hip_atomic_fetch_add(a.ctrl + kCtrlEncFin, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    fin = (uint32_t)__builtin_amdgcn_readfirstlane((int)fin);
    if ((int64_t)fin == a.units - 1) {
      for (int64_t p = lane; p < a.units; p += kLanes)
        __hip_atomic_store(&a.look[p], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lane == 0) {
        __hip_atomic_store(a.ctrl + kCtrlEncFin, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.ctrl + kCtrlEncTicket, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (tid == 0) pc.store(a.phase, g, 0, 5);  // the coder wave's points
  __syncthreads();
  pc.mark(8);  // the unit's payload offset is known
  const uint64_t excl = scr[0];
  const int64_t off = a.header_bytes + 4 * (int64_t)excl;
  if (off + 4 * (int64_t)q > a.out_bytes) return;  // uniform; the host sizes out for the worst case
  uint32_t* hdr = reinterpret_cast<uint32_t*>(a.out);
  if (tid == 0) {
    hdr[kFixedWords + g] = (uint32_t)(4ull * (excl + q));
    hdr[kFixedWords + a.units + g] = hs;
  }
  if (g == 0)
    write_fixed_header<NT>(hdr, tid, a.B, (uint32_t)a.N, (uint32_t)a.C, (uint32_t)a.P,
                           (uint32_t)a.K, (uint32_t)a.chunk_len, a.M, (uint32_t)a.S, dig_lo,
                           dig_hi, a.units, a.header_bytes);
  uint32_t* d32 = reinterpret_cast<uint32_t*>(a.out + off);
  if (wid == 0 && lane < A) d32[lane] = x;
  // u16 words after the states: stream, pad, escape words (zero here)
  uint32_t U16 = W + (zs + 3u) / 4u;
  U16 += U16 & 1u;
  const int64_t n32 = U16 / 2;
  uint32_t* w32 = d32 + A;
  const uint16_t* stg16 = reinterpret_cast<const uint16_t*>(stg);
  if (staged) {
    for (int j = tid; j < (int)n32; j += NT) {
      const int p0 = wp + 2 * j, p1 = p0 + 1;
      uint32_t lo = 0, hi = 0;
      if (p0 < cap) lo = p0 < fl ? ring[p0 & ring_mask] : stg16[p0 - f0];
      if (p1 < cap) hi = p1 < fl ? ring[p1 & ring_mask] : stg16[p1 - f0];
      w32[j] = lo | (hi << 16);
    }
  } else {
    // from the slot in global memory: kPackBatch words' loads in flight per
    // thread before their stores (a store may alias a later load for the
    // compiler, which then keeps each load behind the store before it)
    constexpr int kPackBatch = 8;
    for (int j0 = tid; j0 < (int)n32; j0 += NT * kPackBatch) {
      uint32_t v[kPackBatch];
#pragma unroll
      for (int u = 0; u < kPackBatch; ++u) {
        const int p0 = wp + 2 * (j0 + u * NT), p1 = p0 + 1;
        uint32_t lo = 0, hi = 0;
        if (p0 < cap) lo = p0 < fl ? ring[p0 & ring_mask] : wbuf[p0];
        if (p1 < cap) hi = p1 < fl ? ring[p1 & ring_mask] : wbuf[p1];
        v[u] = lo | (hi << 16);
      }
#pragma unroll
      for (int u = 0; u < kPackBatch; ++u)
        if (j0 + u * NT < (int)n32) w32[j0 + u * NT] = v[u];
    }
  }
  pc.mark(9);  // the words' stores are issued
  if (E > 0) {  // uniform
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    pack_escapes<NT>(a.esc_raw + g * (int64_t)a.seg_cap + (a.seg_cap - E), E, w32, n32, tid,
                     reinterpret_cast<uint32_t*>(scr + 2));
  }
  pc.mark_after_loads(10);  // every store of the coder wave has completed
  if (tid == 0) pc.store(a.phase, g, 8, 11);
}

template <int kMode, bool kImplicit, int SB, int NM>
__global__ __launch_bounds__((NM + 1) * kLanes) void k_encode(EncArgs a) {
  using G = EncGeom<SB, NM>;
  constexpr int kEncMappers = NM;
  constexpr int kWaves = G::kWaves, kThreads = G::kThreads;
  constexpr int kPer = G::kPer;
  // Who lists the escapes: with eight mappers (a CU to each workgroup) the
  // first mapper wave, off the coder's chain (2160x3840 latent encode 95 ->
  // 89 us, hyperprior y 45 -> 44 us at P=16); else the coder, since with
  // four mappers and several workgroups per CU the mappers have no time to
  // spare (batch-64 uniform 67 -> 72 us with the listing moved), and the
  // latents' mappers, which quantize, neither (512x768 latent 17.7 -> 18.1
  // us).
  constexpr bool kMList = NM == 8 && kMode != kModeLatents;
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* ring = reinterpret_cast<uint16_t*>(smem);
  const uint32_t ring_mask = a.ring_mask;  // ring words - 1
  const uint32_t ring_bytes = (uint32_t)enc_ring_bytes((int)ring_mask + 1);
  uint4* recs = reinterpret_cast<uint4*>(smem + ring_bytes);
  uint32_t* eflag = reinterpret_cast<uint32_t*>(smem + ring_bytes + G::kRecBytes);
  uint32_t* part = eflag + G::kFlagBytes / 4;  // per-wave hash, status, escape nibbles
  uint4* lmeta = reinterpret_cast<uint4*>(smem + ring_bytes + G::kTail);
  uint2* lent = reinterpret_cast<uint2*>(smem + ring_bytes + G::kTail + 16 * a.nt_cap);
  float* scl = reinterpret_cast<float*>(smem + a.scales_lds);  // Gaussian: scale table

  const int lane = (int)threadIdx.x & (kLanes - 1);
  const int hw_wave = uni((int)threadIdx.x >> 6);
  PhaseClock pc;
  pc.mark(0);
  // the table blob's header does not depend on the unit: its load is in
  // flight while the unit number is fetched
  const TabHdr th = load_tab_hdr(a.tables);
  const bool fused = a.out != nullptr;  // uniform: pack fused into this kernel
  const bool ticket = fused && a.ticket;
  const uint32_t hwid = hw_id();
  if (a.elect | ticket) {
    if (a.elect && lane == 0) part[hw_wave] = (hwid >> 4) & 3u;  // this wave's SIMD
    // Unit number from the launch's ticket counter, in the order the
    // workgroups start: a unit's look-back only waits on units with lower
    // numbers, which have started and run without waiting on it, so every
    // wait ends whatever order or residency the hardware gives the grid.
    // (When the whole grid fits on the device at once the host sets no
    // ticket and the unit is the workgroup index: every unit can be resident
    // together, so a unit never waits on one that cannot start -- and the
    // one atomic all workgroups would take first costs about 6 us at 768.)
    if (ticket && threadIdx.x == 0)
      eflag[2] = __hip_atomic_fetch_add(a.ctrl + kCtrlEncTicket, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  }
  // Wave roles: the coder is role 0, the mappers 1 .. NM.  Several
  // workgroups on one CU each put their coder on the SIMD numbered by their
  // slot on the CU (HW_ID's thread-group field), when one of their waves is
  // there: the coders then have SIMDs of their own, where the hardware's
  // placement sometimes put two on one SIMD (the younger then got about a
  // quarter fewer issue cycles).  Roles are a permutation of the waves, and
  // the thread index below follows the role, so cooperative loops are
  // unchanged.
  int coder = 0;
  if (a.elect) {
    const uint32_t want = (hwid >> 16) & 3u;
    for (int w = kWaves - 1; w >= 0; --w)
      coder = (uint32_t)uni((int)part[w]) == want ? w : coder;
  }
  const int wid = uni(hw_wave == coder ? 0 : (hw_wave < coder ? hw_wave + 1 : hw_wave));
  const int tid = wid * kLanes + lane;
  int64_t g = blockIdx.x;
  if (ticket) {
    // a counter that did not start at zero (a control block shared or not
    // zeroed, against the contract) still gives every unit number once, in
    // range; the look-backs then end by their time limit
    const uint32_t t = (uint32_t)uni((int)eflag[2]);
    g = t < (uint64_t)a.units ? t : t % (uint32_t)a.units;
  }
  int64_t row;
  int32_t start;
  int len, k;
  unit_range(g, a.K, a.S, a.N, a.chunk_len, row, start, len, k);
  const int T = (len + kLanes - 1) / kLanes;
  const int A = len < kLanes ? len : kLanes;
  const int nblk = (T + SB - 1) / SB;
  uint16_t* __restrict__ wbuf = a.words + g * a.cap_words;
  int wp = a.cap_words;  // coder: wave-uniform write cursor (backwards)
  int fl = a.cap_words;  // coder: words at [fl, cap) are already in wbuf
  uint32_t x = kStateLow;
  uint32_t hash = 0, status = 0, znib = 0;
  int n_esc = 0;  // escapes listed so far (by the coder, or the first mapper wave)
  uint32_t* __restrict__ esc_list = a.esc_raw + g * a.seg_cap + a.seg_cap;

  if (tid < 2) eflag[tid] = 0u;  // visible after the staging barrier
  int t_lo, t_hi;
  stage_range(a.nt_cap, a.stage_all, k, a.P, (int)a.M, t_lo, t_hi);
  const TabMeta* __restrict__ gmeta = reinterpret_cast<const TabMeta*>(a.tables + a.blob.meta_off);
  // the staged range's metadata in the same round trip as the blob header
  // (the metadata lies in the blob whatever its content and is used only
  // when the header check passes)
  const StageBounds bd = stage_bounds(gmeta, t_lo, t_hi, a.M, a.blob.total_dense);
  __builtin_amdgcn_sched_barrier(0);
  Tabs tb;
  tb.gmeta = gmeta;
  tb.gent = reinterpret_cast<const uint2*>(a.tables + a.blob.ent_off);
  tb.glut = nullptr;
  tb.gsub = nullptr;
  tb.lmeta = lmeta;
  tb.lent = lent;
  tb.llut = nullptr;
  tb.lsub = nullptr;
  // mapper wave w (1..kEncMappers) owns steps u = w - 1 + kEncMappers e of every block
  // (steps a wave does not own keep these zeros)
  int32_t ca[kPer] = {}, cb[kPer] = {}, na[kPer] = {}, nb[kPer] = {};
  float cm[kPer] = {}, nm[kPer] = {};
  // The unit's inputs as buffer resources over its len positions: a load's
  // address is the lane's constant byte offset plus the step's (one add, no
  // 64-bit address arithmetic per load), and lanes past the unit's end read
  // 0 (their results are masked).
  const void* in_a_ptr = kMode == kModeSymbols ? (const void*)a.symbols : (const void*)a.y;
  const void* in_b_ptr = kMode == kModeGaussian ? (const void*)a.scales : (const void*)a.indexes;
  const bool has_b = kMode == kModeGaussian || !kImplicit;
  const bool has_m = kMode == kModeGaussian && a.means != nullptr;
  // positions start .. start + span - 1 of the row hold the unit's steps
  // (every S-th step of the chunk from the unit's first)
  const int span = len > 0 ? unit_pos(start, a.S, len - 1) + 1 - start : 0;
  const __amdgpu_buffer_rsrc_t rin_a = unit_rsrc(in_a_ptr, row + start, span);
  const __amdgpu_buffer_rsrc_t rin_b = unit_rsrc(has_b ? in_b_ptr : in_a_ptr, row + start,
                                                 has_b ? span : 0);
  const __amdgpu_buffer_rsrc_t rin_m = unit_rsrc(has_m ? (const void*)a.means : in_a_ptr,
                                                 row + start, has_m ? span : 0);
  const int lane4 = 4 * lane;
  auto load_block = [&](int j, int32_t* ia, int32_t* ib, float* im) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int u = (wid - 1) + kEncMappers * e;
      if (SB % kEncMappers != 0 && u >= SB) break;
      // the range check covers the vector offset only (not a scalar one),
      // so the step's offset is added to the lane's
      const int vo = lane4 + uni(4 * kLanes * a.S * (j * SB + u));
      ia[e] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rin_a, vo, 0, 0);
      if (kMode == kModeGaussian) {
        im[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin_m, vo, 0, 0));
        // the index is found from the scale when the block is mapped
        ib[e] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rin_b, vo, 0, 0);
      } else {
        if (kMode == kModeLatents) {
          int p = lane + kLanes * (j * SB + u);
          p = p < len ? p : len - 1;  // the median's channel stays in the chunk
          im[e] = a.medians[udiv((uint32_t)unit_pos(start, a.S, p), a.div_hw)];
        } else {
          im[e] = 0.0f;
        }
        ib[e] = kImplicit ? 0 : (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rin_b, vo, 0, 0);
      }
    }
  };
  // the mappers' first two blocks of inputs need neither the table check nor
  // the tables: they are in flight while the tables are staged
  if (wid != 0 && nblk > 0) {
    load_block(nblk - 1, ca, cb, cm);
    if (nblk > 1) load_block(nblk - 2, na, nb, nm);
  }
  if (wid == 0) pc.mark_after_loads(1);  // table header and metadata are in
  const bool tab = tables_ok(th, a.M, a.tables_bytes, a.blob);  // uniform
  const bool offsets_safe = (th.flags & kTabOffsetsSafe) != 0;
  if (!tab) status |= GAANS_ST_TABLES;
  if (tab) {
    if (kMode == kModeGaussian) stage_scales<kThreads>(scl, a.scale_table, a.n_scales, tid);
    stage_tables<kThreads>(tb, lmeta, lent, nullptr, nullptr, bd, t_lo, t_hi, tid);
    if (wid == 0) pc.mark(2);
    // the scale table's coarse level, after the staging barrier
    GaussCoarse gc{};
    if (kMode == kModeGaussian && wid != 0) gc = gauss_coarse(scl, a.n_scales);

    // this wave's steps per block: u = wid - 1 + kEncMappers e < SB
    const int nvalid = SB % kEncMappers == 0 ? kPer : (SB - wid + kEncMappers) / kEncMappers;
    // the block's records into the LDS slot of block j, and its steps with
    // escapes into the block's flag word
    auto put_records = [&](int j, const uint4* r, bool fast, uint32_t esc_steps)
                           __attribute__((always_inline)) {
      uint4* dst = recs + (j & 1) * SB * kLanes;
      uint32_t eb = 0;
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const int u = (wid - 1) + kEncMappers * e;
        if (SB % kEncMappers != 0 && u >= SB) break;
        dst[u * kLanes + lane] = r[e];
        if (fast) eb |= ((esc_steps >> e) & 1u) << u;
        else eb |= ballot((r[e].z & 256u) != 0u) != 0ull ? 1u << u : 0u;
      }
      if (eb != 0u && lane == 0)
        __hip_atomic_fetch_or(&eflag[j & 1], eb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    auto map_steps = [&](int j, auto lds_tag) __attribute__((always_inline)) {
      constexpr bool kLds = decltype(lds_tag)::value;
      uint4 r[kPer];
      enc_records<kMode, kImplicit, kLds, kPer>(a, tb, lane, j * SB + wid - 1, kEncMappers,
                                                nvalid, len, start, ca, cb, cm, hash, status,
                                                znib, r);
      put_records(j, r, false, 0u);
    };
    auto map_block = [&](int j) __attribute__((always_inline)) {
      if (kMode == kModeGaussian)
        gauss_indexes<kPer>(cb, scl, a.n_scales, a.scales_pow2, a.scale_bound, gc);
      // A full block first tries the fast path, which checks by itself that
      // every table is staged and every value in range (and changes nothing
      // when it declines), so the check below runs only for the rest.
      if (tb.nt > 0 && offsets_safe && nvalid == kPer && (j + 1) * SB * kLanes <= len) {
        uint4 r[kPer];
        uint32_t esc_steps = 0;
        if (enc_records_fast<kMode, kImplicit, kPer>(a, tb, lane, j * SB + wid - 1, kEncMappers,
                                                     start, ca, cb, cm, hash, status, znib,
                                                     esc_steps, r)) {
          put_records(j, r, true, esc_steps);
          return;
        }
      }
      // LDS tables for the whole block when every active lane's table is staged
      bool lds = tb.nt > 0;
      if (!kImplicit && lds) {
        bool outside = false;
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
          const int u = (wid - 1) + kEncMappers * e;
          outside |= u < SB && lane + kLanes * (j * SB + u) < len &&
                     (uint32_t)(cb[e] - tb.t_lo) >= (uint32_t)tb.nt;
        }
        lds = ballot(outside) == 0;
      }
      if (lds) map_steps(j, std::true_type{});
      else map_steps(j, std::false_type{});
    };

    // The coder and the mappers run separate code (the wave role is uniform
    // per wave) that meets at the same barriers: one before the first block
    // and one per block.  Keeping the roles apart also keeps the mappers'
    // loads in flight out of the coder's wait bookkeeping.
    if (wid == 0) {
      // The coder's chain of dependent steps bounds the block loop; its
      // instructions go first when mapper waves of this or another
      // workgroup on the CU compete for the same SIMD.
      __builtin_amdgcn_s_setprio(3);
      const uint32_t spare = ring_mask + 1u + (uint32_t)lane;
      __syncthreads();
      pc.mark(3);
      pc.cycles(12);
      for (int j = nblk - 1; j >= 0; --j) {
        // coder: steps of block j, last to first
        if (fl - wp > (int)ring_mask + 1 - SB * kLanes) {
          ring_flush(wbuf, ring, wp, fl, lane, ring_mask);
          fl = wp;
        }
        const uint4* src = recs + (j & 1) * SB * kLanes;
        // steps of the block with escapes when the coder lists them; cleared
        // for block j - 2
        const uint32_t any_esc = kMList ? 0u : (uint32_t)uni((int)eflag[j & 1]);
        if (!kMList && lane == 0) eflag[j & 1] = 0u;
        const bool full = (j + 1) * SB <= T;
        // the block's records in groups of at most 8 steps, last group first
        constexpr int H = SB > 8 ? 8 : SB;
#pragma unroll
        for (int h = SB / H - 1; h >= 0; --h) {
          uint4 r[H];
#pragma unroll
          for (int k = 0; k < H; ++k) r[k] = src[(h * H + k) * kLanes + lane];
          if (full) {
            // common case: a full block, no per-step branches
#pragma unroll
            for (int k = H - 1; k >= 0; --k) {
              emit_words(r[k].z, x, ring, wp, spare, ring_mask);
              x = enc_apply(x, r[k]);
            }
          } else {
#pragma unroll
            for (int k = H - 1; k >= 0; --k) {
              if (j * SB + h * H + k >= T) continue;
              emit_words(r[k].z, x, ring, wp, spare, ring_mask);
              x = enc_apply(x, r[k]);
            }
          }
          // escapes of the group (their bins are coded above): list them,
          // last step first, so the list stays in position order
          if (__builtin_expect(any_esc != 0, 0)) {
#pragma unroll
            for (int k = H - 1; k >= 0; --k)
              if (any_esc & (1u << (h * H + k))) enc_escapes(r[k].z, r[k].w, esc_list, n_esc, lane);
          }
        }
        pc.bar_in();
        __syncthreads();
        pc.bar_out();
      }
      pc.cycles(13);
      pc.mark(4);
    } else {
      if (nblk > 0) map_block(nblk - 1);
      __syncthreads();
      for (int j = nblk - 1; j >= 0; --j) {
        // kMList: the first mapper wave lists the escapes of block j (their
        // bins are coded by the coder meanwhile) from the block's records,
        // last step first, so the list stays in position order, eight steps'
        // escape words read at a time (one wait for each group).  The steps'
        // flags are cleared for block j - 2, which is mapped after the next
        // barrier.
        if (kMList && wid == 1) {
          const uint32_t any_esc = (uint32_t)uni((int)eflag[j & 1]);
          eflag[j & 1] = 0u;
          if (any_esc != 0u) {
            const uint4* src = recs + (j & 1) * SB * kLanes;
            constexpr int G8 = SB > 8 ? 8 : SB;
#pragma unroll
            for (int hh = SB / G8 - 1; hh >= 0; --hh) {
              const uint32_t gb = (any_esc >> (hh * G8)) & ((1u << G8) - 1u);
              if (gb == 0u) continue;
              uint32_t z[G8], w[G8];
#pragma unroll
              for (int k = 0; k < G8; ++k) {
                const uint4 rr = src[(hh * G8 + k) * kLanes + lane];
                z[k] = rr.z;
                w[k] = rr.w;
              }
#pragma unroll
              for (int k = G8 - 1; k >= 0; --k)
                if (gb & (1u << k)) enc_escapes(z[k], w[k], esc_list, n_esc, lane);
            }
          }
        }
        if (j > 0) {  // mappers: block j - 1 while the coder codes block j
#pragma unroll
          for (int e = 0; e < kPer; ++e) {
            ca[e] = na[e];
            cb[e] = nb[e];
            cm[e] = nm[e];
          }
          if (j > 1) load_block(j - 2, na, nb, nm);
          map_block(j - 1);
        }
        __syncthreads();
      }
    }
  }

  hash = wave_fold_dpp<false>(hash);
  status = wave_fold_dpp<true>(status);
  znib = wave_fold_dpp<false>(znib);
  if (lane == 0) {
    part[wid] = hash;
    part[kWaves + wid] = status;
    part[2 * kWaves + wid] = znib;
    if (wid == (kMList ? 1 : 0)) part[3 * kWaves] = (uint32_t)n_esc;
    if (wid == 0) {
      part[3 * kWaves + 1] = (uint32_t)(a.cap_words - wp);
      part[kPartWp] = (uint32_t)wp;
      part[kPartFl] = (uint32_t)fl;
    }
  }
  if (fused) {
    // the coder's ring flushes and the escape list (the coder's or the first
    // mapper's) are in memory before the other waves read them back
    if (wid <= 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // the tables' LDS (and the scale table's) is free now: the flushed words
    // are staged there
    fused_pack<kThreads, kWaves>(a, g, tid, lane, wid, A, x, part, ring, ring_mask, wbuf,
                                 reinterpret_cast<uint64_t*>(recs), th.digest_lo, th.digest_hi,
                                 reinterpret_cast<uint32_t*>(lmeta),
                                 a.lds_bytes - (ring_bytes + (uint32_t)G::kTail), pc);
    return;
  }
  __syncthreads();
  // The coder wave's last words and final states are stored only now: the
  // reductions above wait for the mappers' loads, and a wait for loads also
  // waits for every store issued before them.  Pack reads them after this
  // kernel has ended.
  if (wid == 0) {
    if (fl > wp) ring_flush(wbuf, ring, wp, fl, lane, ring_mask);
    if (lane < A) a.states[g * kLanes + lane] = x;
  }
  // The unit's counts are published by the first mapper wave (its escape
  // list stores, if any, complete before the counter too: the wait below
  // covers them; the pack kernel reads the list).  What the last workgroup reads (maybe on another XCD,
  // behind another L2) is stored with agent-scope atomics, coherent across
  // the device, and has completed before the counter is raised: no fence, so
  // no write-back of the XCD's whole L2.
  if (tid == kLanes) {
    uint32_t hs = 0, ss = 0, zs = 0;
    for (int w = 0; w < kWaves; ++w) {
      hs += part[w];
      ss |= part[kWaves + w];
      zs += part[2 * kWaves + w];
    }
    const uint32_t W = part[3 * kWaves + 1];
    a.index_hash[g] = hs;  // read by the pack kernel only
    a.esc[g].x = part[3 * kWaves];
    __hip_atomic_store(&a.chunk_words[g], W, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&a.esc[g].y, zs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint64_t* done = reinterpret_cast<uint64_t*>(a.ctrl + kCtrlEncDone);
    if (ss)
      __hip_atomic_fetch_or(done, (uint64_t)ss << kEncStShift, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint64_t inc = 1ull | ((uint64_t)unit_quads(A, W, zs) << kEncCountBits);
    pc.mark(5);
    const uint64_t old = __hip_atomic_fetch_add(done, inc, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    pc.mark_after_loads(6);  // the atomic returned
    pc.store(a.phase, g, 5, 7);
    const bool last = (old & kEncCountMask) == (uint64_t)(a.units - 1);
    if (last) {
      encode_finish(a, old + inc);
      pc.store_done(a.phase, g);
    }
    part[3 * kWaves + 2] = last;
  }
  if (tid == 0) pc.store(a.phase, g, 0, 5);  // the coder wave's points
  __syncthreads();
  if (part[3 * kWaves + 2]) {  // uniform: the last workgroup
    __syncthreads();  // every wave has read the flag before part is reused
    unit_end_offsets<kThreads>(a, tid, reinterpret_cast<uint64_t*>(part));
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
  const uint2* __restrict__ esc;
  const uint32_t* __restrict__ esc_raw;
  const uint8_t* __restrict__ tables;
  uint8_t* __restrict__ out;
  int64_t out_bytes, header_bytes, cap_words, units, N;
  uint32_t B, N32, C, P, K, chunk_len, M, S, seg_cap;
};

__global__ __launch_bounds__(256) void k_pack(PackArgs a) {
  const int64_t g = blockIdx.x;
  const int tid = threadIdx.x;
  // the unit's offsets, counts and hash are independent loads, issued
  // together (not behind the offsets' bounds check)
  const uint32_t beg = g ? a.end_off[g - 1] : 0u;
  const uint32_t endo = a.end_off[g];
  const int64_t W = a.chunk_words[g];
  const uint2 ez = a.esc[g];  // escape count, escape nibbles
  const uint32_t ihash = a.index_hash[g];
  uint32_t* __restrict__ hdr = reinterpret_cast<uint32_t*>(a.out);
  if (tid == 0) {
    hdr[kFixedWords + g] = endo;
    hdr[kFixedWords + a.units + g] = ihash;
  }
  if (g == 0) {
    const TabHdr* th = reinterpret_cast<const TabHdr*>(a.tables);
    write_fixed_header<256>(hdr, tid, a.B, a.N32, a.C, a.P, a.K, a.chunk_len, a.M, a.S,
                            th->digest_lo, th->digest_hi, a.units, a.header_bytes);
  }
  if ((int64_t)a.header_bytes + endo > a.out_bytes || endo < beg) return;
  const int len = unit_len(g, (int32_t)a.K, (int32_t)a.S, a.N, (int32_t)a.chunk_len);
  const int A = len < kLanes ? len : kLanes;  // final states
  int64_t U = W + (ez.y + 3u) / 4u;
  U += U & 1;  // u16 words after the states: stream, pad, escape words
  uint8_t* dst = a.out + a.header_bytes + beg;
  uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
  for (int j = tid; j < A; j += 256) d32[j] = a.states[g * kLanes + j];
  const uint16_t* src = a.words + g * a.cap_words + (a.cap_words - W);
  uint32_t* w32 = reinterpret_cast<uint32_t*>(dst + 4 * A);
  const int64_t n32 = U / 2;
  for (int64_t j = tid; j < n32; j += 256) {
    const uint32_t lo = (2 * j < W) ? src[2 * j] : 0u;
    const uint32_t hi = (2 * j + 1 < W) ? src[2 * j + 1] : 0u;
    w32[j] = lo | (hi << 16);
  }
  if (ez.x == 0) return;
  __shared__ uint32_t wtot[4];
  // the zeros above are stored before any wave ORs into them
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const uint32_t E = ez.x;
  pack_escapes<256>(a.esc_raw + g * (int64_t)a.seg_cap + (a.seg_cap - E), E, w32, n32, tid, wtot);
}

// ============================================================================
// Decoder
// ============================================================================

// Decode workgroup: wave 0 is the coder, waves 1..kMappers the mappers, the
// last wave the escape reader.
constexpr int kDecWaves = kMappers + 2;
constexpr int kDecThreads = kDecWaves * kLanes;
constexpr int kEscWave = kDecWaves - 1;
// per wave: index hash, status, escape nibbles
constexpr int kDecPartBytes = (12 * kDecWaves + 15) / 16 * 16;
// control words: [1] escape entries available (set when the reader stops),
// [2 + b] steps of block parity b whose tables are not all in LDS (bit per
// step, set by the mappers), [4 + b] block parity b has escapes and [6 + b]
// escape entries consumed before block parity b (set by the coder)
constexpr int kDecCtlBytes = 32;
constexpr uint32_t kNoSym = 0xffffu;  // record of a lane past the chunk end
constexpr uint32_t kAllAvail = 0xffffffffu;

struct DecArgs {
  const uint8_t* __restrict__ payload;
  int64_t payload_bytes;
  const int32_t* __restrict__ indexes;
  const uint8_t* __restrict__ tables;
  uint32_t M, tables_bytes;
  BlobRef blob;
  const float* __restrict__ medians;
  const float* __restrict__ means;        // Gaussian: per element, or NULL
  const float* __restrict__ scales;       // Gaussian: per element
  const float* __restrict__ scale_table;  // Gaussian: L non-decreasing scales
  int32_t n_scales, scales_pow2;
  float scale_bound;
  uint32_t scales_lds;  // LDS byte offset of the staged scale table
  int32_t* __restrict__ out_sym;
  float* __restrict__ out_y;
  int64_t N, header_bytes, units;
  uint32_t B, C, P, K, chunk_len, S;
  UDiv div_hw;
  int32_t nt_cap, ne_cap, nd_cap, stage_all;
  uint32_t starts_words;  // search lookups: 16-byte words of starts to stage
  uint32_t* __restrict__ ctrl;
  uint32_t* __restrict__ status_out;
  PhaseBuf phase;
};

// Decoder geometry for blocks of SB steps (the mappers' lead over the coder
// and the steps between two barriers).
template <int SB>
struct DecGeom {
  static constexpr int kPer = (SB + kMappers - 1) / kMappers;  // steps per mapper wave and block
  static constexpr int kPfU32 = SB >= 16 ? 8 : 4;               // prefetch: u32 per lane
  static constexpr int kPfWords = 2 * kPfU32 * kLanes;         // words per prefetch batch
  static constexpr int kRing = SB >= 8 ? 2048 : 1024;          // stream ring (u16 words)
  static constexpr int kLowWater = SB >= 8 ? 1024 : 512;
  static constexpr int kPre = kLowWater / kPfWords;            // batches staged before block 0
  static constexpr int kEscR = 2 * SB * kLanes;                // escape FIFO entries
  static constexpr int kRingBytes = 2 * kRing;
  static constexpr int kRecBytes = 2 * SB * kLanes * 8;
  static constexpr int kEscBytes = 4 * kEscR;
  static constexpr int kMedBytes = 2 * SB * kLanes * 4;
  // per step of two blocks: escaping lanes (u64) and the first entry's ordinal
  static constexpr int kEscInfoBytes = 2 * SB * 16;
  // [ring][records][escape FIFO][medians (latents)][escape steps][parts][control]
  static constexpr int fixed(bool latents) {
    return kRingBytes + kRecBytes + kEscBytes + (latents ? kMedBytes : 0) + kEscInfoBytes +
           kDecPartBytes + kDecCtlBytes;
  }
  // a block start with fewer than kLowWater words buffered commits a batch:
  // a batch covers one block's words (at most one per lane and step), so
  // every block starts with at least SB * kLanes words buffered
  static_assert(kLowWater >= SB * kLanes && kPfWords >= SB * kLanes &&
                    kLowWater + kPfWords <= kRing && kPre >= 1 && kPfU32 <= kPfU32Max,
                "decoder stream ring too small");
  static_assert((kDecPartBytes + kDecCtlBytes) % 16 == 0, "LDS parts 16-byte aligned");
};

int dec_fixed_lds(bool latents, int sb) {
  return sb >= 16 ? DecGeom<16>::fixed(latents)
                  : (sb >= 8 ? DecGeom<8>::fixed(latents) : DecGeom<4>::fixed(latents));
}

// Mapper record of one lane and step (8 bytes), tables in LDS when the step's
// flag is 1:
//   x: the lane's table | escape symbol << 16 (nsym - 1; kNoSym for a lane
//      past the chunk end); the table is the LDS-local index times the
//      lookup's bucket count (its first bucket: one add fewer per step for
//      the coder), or the global index
//   y: table offset
// The coder overwrites x with the decoded value.
template <bool kImplicit, bool kWide>
__device__ __forceinline__ uint2 dec_record(const DecArgs& a, const Tabs& tb, int lane, int t,
                                            int len, int32_t start, int32_t in_b,
                                            uint32_t& hash, uint32_t& status, bool& all_lds) {
  const int p = lane + kLanes * t;
  const bool act = p < len;
  int32_t tbi =
      kImplicit ? (int32_t)udiv((uint32_t)unit_pos(start, (int32_t)a.S, p), a.div_hw) : in_b;
  const bool bad = act & ((uint32_t)tbi >= a.M);
  const bool ok = act & !bad;
  status |= bad ? GAANS_ST_INDEX : 0u;
  tbi = ok ? tbi : (tb.nt > 0 ? tb.t_lo : 0);
  hash += ok ? index_term((uint32_t)p, (uint32_t)tbi) : 0u;
  const bool staged = (uint32_t)(tbi - tb.t_lo) < (uint32_t)tb.nt;
  all_lds = ballot(!staged) == 0;
  uint32_t nsym, offset;
  if (all_lds) {  // separate loads per memory, as in dec_lookup
    const uint4 lm = tb.lmeta[tbi - tb.t_lo];
    nsym = lm.y;
    offset = lm.z;
    asm volatile("" : "+v"(nsym), "+v"(offset));
  } else {
    const TabMeta gm = tb.gmeta[tbi];
    nsym = gm.nsym;
    offset = (uint32_t)gm.offset;
    asm volatile("" : "+v"(nsym), "+v"(offset));
  }
  uint2 r;
  constexpr int kB = kWide ? kWideBits : kLutBits;
  r.x = (uint32_t)(all_lds ? (tbi - tb.t_lo) << kB : tbi) | ((act ? nsym - 1u : kNoSym) << 16);
  r.y = offset;
  return r;
}

// Mapper record with the search lookups (all tables in LDS): x = the table's
// first segment (table * kSearchEntries, below 2^16 when the blob has the
// search lookups) | starts index of its escape symbol << 16 (kNoSym past the
// chunk end), y = offset - the starts index of its symbol 0, so that the
// decoded starts index + y is the value.
__device__ __forceinline__ uint2 dec_record_search(const DecArgs& a, const Tabs& tb, int lane,
                                                   int t, int len, int32_t in_b, uint32_t& hash,
                                                   uint32_t& status) {
  const int p = lane + kLanes * t;
  const bool act = p < len;
  int32_t tbi = in_b;
  const bool bad = act & ((uint32_t)tbi >= a.M);
  const bool ok = act & !bad;
  status |= bad ? GAANS_ST_INDEX : 0u;
  tbi = ok ? tbi : 0;
  hash += ok ? index_term((uint32_t)p, (uint32_t)tbi) : 0u;
  const uint4 lm = tb.lmeta[tbi];
  uint2 r;
  const uint32_t first = lm.x + (uint32_t)(kStartsTablePad * tbi);  // starts index of symbol 0
  r.x = (uint32_t)tbi * (uint32_t)kSearchEntries | ((act ? first + lm.y - 1u : kNoSym) << 16);
  r.y = lm.z - first;
  return r;
}

// One level down from a dense lookup entry e: entry i of its sub-block (LDS
// when the sub-blocks are staged, else global memory).  The asm keeps the two
// loads apart, so the compiler does not merge them into one generic load
// (which would also wait for the stream prefetch).
template <bool kLds>
__device__ __forceinline__ uint64_t sub_entry(const Tabs& tb, uint64_t e, uint32_t i) {
  uint64_t r;
  if (kLds && (uint32_t)e - tb.sub_first < tb.sub_n) {
    r = tb.lsub[(((uint32_t)e - tb.sub_first) << kSubBits) + i];
    asm volatile("" : "+v"(r));
  } else {
    r = tb.gsub[((size_t)(uint32_t)e << kSubBits) + i];
    asm volatile("" : "+v"(r));
  }
  return r;
}

__device__ __forceinline__ bool dense_entry(uint64_t e) { return (uint32_t)(e >> 48) == 0xffffu; }

// (symbol, start, freq) from a lookup entry with at most one other start
// (see the blob layout): s or s + 1.
__device__ __forceinline__ void lut_pick(uint64_t e, uint32_t cum, uint32_t& s, uint32_t& st,
                                         uint32_t& fr) {
  const uint32_t lo = (uint32_t)e, hi = (uint32_t)(e >> 32);
  const uint32_t st0 = lo & 0xffffu, st1 = (lo >> 16) + 1u;
  const bool up = cum >= st1;
  s = (hi & 0xffffu) + (up ? 1u : 0u);
  st = up ? st1 : st0;
  fr = up ? (hi >> 16) + 1u : st1 - st0;
}

// cum -> (symbol, start, freq) in table t: the table's lookup entry of
// bucket cum >> 8, for a dense bucket the entry of sub-range (cum >> 4) & 15
// of its sub-block, for a dense sub-range the exact entry of value cum & 15
// (see the blob layout).  kWide: the wide lookups, bucket cum >> 5 and, for
// a dense bucket, sub-range (cum >> 1) & 15 of its sub-block.  t is the
// staged table's first bucket (kLds) or the global table index.  kEarly: the
// entry is decoded before the dense test's branch (the asm keeps it there)
// and a dense lane's values are redone from the entry one or two levels
// down, which overlaps the branch's latency with that work (512x768 decode
// 23.6 -> 23.2 us with one workgroup per CU); else after it, which spends
// no issue slots on the redone work (batch-64 skew decode 95.9 -> 93.9 us
// with three per CU).
template <bool kLds, bool kWide = false, bool kEarly = false>
__device__ __forceinline__ void dec_lookup(const Tabs& tb, uint32_t t, uint32_t cum, bool act,
                                           uint32_t& s, uint32_t& st, uint32_t& fr) {
  constexpr int kB = kWide ? kWideBits : kLutBits;
  const uint32_t li = (kLds ? t : t << kB) + (cum >> (16 - kB));
  uint64_t e = kLds ? tb.llut[li] : tb.glut[li];
  if (kEarly) {
    lut_pick(e, cum, s, st, fr);
    asm volatile("" : "+v"(s), "+v"(st), "+v"(fr));
  }
  const uint64_t dm = ballot(act & dense_entry(e));
  if (!kEarly) asm volatile("" ::"s"(dm));
  if (__builtin_expect(dm != 0ull, 0)) {
    if constexpr (kWide) {
      // a wide bucket's sub-ranges (two values) are never dense
      if (act & dense_entry(e)) e = sub_entry<kLds>(tb, e, (cum >> kWideSubShift) & (kSubSize - 1));
    } else {
      if (act & dense_entry(e)) e = sub_entry<kLds>(tb, e, (cum >> kSubBits) & (kSubSize - 1));
      const uint64_t dm3 = ballot(act & dense_entry(e));
      if (__builtin_expect(dm3 != 0ull, 0) && (act & dense_entry(e)))
        e = sub_entry<kLds>(tb, e, cum & (kSubSize - 1));
    }
    if (kEarly) lut_pick(e, cum, s, st, fr);
  }
  if (!kEarly) lut_pick(e, cum, s, st, fr);
}

// cum -> (symbol, start, freq) with the search lookups, all tables in LDS;
// t is the table's first segment.  The segment of cum is a 32-value part in
// the table's first or last kSearchFine buckets (entry (cum >> 5) & 63),
// else its 256-value bucket (entry 64 + (cum >> 8)); both entries are read
// at once and the segment's kept, which leaves one op and a shift before the
// read.  A fitted entry's (m | 0 << 8 | G << 16) line c = G + (((cum & 255)
// * m) >> 8) is at most
// three starts indexes below cum's symbol and never above it, so one read
// of starts c .. c + 4 resolves it; the starts hold start - 1, and the
// padding after each table 0xffff, so "start - 1 < cum" counts exactly the
// candidates at or below cum, with no test of the table's end.  A segment
// no line fits (bits 8-15: n > 3 symbols after its first) has all n + 1
// candidates from G: more than three are first narrowed by a 4-way search
// over their starts (three probe reads per round trip, uniform loop while
// any lane has more than three left).  s is the starts index (the record
// carries offset - the table's first index).
__device__ __forceinline__ void dec_lookup_search(const Tabs& tb, uint32_t t, uint32_t cum,
                                                  bool act, uint32_t& s, uint32_t& st,
                                                  uint32_t& fr) {
  static_assert(kSearchFine == 4 && kSearchFineBits == 5 && kSearchParts == 64,
                "segment arithmetic below");
  uint32_t eb = tb.lclut[t + kSearchParts + (cum >> 8)];
  uint32_t ep = tb.lclut[t + ((cum >> 5) & 63u)];
  asm("" : "+v"(eb), "+v"(ep));  // two reads, not one of a selected address
  const bool fine = (uint16_t)(cum + 1024u) < 2048u;  // cum < 1024 or cum >= 64512
  const uint32_t e = fine ? ep : eb;  // m | n << 8 | G << 16
  uint32_t g = (e >> 16) + (__umul24(cum & 0xffu, e & 0xffu) >> 8);
  // the words holding starts g .. g + 4 (below), read before the search test
  const uint32_t* pw = reinterpret_cast<const uint32_t*>(tb.lstarts) + (g >> 1);
  uint32_t w0 = pw[0], w1 = pw[1], w2 = pw[2];
  asm("" : "+v"(w0), "+v"(w1), "+v"(w2));
  uint32_t nl = (e >> 8) & 0xffu;  // candidates after g: 0 for a fitted segment
  bool wide = act & ((e & 0xffffu) > 0x3ffu);  // nl > 3
  if (__builtin_expect(ballot(wide) != 0ull, 0)) {
    // the probes q, 2q, 3q (q = (nl + 1) / 4 >= 1) split it into four ranges
    do {
      if (wide) {
        const uint32_t q = (nl + 1u) >> 2;
        const bool l1 = tb.lstarts[g + q] < cum, l2 = tb.lstarts[g + 2u * q] < cum,
                   l3 = tb.lstarts[g + 3u * q] < cum;
        const uint32_t kk = (uint32_t)l1 + (uint32_t)l2 + (uint32_t)l3;
        g += kk * q;
        nl = l3 ? nl - 3u * q : q - 1u;
      }
      wide = act & (nl > 3u);
    } while (ballot(wide) != 0ull);
    const uint32_t* pg = reinterpret_cast<const uint32_t*>(tb.lstarts) + (g >> 1);
    w0 = pg[0];
    w1 = pg[1];
    w2 = pg[2];
  }
  // starts g .. g + 4 from the three aligned words that hold them (a b64
  // read at a 2-byte address costs about 55 cycles more than aligned reads)
  // start g's byte shift in w0 is 2 (g & 1): v_alignbyte_b32 reads the low
  // two bits of its shift operand and v_bfe_u32 the low five of its offset,
  // so g << 1 and g << 4 serve as they are (no mask)
  const uint32_t a01 = __builtin_amdgcn_alignbyte(w1, w0, g << 1),
                 a23 = __builtin_amdgcn_alignbyte(w2, w1, g << 1);
  const uint32_t v0 = a01 & 0xffffu, v1 = a01 >> 16, v2 = a23 & 0xffffu, v3 = a23 >> 16;
  uint32_t v4 = __builtin_amdgcn_ubfe(w2, g << 4, 16);
  asm volatile("" : "+v"(v4));  // computed for every lane: selects below, not a branch
  // candidates past the symbol (or the table) hold larger starts or 0xffff
  const bool b1 = v1 < cum, b2 = v2 < cum, b3 = v3 < cum;
  const uint32_t kk = (uint32_t)b1 + (uint32_t)b2 + (uint32_t)b3;
  s = g + kk;
  const uint32_t sm = b3 ? v3 : (b2 ? v2 : (b1 ? v1 : v0));  // start - 1
  const uint32_t nx = b3 ? v4 : (b2 ? v3 : (b1 ? v2 : v1));   // next start - 1
  // freq: the next start - start mod 2^16 (2^16 for a one-symbol table), and
  // start mod 2^16 (a table's first symbol holds 0xffff)
  fr = ((nx - sm - 1u) & 0xffffu) + 1u;
  st = (sm + 1u) & 0xffffu;
}

// Stage every table's search lookups, starts and metadata (whole workgroup
// of NT threads); blob-wide symbol indexes stay valid in LDS.
template <int NT>
__device__ void stage_search(Tabs& T, uint4* lmeta, uint32_t* lclut, uint16_t* lstarts,
                             const uint8_t* tables, const BlobRef& blob, uint32_t M,
                             uint32_t starts_words, int tid) {
  T.t_lo = 0;
  T.nt = (int)M;
  T.sub_first = 0;
  T.sub_n = 0;
  copy16_dma<NT>(reinterpret_cast<uint4*>(lclut),
                 reinterpret_cast<const uint4*>(tables + blob.clut_off), M * (kSearchEntries / 4), tid);
  copy16_dma<NT>(reinterpret_cast<uint4*>(lstarts),
                 reinterpret_cast<const uint4*>(tables + blob.starts_off), starts_words, tid);
  stage_pass<NT, false, false>(T, lmeta, nullptr, nullptr, nullptr, M, 1u, 0u, 0u, 0, tid);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct-to-LDS copies are in
  __syncthreads();
}

// Decoder staging in two halves.  stage_early, at kernel entry (it needs
// neither the payload header nor the blob's checks, only the staged range):
// the lookups' copy straight into LDS -- the staged tables' lookups, or every
// table's search lookups and symbol starts -- and one metadata row per
// thread into registers.  stage_late, once the checks pass: the sub-blocks'
// copy (its range comes from the blob's metadata), the metadata rows into
// LDS, the wait for this wave's copies and the barrier.  The first copies are
// then in flight during the header's round trip instead of after it.
struct EarlyStage {
  int t_lo, nt;
  TabMeta row;  // metadata of staged table t_lo + tid (tid < nt)
};

template <int NT, int LB, bool kSearch>
__device__ __forceinline__ EarlyStage stage_early(const Tabs& T, uint64_t* llut, uint32_t* lclut,
                                                  uint16_t* lstarts, const uint8_t* tables,
                                                  const BlobRef& blob, uint32_t M,
                                                  uint32_t starts_words, int t_lo, int t_hi,
                                                  int tid) {
  EarlyStage e;
  e.t_lo = kSearch ? 0 : t_lo;
  e.nt = kSearch ? (int)M : (t_hi > t_lo ? t_hi - t_lo : 0);
  e.row = TabMeta{0u, 0u, 0, 0u};
  if (e.nt > 0) {
    if constexpr (kSearch) {
      copy16_dma<NT>(reinterpret_cast<uint4*>(lclut),
                     reinterpret_cast<const uint4*>(tables + blob.clut_off),
                     M * (kSearchEntries / 4), tid);
      copy16_dma<NT>(reinterpret_cast<uint4*>(lstarts),
                     reinterpret_cast<const uint4*>(tables + blob.starts_off), starts_words, tid);
    } else {
      copy16_dma<NT>(reinterpret_cast<uint4*>(llut),
                     reinterpret_cast<const uint4*>(T.glut + (int64_t)t_lo * LB),
                     (uint32_t)e.nt * (LB / 2), tid);
    }
    e.row = T.gmeta[e.t_lo + (tid < e.nt ? tid : e.nt - 1)];
  }
  return e;
}

template <int NT, bool kSearch>
__device__ __forceinline__ void stage_late(Tabs& T, const EarlyStage& e, uint4* lmeta,
                                           uint64_t* lsub, uint32_t sub_cap,
                                           const StageBounds& bd, int tid) {
  T.t_lo = e.t_lo;
  T.nt = e.nt;
  T.sub_first = 0;
  T.sub_n = 0;
  if (e.nt > 0) {
    const uint32_t base0 = kSearch ? 0u : bd.base0;
    if (!kSearch && lsub && bd.d1 > bd.d0) {
      // the range's first sub_cap sub-blocks (a plan may hold fewer than the
      // range has: the others are read from global memory)
      T.sub_first = bd.d0;
      T.sub_n = bd.d1 - bd.d0 < sub_cap ? bd.d1 - bd.d0 : sub_cap;
      copy16_dma<NT>(reinterpret_cast<uint4*>(lsub),
                     reinterpret_cast<const uint4*>(T.gsub + (size_t)bd.d0 * kSubSize),
                     T.sub_n * (kSubBytes / 16), tid);
    }
    if (e.nt <= NT) {
      if (tid < e.nt)
        lmeta[tid] = make_uint4(e.row.ent_base - base0, e.row.nsym, (uint32_t)e.row.offset,
                                e.row.ent_base);
    } else {
      stage_pass<NT, false, false>(T, lmeta, nullptr, nullptr, nullptr, (uint32_t)e.nt, 1u, 0u,
                                   base0, e.t_lo, tid);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct-to-LDS copies are in
  }
  __syncthreads();
}

// Word stream of one chunk: prefetched from HBM into registers (kPfWords words
// ahead) and copied into an LDS ring of kRing words holding the words
// [rp, filled) (positions mod kRing), kPfWords words at a time.  At the start
// of every block the coder commits the batch prefetched into registers (pf,
// words [filled, filled + kPfWords)) when fewer than kLowWater words are
// buffered, then prefetches the next batch.  This is the only place pf is
// loaded, so the loads stay in flight between blocks.  A step refills at most
// one word per lane, and a block starts with at least SB * kLanes buffered
// words, so refills need no check.
struct Stream {
  const uint32_t* __restrict__ s32;
  uint32_t lane_off;  // 4 * lane: the loads' only per-lane operand
  int q, q32, rp, filled;
  uint32_t pf[kPfU32Max];  // the first DecGeom<SB>::kPfU32 in use
};

// u32 i32 + 64 kk + lane of the unit's words (kk < N, i32 wave-uniform).
// The loads go through one buffer resource of the words from i32 on (scalar
// base and size), the 256-byte steps in their immediate offsets, which the
// range check includes (unlike the scalar offset): past the unit's end they
// read 0, with no branch (a refill that reaches such words marks the unit
// corrupt).  Their only vector operand is the loop-invariant lane offset:
// the compiler waits for a load to return before any of its vector operands
// is overwritten, so with a computed vector address the next block's first
// LDS read waited for the prefetch, which made the one-batch-ahead prefetch
// synchronous.  One resource per batch instead of one per load: about 25
// scalar instructions fewer per batch.
template <int N>
__device__ __forceinline__ void stream_batch32(const Stream& S, int i32, uint32_t* out) {
  // base and size are wave-uniform: kept in scalar registers (a resource in
  // vector registers makes the compiler loop over the lanes' values)
  const uint64_t base = reinterpret_cast<uint64_t>(S.s32 + i32);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32));
  const int left = uni(S.q32 > i32 ? S.q32 - i32 : 0);
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0, 4 * left, kBufferFlags);
#pragma unroll
  for (int kk = 0; kk < N; ++kk)
    out[kk] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)(S.lane_off + 4u * kLanes * kk), 0, 0);
}

// Block start: commit pf if needed, then fetch the next batch.
template <int SB>
__device__ __forceinline__ void stream_block_start(Stream& S, uint32_t* ring32, int lane) {
  using G = DecGeom<SB>;
  const bool commit = S.filled - S.rp < G::kLowWater && S.filled < S.q;
  if (commit) {
    // a batch starts at a multiple of its size in the ring, which holds a
    // whole number of batches: it never wraps, one mask for all its words
    static_assert((G::kRing / 2) % (G::kPfWords / 2) == 0, "ring of whole batches");
    uint32_t* dst = ring32 + (((uint32_t)S.filled >> 1) & (G::kRing / 2 - 1)) + lane;
#pragma unroll
    for (int kk = 0; kk < G::kPfU32; ++kk) dst[kk * kLanes] = S.pf[kk];
    S.filled = uni(S.filled + G::kPfWords);
    stream_batch32<G::kPfU32>(S, S.filled >> 1, S.pf);
  }
}

// A refill past the stream end reads stale ring words; the chunk is then
// marked corrupt by the final check that exactly the stream was consumed.
// Every lane reads (the lane's rank among the refilling lanes, counted on top
// of the stream position by mbcnt's accumulator) and only refilling lanes
// keep the word (the read's value is opaque to the compiler, so the select
// is not turned into an exec-masked branch around it).  kSkip: the read is
// skipped when no lane refills (a uniform branch on the compare).  Measured
// on MI355X: with one workgroup per CU, where the step's latency bounds the
// launch, the branch lengthens the step (2160x3840 latent 231 -> 238 us,
// 512x768 23.8 -> 24.4 us); with several per CU, where issue slots do, it
// saves them (batch-64 skew 101 -> 95 us, uniform 95 -> 90 us).
template <int SB, bool kSkip>
__device__ __forceinline__ void dec_refill(bool need, uint32_t& x, Stream& S, const uint16_t* ring,
                                           int lane) {
  const uint64_t m = ballot(need);
  if (!kSkip || m != 0ull) {
    // the ring position (< kRing) plus the rank: past the end it reads the
    // mirrored first words
    const uint32_t pos = __builtin_amdgcn_mbcnt_hi(
        (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)S.rp));
    uint32_t w = ring[pos & (DecGeom<SB>::kRing - 1)];
    asm volatile("" : "+v"(w));
    x = need ? ((x << 16) | w) : x;
    S.rp += __popcll(m);
  }
}

// Escape section of one chunk, read from the chunk's end: escape u32 m holds
// the nibbles [8m, 8m + 8), nibble 8m + r at bits 4r; it is the stream's u32
// n32 - 1 - m with its halves swapped.  An entry is a count n then n nibbles
// of raw, and n is the minimal count of raw (raw ? msb(raw) / 4 + 1 : 0).
//
// The coder only marks escapes: per step, the escaping lanes and the ordinal
// of the step's first entry.  The mapper that stores the block (during the
// next block) resolves the values from an LDS FIFO of kEscR = 2 SB kLanes
// raw values (entry e in slot e mod kEscR), which the escape reader (the
// workgroup's last wave) fills in order: during block j it parses up to
// c_j + SB kLanes entries, c_j being the entries consumed before block j
// (published by the coder before the barrier).  Block j consumes at most
// SB kLanes entries, so its entries are there when block j is stored, and
// the entries written during block j (ordinals in [c_j, c_j + SB kLanes))
// never share a slot with those of block j - 1 that the mappers read then
// (ordinals in [c_j - SB kLanes, c_j)).  The reader stops at the first
// invalid entry (count > 8 or not minimal) or at the end of the chunk's
// words, and publishes how many entries are valid; resolving more marks the
// chunk corrupt.
//
// The reader holds escape u32s [base, base + 128) in registers (lane i of w0
// / w1: u32 base + i / base + 64 + i) and parses 64 nibble positions at a
// time: lane l decodes the entry that would start at nibble q + l (count,
// raw value, length, validity), then a scalar walk from q over the lengths
// marks the real entry starts, and the marked lanes write their raw values
// to the FIFO in one store.
struct EscReader {
  const uint32_t* __restrict__ w32;   // the chunk's words after the states
  int n32, base;
  uint32_t q, p;     // nibbles and entries parsed
  bool stopped;
  uint32_t w0, w1;   // window
};

// Escape u32 m (zero past the chunk's words).  A buffer load over the
// chunk's n32 words (wave-uniform base and size in scalar registers): for m
// >= n32 the byte offset 4 (n32 - 1 - m) wraps past the buffer's size and
// the load returns 0, so no branch goes around the load (a branch made each
// load wait for its data before the next one was issued).
__device__ __forceinline__ uint32_t esc_word(const EscReader& E, int m) {
  const uint64_t base = reinterpret_cast<uint64_t>(E.w32);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32));
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0, 4 * uni(E.n32), kBufferFlags);
  const uint32_t v =
      __builtin_amdgcn_raw_buffer_load_b32(r, (int)(4u * (uint32_t)(E.n32 - 1 - m)), 0, 0);
  return (v >> 16) | (v << 16);
}

// Escape u32 base + i of the window for lane-varying i in [0, 128).
__device__ __forceinline__ uint32_t esc_window_word(const EscReader& E, int i) {
  const int addr = (i & (kLanes - 1)) << 2;
  const uint32_t a = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)E.w0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)E.w1);
  return i < kLanes ? a : b;
}

// Parse entries until `target` are available or the section ends.
template <int R>
__device__ void esc_parse(EscReader& E, uint32_t target, uint32_t* fifo, uint32_t* ctl,
                          int lane) {
  const uint32_t qmax = 8u * (uint32_t)E.n32;
  while (!E.stopped && E.p < target) {
    // the 64 positions' entries lie in u32s [q >> 3, (q >> 3) + 10)
    while ((int)(E.q >> 3) + 10 > E.base + 2 * kLanes) {
      E.base += kLanes;
      E.w0 = E.w1;
      E.w1 = esc_word(E, E.base + kLanes + lane);
    }
    const uint32_t pos = E.q + (uint32_t)lane;
    const int i = (int)(pos >> 3) - E.base;
    const uint64_t v = (((uint64_t)esc_window_word(E, i + 1) << 32) | esc_window_word(E, i)) >>
                       (4u * (pos & 7u));
    const uint32_t n = (uint32_t)v & 15u;
    const uint32_t raw = (uint32_t)((v >> 4) & ((1ull << (4u * n)) - 1ull));
    const uint32_t top = (uint32_t)(v >> (4u * n)) & 15u;  // raw's last nibble
    // a valid entry: count <= 8, minimal (last nibble non-zero), inside the words
    const bool valid = n <= 8u && (n == 0u || top != 0u) && pos + 1u + n <= qmax;
    const uint64_t vm = ballot(valid);
    const uint32_t len = 1u + n;
    uint64_t starts = 0;
    uint32_t at = 0, cnt = 0;
    const uint32_t want = target - E.p;
    while (at < (uint32_t)kLanes && cnt < want) {
      if (!((vm >> at) & 1ull)) {
        E.stopped = true;
        break;
      }
      starts |= 1ull << at;
      ++cnt;
      at += (uint32_t)__builtin_amdgcn_readlane((int)len, (int)at);
    }
    if ((starts >> lane) & 1ull) fifo[(E.p + lane_rank(starts)) & (R - 1)] = raw;
    E.p += cnt;
    E.q += at;
  }
  if (E.stopped && lane == 0) ctl[1] = E.p;
}

// Values of the escaping lanes em of one step, decoded by the coder as the
// escape bin: lane L takes FIFO entry base + (escaping lanes below L), with
// CompressAI's mapping (reference warp_ans_kernel.cu:316-327): raw odd ->
// -(raw >> 1) - 1, even -> (raw >> 1) + escape symbol, plus the table offset.
// v holds escape symbol + offset mod 2^32 (the coder's value for the bin),
// off the offset.  enib counts the lane's escape nibbles (1 + n per entry).
template <int R>
__device__ __forceinline__ void esc_resolve(uint64_t em, uint32_t base, uint32_t off, uint32_t& v,
                                            uint32_t avail, const uint32_t* fifo, uint32_t& enib,
                                            uint32_t& status, int lane) {
  const bool e = (em >> lane) & 1ull;
  const uint32_t idx = base + lane_rank(em);
  const uint32_t raw = fifo[idx & (R - 1)];
  const uint32_t maxv = v - off;  // the escape symbol (exact: it is below 2^16)
  const int64_t sv = (int64_t)(int32_t)off +
                     ((raw & 1u) ? -(int64_t)(raw >> 1) - 1 : (int64_t)maxv + (raw >> 1));
  const bool bad = e & ((idx >= avail) | (sv < INT32_MIN) | (sv > INT32_MAX));
  status |= bad ? GAANS_ST_CORRUPT : 0u;
  v = e ? (bad ? 0u : (uint32_t)(int32_t)sv) : v;
  enib += e ? (raw ? ((31u - (uint32_t)__clz((int)raw)) >> 2) + 2u : 1u) : 0u;
}

// One decode step of the coder wave; returns the decoded value and, in em,
// the lanes that decoded the escape bin (their values are resolved by the
// mappers, off the state chain).  kFull: every lane is active and no offset
// can overflow with a symbol index.
template <bool kLds, bool kFull, int SB, bool kSearch = false, bool kWide = false,
          bool kSkip = false>
__device__ __forceinline__ uint32_t dec_step(const Tabs& tb, const uint2 r, uint32_t& x,
                                             Stream& S, const uint16_t* ring, uint64_t& em,
                                             uint32_t& status, int lane) {
  const uint32_t es = r.x >> 16;
  const bool act = kFull || es != kNoSym;
  const uint32_t cum = x & 0xffffu;
  uint32_t s, st, fr;
  if constexpr (kSearch) dec_lookup_search(tb, r.x & 0xffffu, cum, act, s, st, fr);
  else dec_lookup<kLds, kWide, !kSkip>(tb, r.x & 0xffffu, cum, act, s, st, fr);
  const uint32_t xn = __umul24(fr, x >> 16) + cum - st;
  x = act ? xn : x;
  dec_refill<SB, kSkip>(act & (x < kStateLow), x, S, ring, lane);
  // value + offset for an ordinary symbol: s < 2^16, so the int32 sum overflows
  // exactly when it wraps below the offset
  const int32_t o = (int32_t)(s + r.y);
  const bool esc = act & (s == es);
  em = ballot(esc);
  const bool oob = act & !esc & !kFull & (o < (int32_t)r.y);
  status |= oob ? GAANS_ST_CORRUPT : 0u;
  return (uint32_t)(oob ? 0 : o);
}

// Waves per SIMD the decoder is built for: 6 (see the LDS plan); the
// measurement build allows 5, since its phase points would otherwise push
// the 16-step kernels past the 80 registers of 6 waves into scratch (its
// phase times at three workgroups per CU are therefore approximate).
#ifdef GAANS_PHASE_TIMES
constexpr int kDecWavesPerSimd = 5;
#else
constexpr int kDecWavesPerSimd = 6;
#endif

template <int kMode, bool kImplicit, int SB, bool kSearch, bool kWide, bool kSkip = false>
__global__ __launch_bounds__(kDecThreads, kDecWavesPerSimd) void k_decode(DecArgs a) {
  constexpr bool kLatents = kMode != kModeSymbols;  // fp32 output with a per-element add
  using G = DecGeom<SB>;
  constexpr int kPer = G::kPer;
  constexpr int R = G::kEscR;
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* sring = reinterpret_cast<uint16_t*>(smem);
  uint32_t* sring32 = reinterpret_cast<uint32_t*>(smem);
  uint2* recs = reinterpret_cast<uint2*>(smem + G::kRingBytes);
  uint32_t* fifo = reinterpret_cast<uint32_t*>(smem + G::kRingBytes + G::kRecBytes);
  uint8_t* after_fifo = smem + G::kRingBytes + G::kRecBytes + G::kEscBytes;
  float* med = reinterpret_cast<float*>(after_fifo);
  uint4* escm = reinterpret_cast<uint4*>(after_fifo + (kLatents ? G::kMedBytes : 0));
  uint32_t* part = reinterpret_cast<uint32_t*>(escm + 2 * SB);
  uint32_t* ctl = part + kDecPartBytes / 4;
  uint8_t* tsm = smem + G::fixed(kLatents);
  // [luts][meta][sub-blocks], or with the search lookups [bucket entries]
  // [meta][starts]: every part 16-byte aligned
  static_assert(!(kSearch && kWide), "the search lookups have no wide form");
  constexpr int kLutEntry = kSearch ? 4 : 8;
  // lookup entries per staged table
  constexpr int kLB = kSearch ? kSearchEntries : (kWide ? kWideSize : kLutSize);
  uint64_t* llut = reinterpret_cast<uint64_t*>(tsm);
  uint32_t* lclut = reinterpret_cast<uint32_t*>(tsm);
  uint4* lmeta = reinterpret_cast<uint4*>(tsm + kLutEntry * kLB * a.nt_cap);
  uint64_t* lsub = reinterpret_cast<uint64_t*>(tsm + (kLutEntry * kLB + 16) * a.nt_cap);
  // the starts' LDS offset in one scalar register (the compiler would split
  // it into a register and a constant, one add more per lookup)
  int starts_off = G::fixed(kLatents) + (kLutEntry * kLB + 16) * a.nt_cap;
  asm("" : "+s"(starts_off));
  uint16_t* lstarts = reinterpret_cast<uint16_t*>(smem + starts_off);
  float* scl = reinterpret_cast<float*>(smem + a.scales_lds);  // Gaussian: scale table

  const int64_t g = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & (kLanes - 1);
  const int wid = uni(tid >> 6);  // wave role, kept in a scalar register
  PhaseClock pc;
  if (wid == 0) pc.mark(0);
  uint32_t status = 0, hash = 0, enib = 0;
  const uint32_t* __restrict__ hdr = reinterpret_cast<const uint32_t*>(a.payload);
  int64_t row;
  int32_t start;
  int len, k;
  unit_range(g, (int32_t)a.K, (int32_t)a.S, a.N, (int32_t)a.chunk_len, row, start, len, k);
  const int T = (len + kLanes - 1) / kLanes;
  const int A = len < kLanes ? len : kLanes;
  const int nst = A;  // final states
  const int nblk = (T + SB - 1) / SB;
  int t_lo, t_hi;
  stage_range(a.nt_cap, a.stage_all, k, (int)a.P, (int)a.M, t_lo, t_hi);
  const TabMeta* __restrict__ gmeta = reinterpret_cast<const TabMeta*>(a.tables + a.blob.meta_off);
  // Header words, the unit's end offsets and index hash, the table blob's
  // header and the staged range's metadata, all in one round trip: every
  // word is read (the host has checked that the payload holds the header;
  // the metadata lies in the blob whatever its content and is used only
  // when the checks pass), the loads are issued before any of them is used
  // (the scheduling barrier keeps them together), and the checks are
  // branch-free.
  const TabHdr th = load_tab_hdr(a.tables);
  uint32_t hw[13];
#pragma unroll
  for (int i = 0; i < 13; ++i) hw[i] = hdr[i];
  // end offsets of units g - 1 and g: two adjacent words (word 15 of the
  // fixed header stands in for unit -1 and is not used)
  const uint32_t* pe = hdr + (kFixedWords - 1) + g;
  const uint32_t e_prev = pe[0];
  const uint32_t e_end = pe[1];
  const StageBounds bd =
      kSearch ? StageBounds{0u, 0u, 0u, 0u}
              : (kWide ? stage_bounds_wide(reinterpret_cast<const uint32_t*>(a.tables +
                                                                             a.blob.wbase_off),
                                           t_lo, t_hi)
                       : stage_bounds(gmeta, t_lo, t_hi, a.M, a.blob.total_dense));
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t e_hash = hdr[kFixedWords + a.units + g];  // needed at the end only
  Tabs tb;
  tb.gmeta = gmeta;
  tb.gent = reinterpret_cast<const uint2*>(a.tables + a.blob.ent_off);
  tb.glut = reinterpret_cast<const uint64_t*>(a.tables +
                                              (kWide ? a.blob.wide_off : a.blob.lut_off));
  tb.gsub = reinterpret_cast<const uint64_t*>(a.tables +
                                              (kWide ? a.blob.wdense_off : a.blob.dense_off));
  tb.lmeta = lmeta;
  tb.lent = nullptr;
  tb.llut = llut;
  tb.lsub = lsub;
  tb.lclut = lclut;
  tb.lstarts = lstarts;
  const EarlyStage est = stage_early<kDecThreads, kLB, kSearch>(
      tb, llut, lclut, lstarts, a.tables, a.blob, a.M, a.starts_words, t_lo, t_hi, tid);
  int32_t cbx[kPer], nbx[kPer];
  float cm[kPer], nm[kPer];
  auto load_block = [&](int j, int32_t* ib, float* im) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int u = (wid - 1) + kMappers * e;
      if (SB % kMappers != 0 && u >= SB) break;
      int p = lane + kLanes * (j * SB + u);
      p = p < len ? p : len - 1;  // loads stay in the chunk; results are masked
      const int32_t q = unit_pos(start, (int32_t)a.S, p);  // row position
      if (kMode == kModeGaussian) {
        ib[e] = __float_as_int(a.scales[row + q]);  // index found at map time
        im[e] = a.means ? a.means[row + q] : 0.0f;
      } else {
        ib[e] = kImplicit ? 0 : a.indexes[row + q];
        im[e] = kLatents ? a.medians[udiv((uint32_t)q, a.div_hw)] : 0.0f;
      }
    }
  };
  // the mappers' first two blocks of inputs need neither the header checks
  // nor the tables
  if (wid != 0 && wid != kEscWave && nblk > 0) {
    load_block(0, cbx, cm);
    if (nblk > 1) load_block(1, nbx, nm);
  }
  if (wid == 0) pc.mark_after_loads(1);  // header, offsets and metadata are in
  const bool hdr_ok = (hw[0] == kMagic) & (hw[1] == kVersion) & (hw[2] == a.B) &
                      (hw[3] == (uint32_t)a.N) & (hw[4] == a.C) & (hw[5] == a.P) &
                      (hw[6] == a.K) & (hw[7] == a.chunk_len) & (hw[8] == a.M) &
                      (hw[9] == kParams) & (hw[12] == a.S);
  const bool tab_ok = tables_ok(th, a.M, a.tables_bytes, a.blob) & (hw[10] == th.digest_lo) &
                      (hw[11] == th.digest_hi);
  const bool offsets_safe = (th.flags & kTabOffsetsSafe) != 0;
  bool ok = hdr_ok & tab_ok;  // uniform over the workgroup
  status |= !hdr_ok ? GAANS_ST_HEADER : (!tab_ok ? GAANS_ST_TABLES : 0u);
  // the unit's bytes: the offsets are used unconditionally, so that their
  // loads are not moved behind the header checks
  const uint32_t beg = g ? e_prev : 0u;
  const uint32_t endo = e_end;
  const uint32_t want_hash = e_hash;
  const int64_t cb = (int64_t)endo - (int64_t)beg;
  const bool bad_range = (endo < beg) | ((int64_t)endo > a.payload_bytes - a.header_bytes) |
                         ((beg & 3u) != 0u) | (cb < 4 * nst) | (((cb - 4 * nst) & 3) != 0);
  status |= (ok & bad_range) ? GAANS_ST_CORRUPT : 0u;
  ok = ok & !bad_range;
  Stream S;  // the coder's; its final position is checked after the last barrier
  S.rp = 0;
  S.q = 0;
  // each wave's hash, status and escape nibbles -> part, before its last
  // barrier; the mappers publish before they issue the last block's stores,
  // since a wait for loads (the reductions') also waits for stores issued
  // before them
  auto publish = [&]() {
    hash = wave_fold_dpp<false>(hash);
    status = wave_fold_dpp<true>(status);
    enib = wave_fold_dpp<false>(enib);
    if (lane == 0) {
      part[wid] = hash;
      part[kDecWaves + wid] = status;
      part[2 * kDecWaves + wid] = enib;
    }
  };
  if (ok) {
    const uint8_t* cdata = a.payload + a.header_bytes + beg;
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(cdata + 4 * nst);
    const uint32_t* safe = reinterpret_cast<const uint32_t*>(cdata);
    const int q16 = (int)((cb - 4 * nst) / 2);  // u16 words after the states (even)

    // decoded values of block j -> HBM, escapes resolved first
    auto store_block = [&](int j, bool last) {
      const uint2* src = recs + (j & 1) * SB * kLanes;
      const bool any_esc = uni((int)ctl[4 + (j & 1)]) != 0;
      const uint32_t avail = (uint32_t)uni((int)ctl[1]);
      uint32_t vals[kPer];
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const int u = (wid - 1) + kMappers * e;
        if (SB % kMappers != 0 && u >= SB) break;
        const uint2 r = src[u * kLanes + lane];
        // the coder's value: in x, or with the search lookups in y (x keeps
        // the table's first segment, whose table's offset the escape mapping
        // needs)
        uint32_t v = kSearch ? r.y : r.x;
        if (any_esc && j * SB + u < T) {
          const uint4 ei = escm[(j & 1) * SB + u];  // escaping lanes, first entry
          const uint64_t em = (uint64_t)(uint32_t)uni((int)ei.x) |
                              ((uint64_t)(uint32_t)uni((int)ei.y) << 32);
          if (em) {
            const uint32_t off =
                kSearch ? tb.lmeta[(r.x & 0xffffu) / (uint32_t)kSearchEntries].z : r.y;
            esc_resolve<R>(em, (uint32_t)uni((int)ei.z), off, v, avail, fifo, enib, status, lane);
          }
        }
        vals[e] = v;
      }
      if (last) publish();
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const int u = (wid - 1) + kMappers * e;
        if (SB % kMappers != 0 && u >= SB) break;
        const int p = lane + kLanes * (j * SB + u);
        if (p < len) {
          const int64_t i = row + unit_pos(start, (int32_t)a.S, p);
          if (kLatents)
            a.out_y[i] = __fadd_rn((float)(int32_t)vals[e],
                                   med[((j & 1) * SB + u) * kLanes + lane]);
          else a.out_sym[i] = (int32_t)vals[e];
        }
      }
    };
    GaussCoarse gc{};  // the mappers': the scale table's coarse level
    auto map_block = [&](int j) {
      uint2* dst = recs + (j & 1) * SB * kLanes;
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const int u = (wid - 1) + kMappers * e;
        if (SB % kMappers != 0 && u >= SB) break;
        bool all_lds;
        const int32_t ix = kMode == kModeGaussian
                               ? gauss_index(__int_as_float(cbx[e]), scl, a.n_scales,
                                             a.scales_pow2, a.scale_bound, gc)
                               : cbx[e];
        uint2 r;
        if constexpr (kSearch) {
          r = dec_record_search(a, tb, lane, j * SB + u, len, ix, hash, status);
          all_lds = true;
        } else {
          r = dec_record<kImplicit, kWide>(a, tb, lane, j * SB + u, len, start, ix, hash,
                                           status, all_lds);
        }
        dst[u * kLanes + lane] = r;
        if (kLatents) med[((j & 1) * SB + u) * kLanes + lane] = cm[e];
        if (!all_lds && lane == 0)
          __hip_atomic_fetch_or(&ctl[2 + (j & 1)], 1u << u, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    };

    // Loads that do not depend on the tables are issued before the tables are
    // staged, so that they overlap: the coder's initial states and first
    // stream words, the mappers' first two blocks of inputs, the escape
    // reader's window.
    EscReader E;
    uint32_t x = kStateLow;
    uint32_t w0[G::kPre][G::kPfU32];
    if (wid == 0) {
      S.s32 = s32;
      S.lane_off = 4u * (uint32_t)lane;
      S.q = q16;
      S.q32 = q16 / 2;
      S.filled = 0;
      x = safe[lane < A ? lane : 0];  // lanes >= A: below
#pragma unroll
      for (int b = 0; b < G::kPre; ++b) stream_batch32<G::kPfU32>(S, b * (G::kPfWords / 2), w0[b]);
      stream_batch32<G::kPfU32>(S, G::kPre * (G::kPfWords / 2), S.pf);
    } else if (wid == kEscWave) {
      E.w32 = s32;
      E.n32 = q16 / 2;
      E.base = 0;
      E.q = 0;
      E.p = 0;
      E.stopped = false;
      E.w0 = esc_word(E, lane);
      E.w1 = esc_word(E, kLanes + lane);
    }
    if (tid < 8) ctl[tid] = tid == 1 ? kAllAvail : 0u;
    if (kMode == kModeGaussian) stage_scales<kDecThreads>(scl, a.scale_table, a.n_scales, tid);
    stage_late<kDecThreads, kSearch>(tb, est, lmeta, a.nd_cap ? lsub : nullptr,
                                     (uint32_t)a.nd_cap, bd, tid);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no load crosses the role split
    if (wid == 0) pc.mark(2);

    // The coder, the mappers and the escape reader run separate code (the
    // wave role is uniform per wave) that meets at the same barriers: one
    // before the first block and one per block, and one after the mappers'
    // last store.
    if (wid == 0) {
      x = lane < A ? x : kStateLow;
#pragma unroll
      for (int b = 0; b < G::kPre; ++b)
#pragma unroll
        for (int kk = 0; kk < G::kPfU32; ++kk)
          sring32[(b * (G::kPfWords / 2) + kk * kLanes + lane) & (G::kRing / 2 - 1)] = w0[b][kk];
      S.filled = G::kPre * G::kPfWords;
      uint32_t ecur = 0;  // escape entries consumed
      // The coder's chain of dependent steps bounds the block loop; its
      // instructions go first when mapper or escape waves of this or another
      // workgroup on the CU compete for the same SIMD.
      __builtin_amdgcn_s_setprio(3);
      __syncthreads();
      pc.mark(3);
      pc.cycles(12);
      for (int j = 0; j < nblk; ++j) {
        uint2* src = recs + (j & 1) * SB * kLanes;
        uint4* ei = escm + (j & 1) * SB;
        uint2 r[SB];
        uint32_t ov[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) r[u] = src[u * kLanes + lane];
        // steps whose tables are not all in LDS; cleared for block j + 2 (the
        // search lookups stage every table: no read, no wait)
        const uint32_t nl = kSearch ? 0u : (uint32_t)uni((int)ctl[2 + (j & 1)]);
        if (!kSearch) ctl[2 + (j & 1)] = 0u;  // every lane: no exec-mask branch
        // after the block's LDS reads: the compiler makes the first LDS read
        // after the prefetch loads wait for them, so they are issued after
        // the records are read and return during the block's steps
        stream_block_start<SB>(S, sring32, lane);
        uint64_t any_em = 0;
        if ((j + 1) * SB * kLanes <= len && nl == 0 && offsets_safe) {
          // common case: every lane of the block active, LDS tables, no
          // per-step branches
          uint64_t em[SB];
#pragma unroll
          for (int u = 0; u < SB; ++u) {
            ov[u] = dec_step<true, true, SB, kSearch, kWide, kSkip>(tb, r[u], x, S, sring, em[u],
                                                                 status, lane);
            any_em |= em[u];
          }
          if (__builtin_expect(any_em != 0ull, 0)) {
#pragma unroll
            for (int u = 0; u < SB; ++u) {
              if (lane == 0) ei[u] = make_uint4((uint32_t)em[u], (uint32_t)(em[u] >> 32), ecur, 0u);
              ecur += (uint32_t)__popcll(em[u]);
            }
          }
          // decoded values replace the records' x words (y with the search
          // lookups); the mappers store them
#pragma unroll
          for (int u = 0; u < SB; ++u) {
            if constexpr (kSearch) src[u * kLanes + lane].y = ov[u];
            else src[u * kLanes + lane].x = ov[u];
          }
        } else {
          // last block or tables outside LDS: one step at a time
#pragma unroll 1
          for (int u = 0; u < SB && j * SB + u < T; ++u) {
            const uint2 ru = src[u * kLanes + lane];
            uint64_t em;
            uint32_t v;
            if constexpr (kSearch) {
              v = dec_step<true, false, SB, true>(tb, ru, x, S, sring, em, status, lane);
            } else {
              v = ((nl >> u) & 1u) == 0u
                      ? dec_step<true, false, SB, false, kWide>(tb, ru, x, S, sring, em, status,
                                                               lane)
                      : dec_step<false, false, SB, false, kWide>(tb, ru, x, S, sring, em, status,
                                                                lane);
            }
            if (lane == 0) ei[u] = make_uint4((uint32_t)em, (uint32_t)(em >> 32), ecur, 0u);
            ecur += (uint32_t)__popcll(em);
            any_em |= em;
            if constexpr (kSearch) src[u * kLanes + lane].y = v;
            else src[u * kLanes + lane].x = v;
          }
        }
        // every lane writes the same (uniform) values: no exec-mask branch
        ctl[4 + (j & 1)] = any_em != 0ull ? 1u : 0u;
        ctl[6 + ((j + 1) & 1)] = ecur;
        pc.bar_in();
        __syncthreads();
        pc.bar_out();
      }
      pc.cycles(13);
      pc.mark(4);
      if (lane < A && x != kStateLow) status |= GAANS_ST_CORRUPT;
      publish();
      __syncthreads();  // after the mappers' last store
    } else if (wid == kEscWave) {
      __syncthreads();
      for (int j = 0; j < nblk; ++j) {
        // the entries of block j: at most SB kLanes past those consumed before it
        esc_parse<R>(E, (uint32_t)uni((int)ctl[6 + (j & 1)]) + (uint32_t)(SB * kLanes), fifo, ctl,
                     lane);
        __syncthreads();
      }
      publish();
      __syncthreads();
    } else {
      if (kMode == kModeGaussian) gc = gauss_coarse(scl, a.n_scales);  // staged, published
      if (nblk > 0) map_block(0);
      __syncthreads();
      for (int j = 0; j < nblk; ++j) {
        // mappers: store block j - 1 and map block j + 1 while the coder decodes block j
        if (j > 0) store_block(j - 1, false);
        if (j + 1 < nblk) {
#pragma unroll
          for (int e = 0; e < kPer; ++e) {
            cbx[e] = nbx[e];
            cm[e] = nm[e];
          }
          if (j + 2 < nblk) load_block(j + 2, nbx, nm);
          map_block(j + 1);
        }
        __syncthreads();
      }
      if (nblk > 0) store_block(nblk - 1, true);
      else publish();
      __syncthreads();
    }
  }
  if (!ok) {  // uniform
    // the early copies into LDS have landed before the workgroup ends
    __builtin_amdgcn_s_waitcnt(0x0F70);
    publish();
    __syncthreads();
  }
  if (tid == 0) {
    uint32_t hs = 0, st = 0, eq = 0;
    for (int w = 0; w < kDecWaves; ++w) {
      hs += part[w];
      st |= part[kDecWaves + w];
      eq += part[2 * kDecWaves + w];
    }
    if (ok) {
      if (hs != want_hash) st |= GAANS_ST_INDEXHASH;
      // stream, pad and escape words consumed exactly (eq escape nibbles);
      // the pad word and the unused nibbles of the last escape word are zero
      const int qe = (int)((eq + 3u) >> 2);
      const int pad = (S.rp + qe) & 1;
      if (S.rp + qe + pad != S.q) {
        st |= GAANS_ST_CORRUPT;
      } else {
        // u16 word i of the stream: from the ring while it still holds it
        // (the ring keeps the last kRing words committed, [filled - kRing,
        // filled)), else from global memory
        const uint16_t* s16 = reinterpret_cast<const uint16_t*>(S.s32);
        auto word16 = [&](int i) -> uint32_t {
          if (i < S.filled && i >= S.filled - G::kRing) return sring[i & (G::kRing - 1)];
          return s16[i];
        };
        if (pad && word16(S.rp) != 0) st |= GAANS_ST_CORRUPT;
        if (eq & 3u) {
          // escape u32 eq >> 3 holds the first unused nibble (in range: the
          // words were consumed exactly); its halves are swapped in the stream
          const int m = S.q32 - 1 - (int)(eq >> 3);
          const uint32_t v = word16(2 * m + 1) | (word16(2 * m) << 16);
          const uint32_t last = v >> (4u * (eq & 7u));
          if (last & ((1u << (4u * (4u - (eq & 3u)))) - 1u)) st |= GAANS_ST_CORRUPT;
        }
      }
    }
    // Completion counter: one u64, units done in the low half, the OR of
    // the units' status bits in the high half.  A unit with status ORs it in
    // first (and waits for it); atomics on one address take effect in
    // program order, so the add that returns units - 1 done carries every
    // unit's status.  No fence: decoded values need no visibility before
    // the kernel ends.
    uint64_t* done = reinterpret_cast<uint64_t*>(a.ctrl + kCtrlDecDone);
    if (st) {
      __hip_atomic_fetch_or(done, (uint64_t)st << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    pc.mark(5);
    const uint64_t old = __hip_atomic_fetch_add(done, 1ull, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    pc.mark_after_loads(6);  // the atomic returned
    pc.store(a.phase, g, 0, 7);
    if ((uint32_t)old == (uint32_t)(a.units - 1)) {
      const uint32_t all = (uint32_t)(old >> 32);
      a.status_out[0] = all;
      // completion word with the status, one store (no system-wide write-back)
      __hip_atomic_store(&a.status_out[1], 1u | (all << 1), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(done, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pc.store_done(a.phase, g);
    }
  }
}

// ============================================================================
// CompressAI Rans64 streams: one stream per batch row, one lane per stream
// ============================================================================
//
// CompressAI's RansEncoder.encode_with_indexes writes one serial Rans64
// stream per image (64-bit state, L = 2^31, 32-bit words, 16-bit CDFs,
// escapes as 4-bit bypass groups).  One stream cannot be split, so a wave
// decodes up to 64 of them side by side, lane l < spw the stream of row
// spw * blockIdx.x + l, in lockstep over positions.  Lanes of one wave
// diverge at dense lookups and escapes, so the host spreads small batches
// over more waves (down to one stream per wave).  A step: cum = x & 0xffff;
// the prepared tables' decode lookup (LDS, same entries as the GA-ANS
// decoder); x = freq * (x >> 16) + cum - start; one word when x < 2^31.
// Words come from a per-lane LDS ring that the wave refills kR64Pf words at a
// time from registers loaded one refill earlier (so their latency is off the
// chain); a lane that runs its ring dry (long escapes) reads global memory.
// Tables: all staged at the start when they fit; otherwise, with implicit
// indexes (table = channel: every lane is in the same channel at the same
// step), the current channel's table is staged when the channel changes;
// otherwise lookups read global memory.

constexpr int kCtrlR64Done = 32;
constexpr int kCtrlR64Status = 33;
constexpr uint64_t kR64L = 1ull << 31;
constexpr int kR64Steps = 32;                 // steps between ring refills
constexpr int kR64Ring = 128;                 // ring words per lane (power of two)
constexpr int kR64Pf = 32;                    // words per lane per refill
constexpr int kR64RingBytes = 4 * kR64Ring * kLanes;
constexpr int kR64SubCap = 64;                // sub-blocks staged with one channel's table
constexpr int kR64IdxBytes = 4 * kR64Steps * kLanes;  // explicit indexes of one block

struct R64Args {
  const uint8_t* __restrict__ streams;
  int64_t streams_bytes;
  const int64_t* __restrict__ offsets;  // B + 1 byte offsets
  const int32_t* __restrict__ indexes;  // [B, N], or NULL: table = position / HW
  const uint8_t* __restrict__ tables;
  uint32_t M, tables_bytes;
  BlobRef blob;
  int64_t B, N;
  UDiv div_hw;
  int32_t stage;       // 0: global lookups, 1: all tables staged, 2: one channel at a time
  int32_t stage_subs;  // sub-blocks staged too
  uint32_t lds_tabs;   // LDS byte offset of [luts][meta][sub-blocks] (after ring, indexes)
  int32_t nt_cap;      // tables the LDS lookups hold
  int32_t* __restrict__ out;
  uint32_t* __restrict__ ctrl;
  uint32_t* __restrict__ status_out;
  uint32_t nblocks;
  int32_t spw;  // streams per wave (lanes 0 .. spw - 1)
};

struct R64Stream {
  const uint32_t* __restrict__ w;  // the lane's words
  int q;                           // words in the stream (0: no valid stream)
  int rp, filled;                  // next word; words placed in the ring
  uint32_t pf[kR64Pf];             // the next refill
  bool bad;
};

__device__ __forceinline__ void r64_prefetch(R64Stream& S) {
#pragma unroll
  for (int k = 0; k < kR64Pf; ++k) {
    const int i = S.filled + k;
    S.pf[k] = 0u;
    if (i < S.q) S.pf[k] = S.w[i];
  }
}

// Refill: lanes with room commit their prefetched words and load the next.
__device__ __forceinline__ void r64_refill(R64Stream& S, uint32_t* ring, int lane) {
  const bool need = S.filled - S.rp <= kR64Ring - kR64Pf && S.filled < S.q;
  if (ballot(need) == 0ull) return;
  if (need) {
#pragma unroll
    for (int k = 0; k < kR64Pf; ++k)
      ring[((S.filled + k) & (kR64Ring - 1)) * kLanes + lane] = S.pf[k];
    S.filled += kR64Pf;
    r64_prefetch(S);
  }
}

__device__ __forceinline__ uint32_t r64_next(R64Stream& S, const uint32_t* ring, int lane) {
  uint32_t v = 0u;
  if (S.rp < S.filled) {
    v = ring[(S.rp & (kR64Ring - 1)) * kLanes + lane];
  } else if (S.rp < S.q) {
    v = S.w[S.rp];
  }
  S.bad |= S.rp >= S.q;
  ++S.rp;
  return v;
}

__device__ __forceinline__ uint32_t r64_bits4(R64Stream& S, uint64_t& x, const uint32_t* ring,
                                              int lane) {
  const uint32_t v = (uint32_t)x & 15u;
  x >>= 4;
  if (x < kR64L) x = (x << 32) | r64_next(S, ring, lane);
  return v;
}

template <bool kImplicit>
__global__ void __launch_bounds__(kLanes) k_rans64_decode(R64Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint32_t* ring = reinterpret_cast<uint32_t*>(smem);
  int32_t* ibuf = reinterpret_cast<int32_t*>(smem + kR64RingBytes);  // explicit indexes
  uint8_t* tsm = smem + a.lds_tabs;
  uint64_t* llut = reinterpret_cast<uint64_t*>(tsm);
  uint4* lmeta = reinterpret_cast<uint4*>(tsm + 8 * kLutSize * a.nt_cap);
  uint64_t* lsub = reinterpret_cast<uint64_t*>(tsm + (8 * kLutSize + 16) * a.nt_cap);

  const int lane = threadIdx.x;
  const int64_t b = (int64_t)blockIdx.x * a.spw + lane;
  const bool live = lane < a.spw && b < a.B;
  uint32_t status = 0;
  const bool tab = tables_ok(load_tab_hdr(a.tables), a.M, a.tables_bytes, a.blob);
  if (!tab) status |= GAANS_ST_TABLES;

  // the lane's stream: [off_b, off_b+1) inside the buffer, whole words
  R64Stream S;
  S.w = reinterpret_cast<const uint32_t*>(a.streams);
  S.q = 0;
  S.rp = 0;
  S.filled = 0;
  S.bad = false;
  if (live) {
    const int64_t o0 = a.offsets[b], o1 = a.offsets[b + 1];
    const bool fits = o0 >= 0 && o1 >= o0 && o1 <= a.streams_bytes && (o0 & 3) == 0 &&
                      ((o1 - o0) & 3) == 0 && (o1 - o0) / 4 <= 0x7fffffff - 2 * kR64Pf;
    if (fits && o1 - o0 >= 8 && a.N > 0) {
      S.w = reinterpret_cast<const uint32_t*>(a.streams + o0);
      S.q = (int)((o1 - o0) / 4);
    } else if (a.N > 0) {
      status |= GAANS_ST_CORRUPT;  // CompressAI's decoder needs the two state words
    }
  }
  const bool act0 = live && S.q > 0 && tab;

  // first refill: state words and the ring, then the next batch in flight
  r64_prefetch(S);
  r64_refill(S, ring, lane);
  uint64_t x = 0;
  if (act0) {
    const uint32_t lo = r64_next(S, ring, lane), hi = r64_next(S, ring, lane);
    x = (uint64_t)lo | ((uint64_t)hi << 32);
  }

  Tabs tb;
  tb.gmeta = reinterpret_cast<const TabMeta*>(a.tables + a.blob.meta_off);
  tb.gent = nullptr;
  tb.glut = reinterpret_cast<const uint64_t*>(a.tables + a.blob.lut_off);
  tb.gsub = reinterpret_cast<const uint64_t*>(a.tables + a.blob.dense_off);
  tb.lmeta = lmeta;
  tb.lent = nullptr;
  tb.llut = llut;
  tb.lsub = lsub;
  tb.t_lo = 0;
  tb.nt = 0;
  tb.sub_first = 0;
  tb.sub_n = 0;
  const bool any = ballot(act0) != 0ull;
  const uint32_t total_dense = a.blob.total_dense;
  if (any && a.stage == 1)
    stage_tables<kLanes>(tb, lmeta, nullptr, llut, a.stage_subs ? lsub : nullptr,
                         stage_bounds(tb.gmeta, 0, (int)a.M, a.M, total_dense), 0, (int)a.M,
                         lane);
  int cur = -1;  // staged channel (stage 2)
  uint32_t c_nsym = 0;
  int32_t c_off = 0;

  const int64_t row = live ? b * a.N : 0;
  const int64_t nsteps = any ? a.N : 0;
  // explicit indexes: block j + 1's are loaded into registers while block j
  // runs, then stored to LDS at block j + 1's start
  int32_t nb[kR64Steps];
  auto load_indexes = [&](int64_t i0) {
#pragma unroll
    for (int k = 0; k < kR64Steps; ++k) {
      nb[k] = 0;
      if (act0 && i0 + k < nsteps) nb[k] = a.indexes[row + i0 + k];
    }
  };
  if (!kImplicit) load_indexes(0);
  for (int64_t i0 = 0; i0 < nsteps; i0 += kR64Steps) {
    if (!kImplicit) {
#pragma unroll
      for (int k = 0; k < kR64Steps; ++k) ibuf[k * kLanes + lane] = nb[k];
      load_indexes(i0 + kR64Steps);
    }
    r64_refill(S, ring, lane);
    const int n = nsteps - i0 < kR64Steps ? (int)(nsteps - i0) : kR64Steps;
#pragma unroll 1
    for (int k = 0; k < n; ++k) {
      const int64_t i = i0 + k;
      const bool act = act0 & !S.bad;
      uint32_t t;
      if (kImplicit) {
        // the same in every lane: stage the channel's table when it changes
        const int tc = uni((int)udiv((uint32_t)i, a.div_hw));
        if (__builtin_expect(a.stage == 2 && tc != cur, 0)) {
          cur = tc;
          stage_tables<kLanes>(tb, lmeta, nullptr, llut, a.stage_subs ? lsub : nullptr,
                               stage_bounds(tb.gmeta, cur, cur + 1, a.M, total_dense), cur,
                               cur + 1, lane);
          const uint4 lm = lmeta[0];
          c_nsym = lm.y;
          c_off = (int32_t)lm.z;
        }
        t = (uint32_t)tc;
      } else {
        t = (uint32_t)ibuf[k * kLanes + lane];
      }
      const bool bad_t = act & (t >= a.M);
      status |= bad_t ? GAANS_ST_INDEX : 0u;
      const bool ok = act & !bad_t;
      t = ok ? t : 0u;
      uint32_t nsym;
      int32_t off;
      uint32_t tl = t;
      if (a.stage == 2) {
        nsym = c_nsym;
        off = c_off;
        tl = 0u;
      } else if (a.stage == 1) {
        const uint4 lm = lmeta[t];
        nsym = lm.y;
        off = (int32_t)lm.z;
      } else {
        const TabMeta gm = tb.gmeta[t];
        nsym = gm.nsym;
        off = gm.offset;
      }
      const uint32_t cum = (uint32_t)x & 0xffffu;
      uint32_t s, st, fr;
      if (a.stage != 0) dec_lookup<true>(tb, tl << kLutBits, cum, ok, s, st, fr);
      else dec_lookup<false>(tb, tl, cum, ok, s, st, fr);
      x = (uint64_t)fr * (x >> 16) + cum - st;
      if (ok && x < kR64L) x = (x << 32) | r64_next(S, ring, lane);
      int64_t v = (int64_t)s + off;
      if (ok && s == nsym - 1u) {  // escape: 4-bit count, then the raw value's nibbles
        uint32_t cnt = r64_bits4(S, x, ring, lane);
        if (cnt > 8u) {  // 15 continues the count: never for a 32-bit value
          S.bad = true;
          cnt = 0u;
        }
        uint32_t raw = 0;
        for (uint32_t j = 0; j < cnt; ++j) raw |= r64_bits4(S, x, ring, lane) << (4u * j);
        const int64_t u = (raw & 1u) ? -(int64_t)(raw >> 1) - 1
                                     : (int64_t)(raw >> 1) + (int64_t)(nsym - 1u);
        v = u + off;
        if (v < INT32_MIN || v > INT32_MAX) S.bad = true;
      }
      if (ok) a.out[row + i] = (int32_t)v;
    }
  }
  if (act0 && S.bad) status |= GAANS_ST_CORRUPT;

  status = wave_or(status);
  if (lane == 0) {
    if (status)
      __hip_atomic_fetch_or(&a.ctrl[kCtrlR64Status], status, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint32_t done = __hip_atomic_fetch_add(&a.ctrl[kCtrlR64Done], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    if (done == a.nblocks - 1u) {
      const uint32_t all = __hip_atomic_exchange(&a.ctrl[kCtrlR64Status], 0u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
      a.status_out[0] = all;
      __hip_atomic_store(&a.status_out[1], 1u | (all << 1), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(&a.ctrl[kCtrlR64Done], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
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
  if (t->M < 1 || t->M > 65536) return fail(GAANS_EINVAL, "table count M must be in [1, 65536]");
  if (t->bytes < (int64_t)sizeof(TabHdr) || t->bytes > 0xffffffffll)
    return fail(GAANS_EINVAL, "tables bytes %lld out of range", (long long)t->bytes);
  if (t->max_nsym < 1 || t->total_nsym < t->max_nsym || t->max_dense < 0 ||
      t->total_dense < t->max_dense || t->max_wide < 0 || t->total_wide < t->max_wide ||
      t->total_wide > 0xffffffffll)
    return fail(GAANS_EINVAL, "tables descriptor is inconsistent");
  return GAANS_OK;
}

// Section offsets of the blob a descriptor describes (the layout written by
// gaans_tables_prepare); the descriptor's size must match them.
int blob_ref(const gaans_tables* t, BlobRef* r) {
  const bool wide = (t->flags & GAANS_TABLES_WIDE) != 0;
  if (wide != (t->M <= kWideMaxTables))
    return fail(GAANS_EINVAL, "tables descriptor: wide lookups exist exactly for M <= %d",
                kWideMaxTables);
  const BlobLayout L = blob_layout(t->M, t->total_nsym, t->total_dense, wide, t->total_wide);
  if (L.end != t->bytes)
    return fail(GAANS_EINVAL, "tables descriptor does not describe a prepared blob (%lld bytes "
                "for its counts, %lld given)", (long long)L.end, (long long)t->bytes);
  r->meta_off = (uint32_t)sizeof(TabHdr);
  r->ent_off = (uint32_t)L.ent_off;
  r->lut_off = (uint32_t)L.lut_off;
  r->dense_off = (uint32_t)L.dense_off;
  r->total_dense = (uint32_t)t->total_dense;
  r->clut_off = (uint32_t)L.clut_off;
  r->starts_off = (uint32_t)L.starts_off;
  r->wide_off = (uint32_t)L.wide_off;
  r->wdense_off = (uint32_t)L.wdense_off;
  r->wbase_off = (uint32_t)L.wbase_off;
  r->total_wide = (uint32_t)t->total_wide;
  return GAANS_OK;
}

// LDS of the current device: per workgroup and per CU, and the CU count
// (queried once per device).
struct DevLds {
  int per_block, per_cu, cus, dev;
};

int device_lds(DevLds* out) {
  static DevLds cache[kMaxDevices];
  static int ready[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(GAANS_EHIP, "hipGetDevice failed");
  if (!__atomic_load_n(&ready[dev], __ATOMIC_ACQUIRE)) {
    DevLds d{0, 0, 0, dev};
    if (hipDeviceGetAttribute(&d.per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) !=
            hipSuccess ||
        hipDeviceGetAttribute(&d.per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                              dev) != hipSuccess ||
        hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        d.per_block <= 0 || d.cus <= 0)
      return fail(GAANS_EHIP, "device attribute query failed");
    if (d.per_cu < d.per_block) d.per_cu = d.per_block;
    d.dev = dev;
    cache[dev] = d;
    __atomic_store_n(&ready[dev], 1, __ATOMIC_RELEASE);
  }
  *out = cache[dev];
  return GAANS_OK;
}

// LDS staging plan for a launch of `units` workgroups: all tables if they fit
// and are not much larger than a chunk's channel range, else that range (P
// tables, bounded by P times the largest table), else none.  The budget per
// workgroup keeps the launch in one round of workgroups when the tables allow
// it (units / CUs workgroups per CU), and otherwise gives up workgroups per CU
// before it gives up staging.
struct Stage {
  int32_t nt_cap, ne_cap, nd_cap, stage_all;
};

// LDS of one workgroup when occ workgroups share a CU: the CU's LDS divided
// by occ, rounded down to 1 KB, less 1 KB when several share it (measured on
// MI355X: three workgroups of 53,632 bytes fit on a CU, three of 54,272 do
// not).
int64_t lds_budget(const DevLds& d, int64_t occ) {
  int64_t b = d.per_cu / occ;
  if (b > d.per_block) b = d.per_block;
  b = b / 1024 * 1024;
  return occ > 1 ? b - 1024 : b;
}

// Workgroups per CU that keep a launch of units workgroups in one round.
int64_t occ_target(int64_t units, const DevLds& d, int64_t max_occ) {
  int64_t occ = (units + d.cus - 1) / d.cus;
  return occ > max_occ ? max_occ : (occ < 1 ? 1 : occ);
}

// Tables staged in `budget` bytes (per table, per symbol entry and per dense
// block costs): false if not even the chunk's range fits.
// wide: the sub-blocks are the wide lookups' (max_wide, total_wide).
bool fit_stage(const gaans_tables* t, int64_t P, int64_t per_table, int64_t per_sym,
               int64_t per_dense, int64_t budget, Stage* s, bool range_ok = true,
               bool wide = false) {
  const int64_t max_d = wide ? t->max_wide : t->max_dense;
  const int64_t total_d = wide ? t->total_wide : t->total_dense;
  const int64_t all = t->M * per_table + per_sym * t->total_nsym + per_dense * total_d;
  const int64_t range = P * (per_table + per_sym * (int64_t)t->max_nsym + per_dense * max_d);
  // all tables when that is not much more to copy than the chunk's range
  // (or the range does not fit): explicit indexes may use any table
  if (all <= budget && (all <= 2 * range || range > budget)) {
    *s = Stage{t->M, per_sym ? (int32_t)t->total_nsym : 0, per_dense ? (int32_t)total_d : 0, 1};
    return true;
  }
  if (range_ok && range <= budget) {
    *s = Stage{(int32_t)P, per_sym ? (int32_t)(P * t->max_nsym) : 0,
               per_dense ? (int32_t)(P * max_d) : 0, 0};
    return true;
  }
  return false;
}

// Encoder: metadata and both entry words per symbol; 8-step blocks, else
// 4-step blocks (half the records) for each workgroups-per-CU count.
struct EncPlan {
  Stage st;
  int sb;
  size_t lds;
  int64_t occ;  // workgroups per CU the plan allows
  int ring;     // output ring words
};

// `extra` LDS bytes follow the tables (the Gaussian mode's scale table);
// range_ok is false when any table may serve any position (per-element
// indexes computed from scales), so only all tables or none are staged.
// For each block size the output ring shrinks from 4096 words to 2048 and
// 1024 (never below two blocks' worst case) before the block size does:
// a smaller ring only flushes more often, a smaller block doubles the
// per-block work (the batch-64 uniform workload's 16 staged tables of 255
// symbols fit next to 8-step blocks with a 1024-word ring).
EncPlan plan_encode(const gaans_tables* t, int64_t P, int64_t units, const DevLds& d,
                    int64_t extra = 0, bool range_ok = true,
                    bool allow16 = false) {
  for (int64_t occ = occ_target(units, d, 4); occ >= 1; --occ)
    for (int sb = allow16 ? 16 : 8; sb >= 4; sb >>= 1)
      for (int ring = kRingWords; ring >= 2 * sb * kLanes && ring >= 1024; ring >>= 1) {
        Stage s;
        // + 2 entries: the staged copy starts at an even entry and ends on a
        // whole 16-byte word (stage_tables)
        const int64_t fixed = enc_fixed_lds(sb, ring) + 16;
        if (fit_stage(t, P, 16, 8, 0, lds_budget(d, occ) - fixed - extra, &s, range_ok))
          return EncPlan{s, sb,
                         (size_t)(fixed + 16 * (int64_t)s.nt_cap + 8 * (int64_t)s.ne_cap), occ,
                         ring};
      }
  // no tables staged (they read through L1/L2): the largest block allowed
  const int sb = allow16 ? 16 : 8;
  return EncPlan{Stage{0, 0, 0, 0}, sb, (size_t)enc_fixed_lds(sb, kRingWords), 1, kRingWords};
}

// Decoder: lookups and metadata per table; sub-blocks when they are staged
// too.  For each workgroups-per-CU count (at most 3: the kernel is built for
// 6 waves per SIMD, and a 6-wave workgroup puts two waves on two of the CU's
// four SIMDs), the options in order of preference: 8-step blocks with
// sub-blocks, 4-step blocks with sub-blocks (their records, stream ring and
// escape FIFO take half the LDS); then, when the blob has them and every
// position may use any table (explicit or computed indexes), the search
// lookups of all tables; then the lookups without sub-blocks (a dense-bucket
// lookup then reads global memory).
struct DecPlan {
  Stage st;
  int sb;
  size_t lds;
  bool search;            // the search lookups of every table
  uint32_t starts_words;  // search: 16-byte words of starts
  bool wide;              // the wide lookups
};

// Search lookups in LDS: every table's bucket entries and metadata, and
// every symbol's start (with the zero padding).
int64_t search_lds(const gaans_tables* t, uint32_t* starts_words) {
  const int64_t sb = align_up(2 * search_starts(t->M, t->total_nsym), 16);
  *starts_words = (uint32_t)(sb / 16);
  return (int64_t)t->M * (4 * kSearchEntries + 16) + sb;
}

DecPlan plan_decode(const gaans_tables* t, int64_t P, int64_t units, bool latents,
                    const DevLds& d, int64_t extra = 0, bool range_ok = true,
                    bool search_ok = false) {
  const int64_t per_table = 8 * kLutSize + 16;
  const int64_t per_wide = 8 * kWideSize + 16;
  const bool wide_ok = (t->flags & GAANS_TABLES_WIDE) != 0;
  const bool has_dense = t->total_dense > 0;
  uint32_t starts_words = 0;
  const int64_t search_bytes = search_ok ? search_lds(t, &starts_words) : 0;
  for (int64_t occ = occ_target(units, d, 3); occ >= 1; --occ) {
    const int64_t cap = lds_budget(d, occ);
    // The wide lookups with 16- or 8-step blocks and: all of a range's
    // sub-blocks (room for P times the largest per table); else as many as
    // the rest of the LDS holds when that is half again a typical range's
    // count (P times the mean per table), a unit staging its range's first
    // ones and reading the others from global memory (the 2160x3840
    // latent's chunks of 8 tables need 30-115 sub-blocks, 8 x 26 by the
    // bound; 8-step blocks leave room for 123); else none (a dense wide
    // bucket then reads its two-value sub-range from global memory, where
    // the 256-value buckets gave the wide-table units a second or third
    // read in most steps).
    const int64_t typical = (P * t->total_wide + t->M - 1) / t->M * 3 / 2;
    for (int subs = 2; wide_ok && subs >= 0; --subs)
      for (int sb = 16; sb >= 8; sb >>= 1) {
        const int64_t fixed = dec_fixed_lds(latents, sb);
        Stage s;
        if (!fit_stage(t, P, per_wide, 0, subs == 2 ? kSubBytes : 0, cap - fixed - extra, &s,
                       range_ok, true))
          continue;
        if (subs == 1) {  // partial: the sub-blocks the rest of the LDS holds
          const int64_t room = (cap - fixed - extra - per_wide * s.nt_cap) / kSubBytes;
          if (t->total_wide == 0 || room < typical || room < 1) continue;
          s.nd_cap = (int32_t)(room < (int64_t)t->total_wide ? room : t->total_wide);
        }
        return DecPlan{s, sb,
                       (size_t)(fixed + per_wide * s.nt_cap + kSubBytes * (int64_t)s.nd_cap),
                       false, 0, true};
      }
    for (int opt = 0; opt < 9; ++opt) {
      const int sb = 16 >> (opt % 3);  // 16-, 8-, then 4-step blocks of each kind
      const int64_t fixed = dec_fixed_lds(latents, sb);
      if (opt >= 3 && !has_dense) break;  // same as the options already tried
      if (opt >= 3 && opt < 6) {
        if (search_ok && fixed + search_bytes + extra <= cap)
          return DecPlan{Stage{(int32_t)t->M, 0, 0, 1}, sb, (size_t)(fixed + search_bytes), true,
                         starts_words, false};
        continue;
      }
      const bool dense = opt < 3;
      Stage s;
      if (fit_stage(t, P, per_table, 0, dense ? kSubBytes : 0, cap - fixed - extra, &s, range_ok))
        return DecPlan{s, sb,
                       (size_t)(fixed + per_table * s.nt_cap + kSubBytes * (int64_t)s.nd_cap),
                       false, 0, false};
    }
  }
  return DecPlan{Stage{0, 0, 0, 0}, 8, (size_t)dec_fixed_lds(latents, 8), false, 0, false};
}

// Allow dynamic LDS above the default limit (once per kernel and device).
int allow_lds(const void* kernel, size_t bytes, const DevLds& d) {
  if (bytes <= 64 * 1024) return GAANS_OK;
  static std::mutex mu;
  static const void* done_fn[64];
  static int done_dev[64];
  static int n_done = 0;
  std::lock_guard<std::mutex> g(mu);
  for (int i = 0; i < n_done; ++i)
    if (done_fn[i] == kernel && done_dev[i] == d.dev) return GAANS_OK;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, d.per_block) !=
      hipSuccess)
    return fail(GAANS_EHIP, "cannot raise the LDS limit of a kernel to %d bytes", d.per_block);
  if (n_done < 64) {
    done_fn[n_done] = kernel;
    done_dev[n_done++] = d.dev;
  }
  return GAANS_OK;
}

// Gaussian-mode inputs (CompressAI GaussianConditional with a scale table).
struct GaussIn {
  const float* means;   // per element, or NULL
  const float* scales;  // per element
  const float* table;   // n non-decreasing scales (device memory)
  int32_t n;
  float bound;
};

// Scale-table entries: the table is staged in LDS beside the coding tables.
constexpr int32_t kMaxScales = 8192;

int check_gauss(const GaussIn* g) {
  if (!g->scales || !g->table) return fail(GAANS_EINVAL, "scales or scale table pointer is NULL");
  if (g->n < 1 || g->n > kMaxScales)
    return fail(GAANS_EINVAL, "scale table of %d entries outside [1, %d]", g->n, kMaxScales);
  return GAANS_OK;
}

int32_t pow2_floor(int32_t v) {  // largest power of two <= v (0 for v < 1)
  int32_t p = 0;
  while (v > 0 && (p == 0 || ((int64_t)p << 1) <= v)) p = p ? p << 1 : 1;
  return p;
}

// Kernel of a launch: template arguments chosen at run time.
using EncKernel = void (*)(EncArgs);
using DecKernel = void (*)(DecArgs);

template <int kMode, bool kImp, int SB>
EncKernel enc_kernel_nm(int nm) {
  return nm == 8 ? k_encode<kMode, kImp, SB, 8> : k_encode<kMode, kImp, SB, 4>;
}

template <int kMode, bool kImp>
EncKernel enc_kernel_sb(int sb, int nm) {
  return sb == 4 ? enc_kernel_nm<kMode, kImp, 4>(nm) : enc_kernel_nm<kMode, kImp, 8>(nm);
}

// Encode kernel of a mode, index kind, block size and mapper count; 16-step
// blocks are built for explicit or computed indexes only (with table =
// channel the 16-step kernel needs private scratch).
EncKernel enc_kernel(int mode, bool imp, int sb, int nm) {
  if (sb == 16) {
    switch (mode) {
      case kModeGaussian: return enc_kernel_nm<kModeGaussian, false, 16>(nm);
      case kModeLatents: return enc_kernel_nm<kModeLatents, false, 16>(nm);
      default: return enc_kernel_nm<kModeSymbols, false, 16>(nm);
    }
  }
  switch (mode) {
    case kModeGaussian: return enc_kernel_sb<kModeGaussian, false>(sb, nm);
    case kModeLatents:
      return imp ? enc_kernel_sb<kModeLatents, true>(sb, nm)
                 : enc_kernel_sb<kModeLatents, false>(sb, nm);
    default:
      return imp ? enc_kernel_sb<kModeSymbols, true>(sb, nm)
                 : enc_kernel_sb<kModeSymbols, false>(sb, nm);
  }
}

template <int kMode, bool kImp, bool kSearch, bool kWide = false, bool kSkip = false>
DecKernel dec_kernel_sb(int sb) {
  return sb == 4 ? k_decode<kMode, kImp, 4, kSearch, kWide, kSkip>
                 : (sb == 8 ? k_decode<kMode, kImp, 8, kSearch, kWide, kSkip>
                            : k_decode<kMode, kImp, 16, kSearch, kWide, kSkip>);
}

// Decode kernel of a mode, index kind, block size and lookup kind (the
// search lookups serve explicit or computed indexes only; the wide lookups
// are staged with 8- or 16-step blocks only).  skip: the variant whose steps
// skip the refill read when no lane refills, for the 256-bucket lookups.
DecKernel dec_kernel(int mode, bool imp, int sb, bool search, bool wide, bool skip) {
  if (search) {
    switch (mode) {
      case kModeGaussian: return dec_kernel_sb<kModeGaussian, false, true>(sb);
      case kModeLatents: return dec_kernel_sb<kModeLatents, false, true>(sb);
      default: return dec_kernel_sb<kModeSymbols, false, true>(sb);
    }
  }
  if (wide) {
    const int w = sb == 8 ? 8 : 16;
    switch (mode) {
      case kModeGaussian:
        return w == 8 ? k_decode<kModeGaussian, false, 8, false, true>
                      : k_decode<kModeGaussian, false, 16, false, true>;
      case kModeLatents:
        return imp ? (w == 8 ? k_decode<kModeLatents, true, 8, false, true>
                             : k_decode<kModeLatents, true, 16, false, true>)
                   : (w == 8 ? k_decode<kModeLatents, false, 8, false, true>
                             : k_decode<kModeLatents, false, 16, false, true>);
      default:
        return imp ? (w == 8 ? k_decode<kModeSymbols, true, 8, false, true>
                             : k_decode<kModeSymbols, true, 16, false, true>)
                   : (w == 8 ? k_decode<kModeSymbols, false, 8, false, true>
                             : k_decode<kModeSymbols, false, 16, false, true>);
    }
  }
  if (skip) {
    switch (mode) {
      case kModeGaussian: return dec_kernel_sb<kModeGaussian, false, false, false, true>(sb);
      case kModeLatents:
        return imp ? dec_kernel_sb<kModeLatents, true, false, false, true>(sb)
                   : dec_kernel_sb<kModeLatents, false, false, false, true>(sb);
      default:
        return imp ? dec_kernel_sb<kModeSymbols, true, false, false, true>(sb)
                   : dec_kernel_sb<kModeSymbols, false, false, false, true>(sb);
    }
  }
  switch (mode) {
    case kModeGaussian: return dec_kernel_sb<kModeGaussian, false, false>(sb);
    case kModeLatents:
      return imp ? dec_kernel_sb<kModeLatents, true, false>(sb)
                 : dec_kernel_sb<kModeLatents, false, false>(sb);
    default:
      return imp ? dec_kernel_sb<kModeSymbols, true, false>(sb)
                 : dec_kernel_sb<kModeSymbols, false, false>(sb);
  }
}

// Phase buffer of later launches (gaans_debug_phases).
PhaseBuf g_phase{nullptr, 0};

// One encode launch: kernel, geometry and arguments.
struct EncLaunch {
  EncKernel kernel;
  uint32_t grid, block;
  size_t lds;
  EncArgs a;
};

// The parts of an encode launch that follow from the mode, the index kind
// (implicit: table = channel), the tables and the shape; the per-call
// pointers are left NULL (encode_bind sets them).
int encode_prepare(int mode, bool implicit, int32_t n_scales, float scale_bound,
                   const gaans_tables* tables, const Layout& L, EncLaunch* e) {
  int rc;
  if ((rc = check_tables_arg(tables))) return rc;
  if (mode == kModeGaussian && (n_scales < 1 || n_scales > kMaxScales))
    return fail(GAANS_EINVAL, "scale table of %d entries outside [1, %d]", n_scales, kMaxScales);
  BlobRef blob;
  if ((rc = blob_ref(tables, &blob))) return rc;
  DevLds dl;
  if ((rc = device_lds(&dl))) return rc;
  // the scale table, padded (stage_scales), at a 16-byte aligned offset
  const int64_t extra =
      mode == kModeGaussian ? align_up(4 * ((int64_t)n_scales + kGaussPad), 16) + 16 : 0;
  // 16-step blocks for long units only (the coder waits for the first
  // block to be mapped, so short units lose more than the per-block saving
  // gains: measured slower at 96 steps, faster at 4,080), and with explicit
  // or computed indexes only (with table = channel the 16-step kernel needs
  // private scratch)
  const bool long_units = L.seg_cap >= 512 * kLanes;
  const bool gauss = mode == kModeGaussian;
  if (gauss) implicit = false;
  // The Gaussian mode's mappers (a scale-table search and table reads from
  // L2 per element) are the slower half at any length: with 8-step blocks
  // the coder waited about 135 of its 350 cycles per step at the barriers
  // (mean-scale hyperprior y, P = 4 and 16), and 16-step blocks give each
  // mapper wave two steps per block to overlap.
  const EncPlan plan = plan_encode(tables, L.P, L.U, dl, extra, !gauss,
                                   (long_units || gauss) && !implicit);
  const Stage& st = plan.st;
  size_t lds = plan.lds + (size_t)extra;
  if (lds > (size_t)dl.per_block)
    return fail(GAANS_EINVAL, "encode needs %zu bytes of LDS, the device has %d", lds,
                dl.per_block);
  // When the whole grid is resident at once, the LDS the plan's workgroups
  // per CU leave each one costs nothing: the fused pack stages the unit's
  // flushed words there (at most the slot, 2 cap_words bytes, past the
  // ring and the block records) rather than reading them from global memory
  // (the 2160x3840 latent's units flush 20-30 KB, more than their 17 KB of
  // tables).
  if (L.U <= plan.occ * (int64_t)dl.cus) {
    const int64_t want = (int64_t)lds + 2 * L.cap_words + 16;
    const int64_t room = lds_budget(dl, plan.occ);
    if ((int64_t)lds < room) lds = (size_t)(want < room ? want : room);
  }
  EncArgs& a = e->a;
  memset(&a, 0, sizeof(a));
  a.n_scales = gauss ? n_scales : 0;
  a.scales_pow2 = gauss ? pow2_floor(n_scales - 1) : 0;
  a.scale_bound = gauss ? scale_bound : 0.0f;
  a.scales_lds = (uint32_t)align_up((int64_t)plan.lds, 16);
  a.tables = static_cast<const uint8_t*>(tables->dev);
  a.M = (uint32_t)tables->M;
  a.tables_bytes = (uint32_t)tables->bytes;
  a.blob = blob;
  a.N = L.N;
  a.K = (int32_t)L.K;
  a.P = (int32_t)L.P;
  a.C = (int32_t)L.C;
  a.chunk_len = (int32_t)L.chunk_len;
  a.S = (int32_t)L.S;
  a.seg_cap = (int32_t)L.seg_cap;
  a.div_hw = make_udiv((uint32_t)L.HW);
  a.cap_words = (int32_t)L.cap_words;
  a.units = L.U;
  a.header_bytes = L.header_bytes;
  a.B = (uint32_t)L.B;
  a.nt_cap = st.nt_cap;
  a.stage_all = st.stage_all;
  a.ring_mask = (uint32_t)(plan.ring - 1);
  // fused encode: unit numbers from tickets unless the grid fits the device
  // in one round at the plan's workgroups per CU
  a.ticket = L.U > plan.occ * (int64_t)dl.cus ? 1u : 0u;
  a.elect = L.U > (int64_t)dl.cus ? 1u : 0u;
  a.lds_bytes = (uint32_t)lds;
  // 8 mapper waves when every workgroup has a CU to itself
  const int nm = plan.occ == 1 && L.U <= dl.cus ? 8 : 4;
  e->kernel = enc_kernel(mode, implicit, plan.sb, nm);
  e->grid = (uint32_t)L.U;
  e->block = (uint32_t)((nm + 1) * kLanes);
  e->lds = lds;
  return allow_lds(reinterpret_cast<const void*>(e->kernel), lds, dl);
}

// Checks of an encode call's pointers (before any device query).
int encode_check(int mode, bool implicit, const Layout& L, const int32_t* symbols,
                 const float* y, const float* medians, const int32_t* indexes, const GaussIn* g,
                 const void* ws, int64_t ws_bytes, const void* ctrl) {
  if (mode == kModeSymbols ? !symbols : (!y || (mode == kModeLatents && !medians)))
    return fail(GAANS_EINVAL, "input pointer is NULL");
  if (mode == kModeGaussian) {
    if (!g->scales || !g->table)
      return fail(GAANS_EINVAL, "scales or scale table pointer is NULL");
  } else if (implicit != (indexes == nullptr)) {
    return fail(GAANS_EINVAL, implicit ? "indexes given to a plan made for table = channel"
                                       : "indexes missing for a plan made for explicit indexes");
  }
  if (!ctrl) return fail(GAANS_EINVAL, "control block pointer is NULL");
  if (!ws || ws_bytes < L.ws_bytes)
    return fail(GAANS_EINVAL, "workspace too small (%lld < %lld bytes)", (long long)ws_bytes,
                (long long)L.ws_bytes);
  return GAANS_OK;
}

// Per-call pointers of an encode launch (the workspace carved by the layout).
void encode_bind(int mode, EncArgs& a, const Layout& L, const int32_t* symbols, const float* y,
                 const float* medians, const int32_t* indexes, const GaussIn* g, void* ws,
                 void* ctrl, uint64_t* info_out) {
  uint8_t* w = static_cast<uint8_t*>(ws);
  a.symbols = symbols;
  a.y = y;
  a.medians = medians;
  a.means = mode == kModeGaussian ? g->means : nullptr;
  a.scales = mode == kModeGaussian ? g->scales : nullptr;
  a.scale_table = mode == kModeGaussian ? g->table : nullptr;
  a.indexes = mode == kModeGaussian ? nullptr : indexes;
  a.chunk_words = reinterpret_cast<uint32_t*>(w + L.o_words_cnt);
  a.index_hash = reinterpret_cast<uint32_t*>(w + L.o_hash);
  a.end_off = reinterpret_cast<uint32_t*>(w + L.o_end);
  a.ws_info = reinterpret_cast<uint64_t*>(w + L.o_info);
  a.states = reinterpret_cast<uint32_t*>(w + L.o_states);
  a.words = reinterpret_cast<uint16_t*>(w + L.o_words);
  a.esc = reinterpret_cast<uint2*>(w + L.o_esc);
  a.esc_raw = reinterpret_cast<uint32_t*>(w + L.o_esc_raw);
  a.ctrl = static_cast<uint32_t*>(ctrl);
  a.info_out = info_out;
  a.look = reinterpret_cast<uint64_t*>(w + L.o_look);
  a.out = nullptr;  // stage 1 only unless the caller fuses the pack (encode_fuse)
  a.out_bytes = 0;
  a.phase = g_phase;
}

// Fuse the pack into an encode launch: the payload buffer must hold the
// shape's worst case, since each unit writes at the offset its look-back
// finds before the launch's size is known.
int encode_fuse(EncArgs& a, const Layout& L, uint8_t* out, int64_t out_bytes) {
  if (!out || out_bytes < L.max_payload)
    return fail(GAANS_EINVAL, "payload buffer of %lld bytes, the shape's worst case is %lld",
                (long long)out_bytes, (long long)L.max_payload);
  a.out = out;
  a.out_bytes = out_bytes;
  return GAANS_OK;
}

int encode_launch(const EncLaunch& e, void* stream) {
  e.kernel<<<dim3(e.grid), dim3(e.block), e.lds, static_cast<hipStream_t>(stream)>>>(e.a);
  return check_launch("encode");
}

// out != NULL: the pack fused into the launch (payload buffer of out_bytes)
int encode_stage1(int mode, void* stream, const int32_t* symbols, const float* y,
                  const float* medians, const int32_t* indexes, const GaussIn* g,
                  const gaans_tables* tables, int64_t B, int64_t N, int64_t C, int64_t P,
                  int64_t S, void* ws, int64_t ws_bytes, void* ctrl, uint64_t* info_out,
                  uint8_t* out = nullptr, int64_t out_bytes = 0) {
  Layout L;
  int rc = make_layout(B, N, C, P, S, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables))) return rc;
  if (mode == kModeGaussian && (rc = check_gauss(g))) return rc;
  const bool implicit = indexes == nullptr;
  if ((rc = encode_check(mode, implicit, L, symbols, y, medians, indexes, g, ws, ws_bytes, ctrl)))
    return rc;
  EncLaunch e;
  if ((rc = encode_prepare(mode, implicit, g ? g->n : 0, g ? g->bound : 0.0f, tables, L, &e)))
    return rc;
  encode_bind(mode, e.a, L, symbols, y, medians, indexes, g, ws, ctrl, info_out);
  if (out && (rc = encode_fuse(e.a, L, out, out_bytes))) return rc;
  return encode_launch(e, stream);
}

// One decode launch: kernel, geometry and arguments.
struct DecLaunch {
  DecKernel kernel;
  uint32_t grid, block;
  size_t lds;
  DecArgs a;
};

// The parts of a decode launch that follow from the mode, the index kind,
// the tables and the shape; per-call pointers are left NULL (decode_bind).
int decode_prepare(int mode, bool implicit, int32_t n_scales, float scale_bound,
                   const gaans_tables* tables, const Layout& L, DecLaunch* e) {
  int rc;
  if ((rc = check_tables_arg(tables))) return rc;
  if (mode == kModeGaussian && (n_scales < 1 || n_scales > kMaxScales))
    return fail(GAANS_EINVAL, "scale table of %d entries outside [1, %d]", n_scales, kMaxScales);
  BlobRef blob;
  if ((rc = blob_ref(tables, &blob))) return rc;
  DevLds dl;
  if ((rc = device_lds(&dl))) return rc;
  const bool gauss = mode == kModeGaussian;
  if (gauss) implicit = false;
  const bool latents = mode != kModeSymbols;
  const int64_t extra =
      gauss ? align_up(4 * ((int64_t)n_scales + kGaussPad), 16) + 16 : 0;  // as for the encoder
  const bool search_ok = (tables->flags & GAANS_TABLES_SEARCH) != 0 && !implicit;
  const DecPlan plan = plan_decode(tables, L.P, L.U, latents, dl, extra, !gauss, search_ok);
  const Stage& st = plan.st;
  const size_t lds = plan.lds + (size_t)extra;
  if (lds > (size_t)dl.per_block)
    return fail(GAANS_EINVAL, "decode needs %zu bytes of LDS, the device has %d", lds,
                dl.per_block);
  DecArgs& a = e->a;
  memset(&a, 0, sizeof(a));
  a.tables = static_cast<const uint8_t*>(tables->dev);
  a.M = (uint32_t)tables->M;
  a.tables_bytes = (uint32_t)tables->bytes;
  a.blob = blob;
  a.n_scales = gauss ? n_scales : 0;
  a.scales_pow2 = gauss ? pow2_floor(n_scales - 1) : 0;
  a.scale_bound = gauss ? scale_bound : 0.0f;
  a.scales_lds = (uint32_t)align_up((int64_t)plan.lds, 16);
  a.N = L.N;
  a.header_bytes = L.header_bytes;
  a.units = L.U;
  a.B = (uint32_t)L.B;
  a.C = (uint32_t)L.C;
  a.P = (uint32_t)L.P;
  a.K = (uint32_t)L.K;
  a.chunk_len = (uint32_t)L.chunk_len;
  a.S = (uint32_t)L.S;
  a.div_hw = make_udiv((uint32_t)L.HW);
  a.nt_cap = st.nt_cap;
  a.ne_cap = st.ne_cap;
  a.nd_cap = st.nd_cap;
  a.stage_all = st.stage_all;
  a.starts_words = plan.starts_words;
  // the refill-skipping steps when the grid needs more than one workgroup
  // per CU (issue slots, not one unit's step latency, bound the launch)
  e->kernel = dec_kernel(mode, implicit, plan.sb, plan.search, plan.wide, L.U > (int64_t)dl.cus);
  e->grid = (uint32_t)L.U;
  e->block = (uint32_t)kDecThreads;
  e->lds = lds;
  return allow_lds(reinterpret_cast<const void*>(e->kernel), lds, dl);
}

// Checks of a decode call's pointers (before any device query).
int decode_check(int mode, bool implicit, const Layout& L, const uint8_t* payload,
                 int64_t payload_bytes, const int32_t* indexes, const GaussIn* g,
                 const float* medians, const void* out, const void* ctrl,
                 const uint32_t* status_out) {
  if (!payload || !status_out || !ctrl || !out || (mode == kModeLatents && !medians))
    return fail(GAANS_EINVAL, "payload, output, control or status pointer is NULL");
  if (mode == kModeGaussian) {
    if (!g->scales || !g->table)
      return fail(GAANS_EINVAL, "scales or scale table pointer is NULL");
  } else if (implicit != (indexes == nullptr)) {
    return fail(GAANS_EINVAL, implicit ? "indexes given to a plan made for table = channel"
                                       : "indexes missing for a plan made for explicit indexes");
  }
  if (payload_bytes < L.header_bytes)
    return fail(GAANS_EINVAL, "payload (%lld bytes) is shorter than its header (%lld bytes)",
                (long long)payload_bytes, (long long)L.header_bytes);
  return GAANS_OK;
}

void decode_bind(int mode, DecArgs& a, const uint8_t* payload, int64_t payload_bytes,
                 const int32_t* indexes, const GaussIn* g, const float* medians, void* out,
                 void* ctrl, uint32_t* status_out) {
  a.payload = payload;
  a.payload_bytes = payload_bytes;
  a.indexes = mode == kModeGaussian ? nullptr : indexes;
  a.medians = medians;
  a.means = mode == kModeGaussian ? g->means : nullptr;
  a.scales = mode == kModeGaussian ? g->scales : nullptr;
  a.scale_table = mode == kModeGaussian ? g->table : nullptr;
  a.out_sym = mode == kModeSymbols ? static_cast<int32_t*>(out) : nullptr;
  a.out_y = mode == kModeSymbols ? nullptr : static_cast<float*>(out);
  a.ctrl = static_cast<uint32_t*>(ctrl);
  a.status_out = status_out;
  a.phase = g_phase;
}

int decode_launch(const DecLaunch& e, void* stream) {
  e.kernel<<<dim3(e.grid), dim3(e.block), e.lds, static_cast<hipStream_t>(stream)>>>(e.a);
  return check_launch("decode");
}

int decode_impl(int mode, void* stream, const uint8_t* payload, int64_t payload_bytes,
                const int32_t* indexes, const GaussIn* g, const gaans_tables* tables,
                const float* medians, int64_t B, int64_t N, int64_t C, int64_t P, int64_t S,
                int32_t* out_sym, float* out_y, void* ctrl, uint32_t* status_out) {
  Layout L;
  int rc = make_layout(B, N, C, P, S, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables))) return rc;
  if (mode == kModeGaussian && (rc = check_gauss(g))) return rc;
  const bool implicit = indexes == nullptr;
  void* out = mode == kModeSymbols ? static_cast<void*>(out_sym) : static_cast<void*>(out_y);
  if ((rc = decode_check(mode, implicit, L, payload, payload_bytes, indexes, g, medians, out, ctrl,
                         status_out)))
    return rc;
  DecLaunch e;
  if ((rc = decode_prepare(mode, implicit, g ? g->n : 0, g ? g->bound : 0.0f, tables, L, &e)))
    return rc;
  decode_bind(mode, e.a, payload, payload_bytes, indexes, g, medians, out, ctrl, status_out);
  return decode_launch(e, stream);
}

// CompressAI Rans64 streams: plan the LDS (all tables; else, with implicit
// indexes, one channel's table at a time; else global lookups) and launch.
int rans64_decode_impl(void* stream, const uint8_t* streams, int64_t streams_bytes,
                       const int64_t* offsets, const int32_t* indexes,
                       const gaans_tables* tables, int64_t B, int64_t N, int64_t C,
                       int32_t* out, void* ctrl, uint32_t* status_out) {
  int rc = check_tables_arg(tables);
  if (rc) return rc;
  if (B < 1 || N < 1 || C < 1 || N % C != 0)
    return fail(GAANS_EINVAL, "need B, N, C >= 1 and N %% C == 0 (B=%lld N=%lld C=%lld)",
                (long long)B, (long long)N, (long long)C);
  if (N > 0x7fffffffll - kR64Steps || B > 0x7fffffffll)
    return fail(GAANS_EINVAL, "N must stay below 2^31 - %d symbols per stream", kR64Steps);
  if (streams_bytes < 0 || (!streams && streams_bytes > 0))
    return fail(GAANS_EINVAL, "streams pointer is NULL or streams_bytes is negative");
  if (!offsets || !out || !ctrl || !status_out)
    return fail(GAANS_EINVAL, "offsets, output, control or status pointer is NULL");
  if (!indexes && C > tables->M)
    return fail(GAANS_EINVAL, "table = channel needs a table per channel (C=%lld > M=%d)",
                (long long)C, tables->M);
  BlobRef blob;
  if ((rc = blob_ref(tables, &blob))) return rc;
  DevLds dl;
  if ((rc = device_lds(&dl))) return rc;
  const int64_t fixed = kR64RingBytes + (indexes ? kR64IdxBytes : 0);
  const int64_t budget = (int64_t)dl.per_block - fixed;
  const int64_t per_table = 8 * kLutSize + 16;
  const int64_t M = tables->M;
  int stage = 0, subs = 0;
  int64_t nt_cap = 0, sub_cap = 0;
  if (M * per_table + tables->total_dense * kSubBytes <= budget) {
    stage = 1, subs = 1, nt_cap = M, sub_cap = tables->total_dense;
  } else if (M * per_table <= budget) {
    stage = 1, nt_cap = M;
  } else if (!indexes) {
    stage = 2, nt_cap = 1;
    if (tables->max_dense <= kR64SubCap) subs = 1, sub_cap = kR64SubCap;
  }
  R64Args a;
  a.streams = streams;
  a.streams_bytes = streams_bytes;
  a.offsets = offsets;
  a.indexes = indexes;
  a.tables = static_cast<const uint8_t*>(tables->dev);
  a.M = (uint32_t)M;
  a.tables_bytes = (uint32_t)tables->bytes;
  a.blob = blob;
  a.B = B;
  a.N = N;
  a.div_hw = make_udiv((uint32_t)(N / C));
  a.stage = stage;
  a.stage_subs = subs;
  a.lds_tabs = (uint32_t)fixed;
  a.nt_cap = (int32_t)nt_cap;
  a.out = out;
  a.ctrl = static_cast<uint32_t*>(ctrl);
  a.status_out = status_out;
  // one stream per wave while the SIMDs have room, more (up to 64) beyond
  const int64_t simds = 4 * (int64_t)dl.cus;
  const int64_t spw = B <= simds ? 1 : ((B + simds - 1) / simds < kLanes ? (B + simds - 1) / simds
                                                                          : kLanes);
  const int64_t grid = (B + spw - 1) / spw;
  a.spw = (int32_t)spw;
  a.nblocks = (uint32_t)grid;
  const size_t lds = (size_t)(fixed + nt_cap * per_table + sub_cap * kSubBytes);
  if (lds > (size_t)dl.per_block)
    return fail(GAANS_EINVAL, "Rans64 decode needs %zu bytes of LDS, the device has %d", lds,
                dl.per_block);
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto kernel) -> int {
    int r = allow_lds(reinterpret_cast<const void*>(kernel), lds, dl);
    if (r) return r;
    kernel<<<dim3((uint32_t)grid), dim3(kLanes), lds, s>>>(a);
    return check_launch("Rans64 decode");
  };
  return indexes ? launch(k_rans64_decode<false>) : launch(k_rans64_decode<true>);
}

// Clear n u32 words (the no-allocation entry point's control block, once per
// device before its first use; a kernel rather than a memset so that the call
// can be captured into a graph).
// Pack launch: the shape part (pack_prepare), the per-call pointers
// (pack_bind) and the launch.
void pack_prepare(const gaans_tables* tables, const Layout& L, PackArgs& a) {
  memset(&a, 0, sizeof(a));
  a.tables = static_cast<const uint8_t*>(tables->dev);
  a.header_bytes = L.header_bytes;
  a.cap_words = L.cap_words;
  a.units = L.U;
  a.N = L.N;
  a.B = (uint32_t)L.B;
  a.N32 = (uint32_t)L.N;
  a.C = (uint32_t)L.C;
  a.P = (uint32_t)L.P;
  a.K = (uint32_t)L.K;
  a.chunk_len = (uint32_t)L.chunk_len;
  a.M = (uint32_t)tables->M;
  a.S = (uint32_t)L.S;
  a.seg_cap = (uint32_t)L.seg_cap;
}

void pack_bind(PackArgs& a, const Layout& L, const void* ws, uint8_t* out, int64_t out_bytes) {
  const uint8_t* w = static_cast<const uint8_t*>(ws);
  a.chunk_words = reinterpret_cast<const uint32_t*>(w + L.o_words_cnt);
  a.index_hash = reinterpret_cast<const uint32_t*>(w + L.o_hash);
  a.end_off = reinterpret_cast<const uint32_t*>(w + L.o_end);
  a.states = reinterpret_cast<const uint32_t*>(w + L.o_states);
  a.words = reinterpret_cast<const uint16_t*>(w + L.o_words);
  a.esc = reinterpret_cast<const uint2*>(w + L.o_esc);
  a.esc_raw = reinterpret_cast<const uint32_t*>(w + L.o_esc_raw);
  a.out = out;
  a.out_bytes = out_bytes;
}

int pack_launch(const PackArgs& a, void* stream) {
  k_pack<<<dim3((uint32_t)a.units), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch("pack");
}

// ---- call plans -----------------------------------------------------------
// A plan holds an encode (pack fused) or decode launch with every
// shape-dependent field filled; a run copies it, sets the call's pointers and
// launches.  Stored in the caller's gaans_plan (opaque bytes).
constexpr uint32_t kPlanEncMagic = 0x4E504147u;  // "GAPN" (encode)
constexpr uint32_t kPlanDecMagic = 0x44504147u;  // "GAPD" (decode)

struct PlanHead {
  uint32_t magic;
  int32_t mode, implicit, dev;
  Layout L;
};
struct EncPlanRec {
  PlanHead h;
  EncLaunch e;
};
struct DecPlanRec {
  PlanHead h;
  DecLaunch e;
};
static_assert(sizeof(EncPlanRec) <= GAANS_PLAN_BYTES && sizeof(DecPlanRec) <= GAANS_PLAN_BYTES,
              "gaans_plan too small");
static_assert(alignof(EncPlanRec) <= 8 && alignof(DecPlanRec) <= 8, "gaans_plan alignment");

int plan_mode(int32_t mode) {
  return mode == GAANS_MODE_SYMBOLS || mode == GAANS_MODE_LATENTS || mode == GAANS_MODE_GAUSSIAN
             ? GAANS_OK
             : fail(GAANS_EINVAL, "plan mode %d is not a GAANS_MODE_* value", mode);
}

// The device a plan was made on must be current when it runs (its kernels'
// LDS limits and launch shape were set up there).
int plan_device(const PlanHead& h) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(GAANS_EHIP, "hipGetDevice failed");
  if (dev != h.dev)
    return fail(GAANS_EINVAL, "plan made on device %d runs with device %d current", h.dev, dev);
  return GAANS_OK;
}

// Spin until the word a launch sets on completion is nonzero (see
// gaans_wait_host_word).
// Spins on the word; the stream is queried (a failed stream, or one that
// drained without setting the word, ends the wait) once per 100 us of
// spinning, so that the runtime call does not delay the word's detection
// (a query every few hundred reads kept the thread inside it much of the
// time).
int wait_word(void* stream, const uint32_t* word) {
  using clock = std::chrono::steady_clock;
  constexpr auto kQueryEvery = std::chrono::microseconds(100);
  auto next = clock::now() + kQueryEvery;
  for (uint32_t i = 1;; ++i) {
    if (__atomic_load_n(word, __ATOMIC_ACQUIRE) != 0) return GAANS_OK;
    if ((i & 63u) == 0 && clock::now() >= next) {
      const hipError_t e = hipStreamQuery(static_cast<hipStream_t>(stream));
      if (e == hipSuccess) {
        if (__atomic_load_n(word, __ATOMIC_ACQUIRE) != 0) return GAANS_OK;
        return fail(GAANS_EHIP, "stream finished without setting the completion word");
      }
      if (e != hipErrorNotReady)
        return fail(GAANS_EHIP, "stream reported an error: %s", hipGetErrorString(e));
      next = clock::now() + kQueryEvery;
    }
  }
}

__global__ __launch_bounds__(256) void k_clear_words(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = 0u;
}

}  // namespace

// Device scratch of the no-allocation encode entry point
// (gaans_encode_symbols_noalloc): the control block (GAANS_CTRL_BYTES) then
// the encode workspace.  One copy per GPU, held until the process ends; every
// call on a GPU shares it.  Host code never uses this name as an address: the
// device address comes from hipGetSymbolAddress (noalloc_scratch below).
static __device__ __align__(256) uint8_t scratch[GAANS_NOALLOC_SCRATCH_BYTES];

namespace {

// Address of `scratch` on the current device, looked up once per device
// (with that device current) and cleared on `stream` before the first call
// that uses it (control block and workspace, whose look-back words the fused
// encode needs zeroed); the encode kernels leave the control block and the
// look-back words zeroed again after every launch.
int noalloc_scratch(hipStream_t stream, uint8_t** out) {
  static std::mutex mu;
  static uint8_t* addr[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(GAANS_EHIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> g(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(GAANS_EHIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    k_clear_words<<<256, 256, 0, stream>>>(static_cast<uint32_t*>(p),
                                           (int64_t)GAANS_NOALLOC_SCRATCH_BYTES / 4);
    const int rc = check_launch("scratch clear");
    if (rc) return rc;
    addr[dev] = static_cast<uint8_t*>(p);
  }
  *out = addr[dev];
  return GAANS_OK;
}

}  // namespace

// =============================================================================
// C ABI
// =============================================================================

extern "C" {

int gaans_encode_symbols(void* stream, const int32_t* symbols_dev, const int32_t* indexes_dev,
                         const gaans_tables* tables, int64_t B, int64_t N, int64_t C, int64_t P,
                         int32_t segments, void* workspace_dev, int64_t workspace_bytes,
                         void* ctrl_dev, uint64_t* info_out) {
  return encode_stage1(kModeSymbols, stream, symbols_dev, nullptr, nullptr, indexes_dev, nullptr,
                       tables, B, N, C, P, segments, workspace_dev, workspace_bytes, ctrl_dev,
                       info_out);
}

int gaans_encode_latents(void* stream, const float* y_dev, const float* medians_dev,
                         const int32_t* indexes_dev, const gaans_tables* tables, int64_t B,
                         int64_t N, int64_t C, int64_t P, int32_t segments, void* workspace_dev,
                         int64_t workspace_bytes, void* ctrl_dev, uint64_t* info_out) {
  return encode_stage1(kModeLatents, stream, nullptr, y_dev, medians_dev, indexes_dev, nullptr,
                       tables, B, N, C, P, segments, workspace_dev, workspace_bytes, ctrl_dev,
                       info_out);
}

int gaans_encode_gaussian(void* stream, const float* y_dev, const float* means_dev,
                          const float* scales_dev, const float* scale_table_dev,
                          int32_t n_scales, float scale_bound, const gaans_tables* tables,
                          int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                          void* workspace_dev, int64_t workspace_bytes, void* ctrl_dev,
                          uint64_t* info_out) {
  const GaussIn g{means_dev, scales_dev, scale_table_dev, n_scales, scale_bound};
  return encode_stage1(kModeGaussian, stream, nullptr, y_dev, nullptr, nullptr, &g, tables, B, N,
                       C, P, segments, workspace_dev, workspace_bytes, ctrl_dev, info_out);
}

int gaans_encode_pack(void* stream, const void* workspace_dev, int64_t workspace_bytes,
                      const gaans_tables* tables, int64_t B, int64_t N, int64_t C, int64_t P,
                      int32_t segments, uint8_t* out_dev, int64_t out_bytes) {
  Layout L;
  int rc = make_layout(B, N, C, P, segments, &L);
  if (rc) return rc;
  if ((rc = check_tables_arg(tables))) return rc;
  if (!workspace_dev || workspace_bytes < L.ws_bytes)
    return fail(GAANS_EINVAL, "workspace too small");
  if (!out_dev || out_bytes < L.header_bytes)
    return fail(GAANS_EINVAL, "output buffer smaller than the payload header");
  PackArgs a;
  pack_prepare(tables, L, a);
  pack_bind(a, L, workspace_dev, out_dev, out_bytes);
  return pack_launch(a, stream);
}

int gaans_encode_symbols_noalloc(void* stream, const int32_t* symbols_dev,
                                 const int32_t* indexes_dev, const gaans_tables* tables,
                                 int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                                 uint8_t* out_dev, int64_t out_bytes, uint64_t* info_out) {
  Layout L;
  int rc = make_layout(B, N, C, P, segments, &L);
  if (rc) return rc;
  // the size limit first: it needs no device
  const int64_t need = (int64_t)GAANS_CTRL_BYTES + L.ws_bytes;
  if (need > (int64_t)GAANS_NOALLOC_SCRATCH_BYTES)
    return fail(GAANS_EINVAL,
                "B=%lld x N=%lld at P=%lld needs %lld bytes of device scratch; the "
                "no-allocation encode holds %lld (use gaans_encode_symbols with a workspace)",
                (long long)B, (long long)N, (long long)P, (long long)need,
                (long long)GAANS_NOALLOC_SCRATCH_BYTES);
  if (!info_out) return fail(GAANS_EINVAL, "info_out pointer is NULL");
  // every unit writes at the offset its look-back finds: the buffer must
  // hold the worst case (also checked by encode_fuse, before any device work)
  if (!out_dev || out_bytes < L.max_payload)
    return fail(GAANS_EINVAL, "payload buffer of %lld bytes, the shape's worst case is %lld",
                (long long)out_bytes, (long long)L.max_payload);
  uint8_t* base = nullptr;
  if ((rc = noalloc_scratch(static_cast<hipStream_t>(stream), &base))) return rc;
  void* ctrl = base;
  void* ws = base + GAANS_CTRL_BYTES;
  return encode_stage1(kModeSymbols, stream, symbols_dev, nullptr, nullptr, indexes_dev, nullptr,
                       tables, B, N, C, P, segments, ws, L.ws_bytes, ctrl, info_out, out_dev,
                       out_bytes);
}

int gaans_decode_symbols(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                         const int32_t* indexes_dev, const gaans_tables* tables, int64_t B,
                         int64_t N, int64_t C, int64_t P, int32_t segments, int32_t* out_dev,
                         void* ctrl_dev, uint32_t* status_out) {
  return decode_impl(kModeSymbols, stream, payload_dev, payload_bytes, indexes_dev, nullptr,
                     tables, nullptr, B, N, C, P, segments, out_dev, nullptr, ctrl_dev,
                     status_out);
}

int gaans_decode_latents(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                         const int32_t* indexes_dev, const gaans_tables* tables,
                         const float* medians_dev, int64_t B, int64_t N, int64_t C, int64_t P,
                         int32_t segments, float* y_hat_dev, void* ctrl_dev,
                         uint32_t* status_out) {
  return decode_impl(kModeLatents, stream, payload_dev, payload_bytes, indexes_dev, nullptr,
                     tables, medians_dev, B, N, C, P, segments, nullptr, y_hat_dev, ctrl_dev,
                     status_out);
}

int gaans_decode_gaussian(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                          const float* scales_dev, const float* means_dev,
                          const float* scale_table_dev, int32_t n_scales, float scale_bound,
                          const gaans_tables* tables, int64_t B, int64_t N, int64_t C,
                          int64_t P, int32_t segments, float* y_hat_dev, void* ctrl_dev,
                          uint32_t* status_out) {
  const GaussIn g{means_dev, scales_dev, scale_table_dev, n_scales, scale_bound};
  return decode_impl(kModeGaussian, stream, payload_dev, payload_bytes, nullptr, &g, tables,
                     nullptr, B, N, C, P, segments, nullptr, y_hat_dev, ctrl_dev, status_out);
}

int gaans_rans64_decode(void* stream, const uint8_t* streams_dev, int64_t streams_bytes,
                        const int64_t* offsets_dev, const int32_t* indexes_dev,
                        const gaans_tables* tables, int64_t B, int64_t N, int64_t C,
                        int32_t* out_dev, void* ctrl_dev, uint32_t* status_out) {
  return rans64_decode_impl(stream, streams_dev, streams_bytes, offsets_dev, indexes_dev, tables,
                            B, N, C, out_dev, ctrl_dev, status_out);
}

int gaans_plan_encode(const gaans_tables* tables, int32_t mode, int32_t explicit_indexes,
                      int32_t n_scales, float scale_bound, int64_t B, int64_t N, int64_t C,
                      int64_t P, int32_t segments, gaans_plan* plan) {
  if (!plan) return fail(GAANS_EINVAL, "plan pointer is NULL");
  memset(plan, 0, sizeof(*plan));
  int rc = plan_mode(mode);
  if (rc) return rc;
  EncPlanRec* r = reinterpret_cast<EncPlanRec*>(plan);
  if ((rc = make_layout(B, N, C, P, segments, &r->h.L))) return rc;
  const bool implicit = mode != GAANS_MODE_GAUSSIAN && !explicit_indexes;
  if ((rc = encode_prepare(mode, implicit, n_scales, scale_bound, tables, r->h.L, &r->e)))
    return rc;
  r->h.mode = mode;
  r->h.implicit = implicit;
  if (hipGetDevice(&r->h.dev) != hipSuccess) return fail(GAANS_EHIP, "hipGetDevice failed");
  r->h.magic = kPlanEncMagic;
  return GAANS_OK;
}

int gaans_plan_decode(const gaans_tables* tables, int32_t mode, int32_t explicit_indexes,
                      int32_t n_scales, float scale_bound, int64_t B, int64_t N, int64_t C,
                      int64_t P, int32_t segments, gaans_plan* plan) {
  if (!plan) return fail(GAANS_EINVAL, "plan pointer is NULL");
  memset(plan, 0, sizeof(*plan));
  int rc = plan_mode(mode);
  if (rc) return rc;
  DecPlanRec* r = reinterpret_cast<DecPlanRec*>(plan);
  if ((rc = make_layout(B, N, C, P, segments, &r->h.L))) return rc;
  const bool implicit = mode != GAANS_MODE_GAUSSIAN && !explicit_indexes;
  if ((rc = decode_prepare(mode, implicit, n_scales, scale_bound, tables, r->h.L, &r->e)))
    return rc;
  r->h.mode = mode;
  r->h.implicit = implicit;
  if (hipGetDevice(&r->h.dev) != hipSuccess) return fail(GAANS_EHIP, "hipGetDevice failed");
  r->h.magic = kPlanDecMagic;
  return GAANS_OK;
}

int gaans_run_encode(const gaans_plan* plan, void* stream, const void* in0, const void* in1,
                     const void* in2, const void* in3, void* workspace_dev,
                     int64_t workspace_bytes, void* ctrl_dev, uint8_t* out_dev,
                     int64_t out_bytes, uint64_t* info_host) {
  if (!info_host) return fail(GAANS_EINVAL, "info_host pointer is NULL");
  uint32_t* done = reinterpret_cast<uint32_t*>(&info_host[2]);  // low half of info[2]
  __atomic_store_n(done, 0u, __ATOMIC_RELEASE);
  const int rc = gaans_enqueue_encode(plan, stream, in0, in1, in2, in3, workspace_dev,
                                      workspace_bytes, ctrl_dev, out_dev, out_bytes, info_host);
  return rc ? rc : wait_word(stream, done);
}

int gaans_enqueue_encode(const gaans_plan* plan, void* stream, const void* in0, const void* in1,
                         const void* in2, const void* in3, void* workspace_dev,
                         int64_t workspace_bytes, void* ctrl_dev, uint8_t* out_dev,
                         int64_t out_bytes, uint64_t* info_out) {
  const EncPlanRec* r = reinterpret_cast<const EncPlanRec*>(plan);
  if (!r || r->h.magic != kPlanEncMagic)
    return fail(GAANS_EINVAL, "not an encode plan (gaans_plan_encode)");
  const Layout& L = r->h.L;
  const int mode = r->h.mode;
  const int32_t* symbols = nullptr;
  const int32_t* indexes = nullptr;
  const float *y = nullptr, *medians = nullptr;
  GaussIn g{nullptr, nullptr, nullptr, r->e.a.n_scales, r->e.a.scale_bound};
  if (mode == GAANS_MODE_SYMBOLS) {
    symbols = static_cast<const int32_t*>(in0);
    indexes = static_cast<const int32_t*>(in1);
  } else if (mode == GAANS_MODE_LATENTS) {
    y = static_cast<const float*>(in0);
    medians = static_cast<const float*>(in1);
    indexes = static_cast<const int32_t*>(in2);
  } else {
    y = static_cast<const float*>(in0);
    g.means = static_cast<const float*>(in1);
    g.scales = static_cast<const float*>(in2);
    g.table = static_cast<const float*>(in3);
  }
  int rc = encode_check(mode, r->h.implicit, L, symbols, y, medians, indexes, &g, workspace_dev,
                        workspace_bytes, ctrl_dev);
  if (rc || (rc = plan_device(r->h))) return rc;
  EncLaunch e = r->e;
  encode_bind(mode, e.a, L, symbols, y, medians, indexes, &g, workspace_dev, ctrl_dev, info_out);
  if ((rc = encode_fuse(e.a, L, out_dev, out_bytes))) return rc;
  return encode_launch(e, stream);
}

int gaans_run_decode(const gaans_plan* plan, void* stream, const uint8_t* payload_dev,
                     int64_t payload_bytes, const void* in0, const void* in1, const void* in2,
                     void* out_dev, void* ctrl_dev, uint32_t* status_host) {
  if (!status_host) return fail(GAANS_EINVAL, "status pointer is NULL");
  uint32_t* done = status_host + 1;
  __atomic_store_n(done, 0u, __ATOMIC_RELEASE);
  const int rc = gaans_enqueue_decode(plan, stream, payload_dev, payload_bytes, in0, in1, in2,
                                      out_dev, ctrl_dev, status_host);
  return rc ? rc : wait_word(stream, done);
}

int gaans_enqueue_decode(const gaans_plan* plan, void* stream, const uint8_t* payload_dev,
                         int64_t payload_bytes, const void* in0, const void* in1,
                         const void* in2, void* out_dev, void* ctrl_dev, uint32_t* status_host) {
  const DecPlanRec* r = reinterpret_cast<const DecPlanRec*>(plan);
  if (!r || r->h.magic != kPlanDecMagic)
    return fail(GAANS_EINVAL, "not a decode plan (gaans_plan_decode)");
  const int mode = r->h.mode;
  const int32_t* indexes = nullptr;
  const float* medians = nullptr;
  GaussIn g{nullptr, nullptr, nullptr, r->e.a.n_scales, r->e.a.scale_bound};
  if (mode == GAANS_MODE_SYMBOLS) {
    indexes = static_cast<const int32_t*>(in0);
  } else if (mode == GAANS_MODE_LATENTS) {
    medians = static_cast<const float*>(in0);
    indexes = static_cast<const int32_t*>(in1);
  } else {
    g.scales = static_cast<const float*>(in0);
    g.means = static_cast<const float*>(in1);
    g.table = static_cast<const float*>(in2);
  }
  int rc = decode_check(mode, r->h.implicit, r->h.L, payload_dev, payload_bytes, indexes, &g,
                        medians, out_dev, ctrl_dev, status_host);
  if (rc || (rc = plan_device(r->h))) return rc;
  DecLaunch e = r->e;
  decode_bind(mode, e.a, payload_dev, payload_bytes, indexes, &g, medians, out_dev, ctrl_dev,
              status_host);
  return decode_launch(e, stream);
}

int gaans_run_encode_call(const gaans_encode_call* c) {
  if (!c) return fail(GAANS_EINVAL, "call pointer is NULL");
  return gaans_run_encode(c->plan, c->stream, c->in[0], c->in[1], c->in[2], c->in[3],
                          c->workspace_dev, c->workspace_bytes, c->ctrl_dev, c->out_dev,
                          c->out_bytes, c->info_host);
}

int gaans_run_decode_call(const gaans_decode_call* c) {
  if (!c) return fail(GAANS_EINVAL, "call pointer is NULL");
  return gaans_run_decode(c->plan, c->stream, c->payload_dev, c->payload_bytes, c->in[0],
                          c->in[1], c->in[2], c->out_dev, c->ctrl_dev, c->status_host);
}

int gaans_debug_phases(void* buffer_dev, int64_t units, int32_t* wall_clock_khz) {
#ifndef GAANS_PHASE_TIMES
  if (buffer_dev != nullptr && units > 0)
    return fail(GAANS_EINVAL, "this library is built without phase timestamps "
                "(build the GAANS_PHASE_TIMES variant)");
#endif
  if (wall_clock_khz) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(wall_clock_khz, hipDeviceAttributeWallClockRate, dev) !=
            hipSuccess)
      return fail(GAANS_EHIP, "cannot query the device's wall clock rate");
  }
  if (buffer_dev == nullptr || units <= 0) {
    g_phase = PhaseBuf{nullptr, 0};
    return GAANS_OK;
  }
  g_phase = PhaseBuf{static_cast<uint64_t*>(buffer_dev), units};  // kPhaseSlots u64 per unit
  return GAANS_OK;
}

int gaans_wait_host_word(void* stream, const uint32_t* word) {
  if (!word) return fail(GAANS_EINVAL, "completion word pointer is NULL");
  return wait_word(stream, word);
}

}  // extern "C"
