/*
 * CPU oracle for the GA-ANS latent-coding path.  TEST INFRASTRUCTURE ONLY:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / CPU baseline, never as the
 * product path.
 *
 * Two coders live here, written independently of the HIP kernels:
 *
 *  1. rans64_ref_*  -- a restatement of CompressAI's single-stream Rans64
 *     coder with 4-bit bypass escapes (64-bit state, L = 2^31, 32-bit words,
 *     16-bit CDF precision).  Follows, in the reference repository:
 *       src/fast_compressai/coders/cuda/rans64_gpu.cuh:5-55      (EncInit/Put/Flush/PutBits)
 *       src/fast_compressai/coders/cuda/rans64dec_gpu.cuh:8-48   (DecInit/Get/Advance/GetBits)
 *       src/fast_compressai/coders/cuda/warp_ans_kernel_v2.cu:139-169 (escape mapping)
 *       src/fast_compressai/coders/cuda/warp_ans_kernel.cu:299-327     (escape decode)
 *       src/fast_compressai/coders/cuda/ans_gpu_kernel.cu:133-194, :341-393 (one stream, reverse order)
 *     It is meant to equal CompressAI's BufferedRansEncoder.flush() output
 *     for the same symbols (little-endian u32 words, memory order).  CompressAI
 *     is not installed here, so that equality is parity unpinned: the tests pin
 *     this coder with hand-derived known answers of the arithmetic above, the
 *     reference's own CPU test cases as round trips, and length against the
 *     information content.
 *
 *  2. gaans_ref_*   -- a sequential emulation of the wave64 GA-ANS payload
 *     format ("gaans-w64-v3") that the GPU kernels must reproduce byte for
 *     byte.  The format is specified in the comment block of gaans_oracle.c.
 *
 * Every function returns 0 on success or a negative GAANS_REF_E* code.
 */
#ifndef GAANS_ORACLE_H
#define GAANS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  GAANS_REF_OK = 0,
  GAANS_REF_EINVAL = -1,      /* bad shapes / arguments */
  GAANS_REF_ETABLE = -2,      /* CDF table not a valid 16-bit quantized CDF */
  GAANS_REF_EINDEX = -3,      /* table index out of range */
  GAANS_REF_ERANGE = -4,      /* symbol escape value does not fit 32 bits */
  GAANS_REF_ESPACE = -5,      /* output buffer too small */
  GAANS_REF_ECORRUPT = -6,    /* payload inconsistent / stream corrupt */
  GAANS_REF_EMISMATCH = -7,   /* payload made with other tables or indexes */
};

/* ---- CompressAI-equivalent Rans64 single stream -------------------------- */

/* Encode n symbols (one stream).  out_words receives the stream in memory
 * order; *n_words is set to its length.  cdfs is [M, Lmax] int32 row-major. */
int rans64_ref_encode(const int32_t* symbols, const int32_t* indexes, int64_t n,
                      const int32_t* cdfs, int32_t M, int32_t Lmax,
                      const int32_t* cdf_sizes, const int32_t* offsets,
                      uint32_t* out_words, int64_t cap_words, int64_t* n_words);

int rans64_ref_decode(const uint32_t* words, int64_t n_words,
                      const int32_t* indexes, int64_t n,
                      const int32_t* cdfs, int32_t M, int32_t Lmax,
                      const int32_t* cdf_sizes, const int32_t* offsets,
                      int32_t* out_symbols);

/* ---- wave64 GA-ANS format ------------------------------------------------ */

/* Upper bound on the payload size (bytes) for the given shape and S
 * segments per chunk; -1 for an invalid shape or S. */
int64_t gaans_ref_max_payload_bytes(int32_t B, int32_t N, int32_t C, int32_t P, int32_t S);

/* One position's term of a coding unit's index hash: MurmurHash3 fmix32 of
 * (p * 0x9E3779B9 + tb + 1) mod 2^32. */
uint32_t gaans_ref_index_term(int64_t p, int32_t tb);

/* FNV-1a 64 digest of the tables, as stored in the payload header. */
uint64_t gaans_ref_table_digest(const int32_t* cdfs, int32_t M, int32_t Lmax,
                                const int32_t* cdf_sizes, const int32_t* offsets);

/* indexes may be NULL: then the table of position i is its channel i / (N/C). */
int gaans_ref_encode(const int32_t* symbols, const int32_t* indexes,
                     int32_t B, int32_t N, int32_t C, int32_t P, int32_t S,
                     const int32_t* cdfs, int32_t M, int32_t Lmax,
                     const int32_t* cdf_sizes, const int32_t* offsets,
                     uint8_t* out, int64_t out_cap, int64_t* out_len);

int gaans_ref_decode(const uint8_t* payload, int64_t payload_len,
                     const int32_t* indexes,
                     int32_t B, int32_t N, int32_t C, int32_t P, int32_t S,
                     const int32_t* cdfs, int32_t M, int32_t Lmax,
                     const int32_t* cdf_sizes, const int32_t* offsets,
                     int32_t* out_symbols);

/* Fused quantize/dequantize closed forms of CompressAI's EntropyModel
 * (quantize(..., "symbols", means) and dequantize(symbols, means)):
 *   symbol = (int32) rint_half_even(fp32(y) - fp32(median))
 *   y_hat  = fp32(symbol) + fp32(median)
 * medians are per channel; y is [B, C, HW] row-major. */
void gaans_ref_quantize(const float* y, const float* medians, int32_t B, int32_t C,
                        int64_t HW, int32_t* symbols);
void gaans_ref_dequantize(const int32_t* symbols, const float* medians, int32_t B,
                          int32_t C, int64_t HW, float* y_hat);

/* CompressAI GaussianConditional.build_indexes restated (see the .c file). */
void gaans_ref_build_indexes(const float* scales, int64_t n, const float* table, int32_t L,
                             float bound, int32_t* indexes);

/* Elementwise quantize / dequantize with optional per-element means. */
void gaans_ref_quantize_elem(const float* y, const float* means, int64_t n, int32_t* symbols);
void gaans_ref_dequantize_elem(const int32_t* symbols, const float* means, int64_t n,
                               float* y_hat);

#ifdef __cplusplus
}
#endif
#endif
