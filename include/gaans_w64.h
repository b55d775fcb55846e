/*
 * gaans_w64.h -- C ABI of the MI355X (gfx950) GA-ANS latent coder.
 *
 * Library: fast-compressai_amd/fast_compressai/coders/lib/libgaans_w64.so
 *
 * The library replaces the reference's pybind11 module
 * fast_compressai.coders._warp_div (src/fast_compressai/coders/cuda/ans_gpu.cpp:25-30):
 *   encode_warp_div(symbols, indexes, cdfs, cdf_sizes, offsets, P)
 *       -> gaans_encode_symbols + gaans_encode_pack   (+ gaans_encode_latents,
 *          which also fuses CompressAI's quantize, reference
 *          src/fast_compressai/coders/factorized.py:46-49)
 *   decode_warp_div(packed, max_rounds, header_bytes, chunk_len, P, indexes,
 *                   cdfs, cdf_sizes, offsets)
 *       -> gaans_decode_symbols                       (+ gaans_decode_latents,
 *          which also fuses dequantize, reference factorized.py:99-101)
 * gaans_tables_prepare replaces the kernels' reads of the padded [M, Lmax]
 * int32 CDF tensor and of the 512 KB magic table (reference
 * warp_ans_kernel_v2.cu:230-247).
 *
 * Conventions
 *  - Every function returns 0 (GAANS_OK) or a positive GAANS_E* code and
 *    leaves a message for gaans_last_error() (thread-local).  No C++
 *    exception crosses this boundary.
 *  - Pointers named *_dev are device pointers.  The library never allocates
 *    memory: the caller passes every buffer, sized with gaans_get_layout /
 *    gaans_tables_bytes.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream).  Device
 *    functions only enqueue work on that stream; none of them synchronises.
 *  - ctrl_dev is a caller-owned control block of GAANS_CTRL_BYTES bytes of
 *    device memory, zeroed once by the caller; every encode/decode leaves it
 *    zeroed again.  Calls that share one control block must be ordered on
 *    one stream (each stream should own its own block).
 *  - Problems the kernels find (bad symbols, corrupt payloads) are reported
 *    as GAANS_ST_* bits in a status word that the last block of the launch
 *    writes to caller memory (device or pinned host memory); read it after
 *    the stream has finished, or, with pinned host memory, once the
 *    launch's completion word is set (gaans_wait_host_word).
 *
 *  - `segments` (S, 1..256) splits every chunk of P channels into S
 *    interleaved segments of whole 64-position steps (segment s: steps s,
 *    s + S, s + 2 S, ... of the chunk, so every segment sees the chunk's
 *    channels in equal shares).  Each segment is a coding unit with its own
 *    states, words and escapes, coded by its own workgroup, so a launch of
 *    few long chunks uses S times more CUs, for 4 * 64 more bytes per extra
 *    unit.  Every unit holds at least one step: S <= the steps of a row's
 *    last (shortest) chunk.  The payload header records S and decode must be
 *    called with the same value.
 *    U = B * K * S coding units per call, at most 2^24 - 1, and a shape's
 *    worst-case payload (7 bytes per symbol plus 264 per unit) must stay
 *    below 2^38 bytes; larger calls return GAANS_EINVAL.
 *
 * Payload format "gaans-w64-v5": defined byte for byte by the CPU oracle,
 * oracle/gaans_oracle.c.
 */
#ifndef GAANS_W64_H
#define GAANS_W64_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GAANS_ABI_VERSION 14
#define GAANS_CTRL_BYTES 256

/* return codes */
#define GAANS_OK 0
#define GAANS_EINVAL 1  /* bad argument, shape or buffer size */
#define GAANS_ETABLE 2  /* CDF tables are not valid 16-bit quantized CDFs */
#define GAANS_EHIP 3    /* a HIP runtime call failed */

/* status bits written by the kernels */
#define GAANS_ST_RANGE 0x01u     /* symbol cannot be coded (escape >= 2^32, non-finite latent) */
#define GAANS_ST_INDEX 0x02u     /* table index out of range */
#define GAANS_ST_HEADER 0x04u    /* payload header does not match the call */
#define GAANS_ST_TABLES 0x08u    /* payload made with other tables, or bad table blob */
#define GAANS_ST_CORRUPT 0x10u   /* unit offsets or rANS stream inconsistent */
#define GAANS_ST_INDEXHASH 0x20u /* payload made with other indexes */
#define GAANS_ST_SIZE 0x40u      /* payload would exceed the 4 GiB format limit */
#define GAANS_ST_TIMEOUT 0x80u   /* a fused encode unit waited 10 s for the units before it */

/* Shape of one coding call (pure host arithmetic, see gaans_get_layout). */
typedef struct gaans_layout {
  int64_t B, N, C, P;     /* batch rows, symbols per row, channels, channels per chunk */
  int64_t S;              /* segments per chunk */
  int64_t HW, K, chunk_len;
  int64_t U;              /* coding units: B * K * S */
  int64_t header_bytes;   /* payload header size (multiple of 16) */
  int64_t max_payload_bytes; /* worst case: every symbol an escape with 8 nibbles */
  int64_t cap_words;      /* staging words per unit (worst case) */
  int64_t workspace_bytes;
  /* byte offsets inside the encode workspace */
  int64_t ws_chunk_words, ws_chunk_status, ws_index_hash, ws_end_off, ws_info,
      ws_states, ws_words, ws_esc, ws_esc_raw;
  /* the fused encode's look-back words (8 bytes per unit, at offset 0, so
   * that their place does not depend on the shape): zero before the first
   * fused encode (gaans_run_encode, gaans_enqueue_encode) that uses the
   * workspace; every such launch leaves them zero */
  int64_t ws_look;
} gaans_layout;

/* Prepared tables: filled by gaans_tables_prepare except `dev`, which the
 * caller sets to the device copy of the prepared blob. */
typedef struct gaans_tables {
  const void* dev;    /* device copy of the prepared blob */
  int64_t bytes;      /* blob size */
  int32_t M;          /* number of tables */
  int32_t max_nsym;   /* largest alphabet (cdf_size - 1) */
  int64_t total_nsym; /* sum of the alphabets */
  uint64_t digest;    /* table digest recorded in payload headers */
  int32_t max_dense;  /* most decode sub-blocks (128 B each: one per 256-value bucket, and
                         per 16-value sub-range, with >= 2 symbol starts) of one table */
  int32_t flags;      /* GAANS_TABLES_* */
  int64_t total_dense; /* decode sub-blocks over all tables */
  float mean_bits;     /* mean over the tables of their entropy (bits per symbol) */
  int32_t max_wide;    /* most wide-lookup sub-blocks of one table (GAANS_TABLES_WIDE) */
  int64_t total_wide;  /* wide-lookup sub-blocks over all tables */
} gaans_tables;

/* gaans_tables.flags: the blob holds compact search lookups (one u32 per
 * 256-value bucket and a u16 start per symbol), which the decoder uses when
 * the sub-blocks do not fit in LDS; set when there are at most 65,527
 * symbols in all and every offset is at least INT32_MIN + 65536. */
#define GAANS_TABLES_SEARCH 1
/* gaans_tables.flags: the blob holds wide decode lookups (2048 buckets of 32
 * values per table, 16 KB, and a 16-entry sub-block of two-value ranges for
 * every bucket in which two or more symbols start after its first value),
 * which the decoder stages instead of the 256-bucket ones when they fit in
 * LDS: fewer steps need a second lookup, none a third; set for M <= 4096. */
#define GAANS_TABLES_WIDE 2

int gaans_abi_version(void);
const char* gaans_last_error(void);

/* Chunking and buffer sizes for B rows of N symbols, C channels, P per chunk
 * and `segments` per chunk.  Requires B, N, C, P >= 1, N % C == 0, P <= C,
 * 1 <= segments <= min(256, steps of a row's last chunk). */
int gaans_get_layout(int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                     gaans_layout* out);

/* The segments per chunk this library picks for a shape (pure host
 * arithmetic): the most that (a) the shape allows, (b) are needed for
 * B * K * S >= target_units (no limit when target_units <= 0; callers pass
 * the device's CU count), and (c) keep the extra bytes of the added units
 * (3.125 bytes per lane plus 4, as measured: an added unit's final states
 * less what its fresh states absorb, a pad and a partly used escape word)
 * within `budget` (a fraction: 0.006 = 0.6%) of a chunk's expected payload,
 * estimated as chunk symbols * tables->mean_bits / 8 plus its states.  No
 * counterpart in the reference (one chunk is one warp's serial loop,
 * warp_ans_kernel_v2.cu:121-126). */
int gaans_choose_segments(const gaans_tables* tables, int64_t B, int64_t N, int64_t C,
                          int64_t P, double budget, int64_t target_units, int32_t* segments);

/* ---- table upload (host memory) ----------------------------------------- */

/* Bytes of the prepared table blob for M tables (cdfs [M, Lmax] and
 * cdf_sizes in host memory; the size depends on the CDF values).  Validates
 * the tables as gaans_tables_prepare does (GAANS_ETABLE otherwise). */
int gaans_tables_bytes(const int32_t* cdfs, const int32_t* cdf_sizes, int32_t M, int32_t Lmax,
                       int64_t* bytes);

/* Validate CompressAI-style tables (cdfs [M, Lmax] int32 row-major, rows
 * zero-padded beyond cdf_sizes[t]; cdf[0] = 0, cdf[S-1] = 65536, strictly
 * increasing; 1 <= M <= 65536 tables of 2 <= S <= 65536 entries) and lay
 * them out for the kernels: per-table metadata, packed (start, freq-1)
 * entries with the encoder's division constant, a 256-bucket decode lookup
 * per table, and for each bucket in which two or more symbols start a
 * 16-entry second-level lookup (16-value sub-ranges), with a 16-entry
 * third level (single values) for each such sub-range.  The caller copies
 * `out` to device memory unchanged and stores its address in desc->dev.
 * Replaces the reference's use of the raw tensors at
 * src/fast_compressai/coders/factorized.py:23-31. */
int gaans_tables_prepare(const int32_t* cdfs, const int32_t* cdf_sizes,
                         const int32_t* offsets, int32_t M, int32_t Lmax,
                         void* out, int64_t out_bytes, gaans_tables* desc);

/* ---- encode ------------------------------------------------------------- */

/* Stage 1: code every unit into `workspace_dev` (layout->workspace_bytes).
 * The launch's last block scans the unit sizes into payload offsets and
 * writes info = {u64 payload bytes incl. header, u64 status} both to the
 * workspace (at layout->ws_info) and, when info_out is not NULL, to
 * info_out[0..1] (device or pinned host memory), and the completion word
 * info_out[2] = 1 | status << 1 | payload bytes << 16 in one 64-bit store
 * (info_out holds 3 u64).  `indexes_dev` may be NULL: then
 * position i of a row uses table i / HW (CompressAI EntropyBottleneck
 * indexes).  Reference: encode_with_indexes_warp_v2_cuda,
 * src/fast_compressai/coders/cuda/warp_ans_kernel_v2.cu:183-273. */
int gaans_encode_symbols(void* stream, const int32_t* symbols_dev,
                         const int32_t* indexes_dev, const gaans_tables* tables,
                         int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                         void* workspace_dev, int64_t workspace_bytes, void* ctrl_dev,
                         uint64_t* info_out);

/* Stage 1 with CompressAI's quantize fused in: symbol = int32(rint(y -
 * medians[c])) for latents y [B, C, HW] fp32 and per-channel medians [C].
 * Reference: FactorizedWarpDivCodec.compress, factorized.py:46-59. */
int gaans_encode_latents(void* stream, const float* y_dev, const float* medians_dev,
                         const int32_t* indexes_dev, const gaans_tables* tables,
                         int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                         void* workspace_dev, int64_t workspace_bytes, void* ctrl_dev,
                         uint64_t* info_out);

/* Stage 1 for CompressAI's GaussianConditional (mean-scale and scale
 * hyperpriors) with its index building and quantize fused in: for every
 * element, index = CompressAI build_indexes(scale) over the scale table
 * (lb = max(scale, scale_bound), NaN kept; index = (n - 1) - #{k < n - 1 :
 * lb <= scale_table[k]}), symbol = int32(rint(y - mean)) (mean = 0 when
 * means_dev is NULL: the scale-only hyperprior).  y, means and scales are
 * fp32 [B, C, HW]; scale_table_dev holds n_scales (1..8192) non-decreasing
 * finite scales in device memory, one per CDF table (tables->M == n_scales
 * for CompressAI models; an index >= M sets GAANS_ST_INDEX).  Chunks hold P
 * latent channels.  No counterpart in the reference's coder, whose
 * accelerate() accepts only FactorizedPrior (src/fast_compressai/api.py:177-182);
 * it replaces CompressAI's GaussianConditional.compress (build_indexes +
 * quantize + RansEncoder) for those models. */
int gaans_encode_gaussian(void* stream, const float* y_dev, const float* means_dev,
                          const float* scales_dev, const float* scale_table_dev,
                          int32_t n_scales, float scale_bound, const gaans_tables* tables,
                          int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                          void* workspace_dev, int64_t workspace_bytes, void* ctrl_dev,
                          uint64_t* info_out);

/* Stage 2: write the payload (header + units) to out_dev.  May be enqueued
 * right after stage 1 on the same stream into a buffer of
 * layout->max_payload_bytes, or after the caller has read the payload size
 * into an exact buffer; units that would not fit out_bytes are skipped.
 * Reference: write_warp_tight_header_kernel and warp_pack_tight_payload_kernel,
 * warp_ans_kernel_v2.cu:274-296. */
int gaans_encode_pack(void* stream, const void* workspace_dev, int64_t workspace_bytes,
                      const gaans_tables* tables, int64_t B, int64_t N, int64_t C,
                      int64_t P, int32_t segments, uint8_t* out_dev, int64_t out_bytes);

/* gaans_encode_symbols + gaans_encode_pack as one fused kernel (as
 * gaans_run_encode) in a call that allocates nothing and takes no workspace
 * or control block: both live in a static device array of
 * GAANS_NOALLOC_SCRATCH_BYTES per GPU (its control block first,
 * GAANS_CTRL_BYTES, then the workspace), held until the process ends.  The
 * caller passes the inputs, the payload buffer (out_dev, out_bytes: at least
 * layout->max_payload_bytes, else GAANS_EINVAL) and info_out (3 u64 in device
 * or pinned host memory, as in gaans_encode_symbols; the completion word
 * info_out[2] carries size and status).  The first call on a GPU looks the
 * array up and clears it on `stream`; the kernels leave its control block
 * and look-back words zeroed after every launch.  Shapes whose control block
 * and workspace exceed the array return GAANS_EINVAL before any device work.
 * Every call on one GPU shares the array: calls that overlap on one GPU
 * (other streams, other threads) race and must be ordered by the caller.
 * No counterpart in the reference: this entry point is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Calls no hipMalloc / hipFree. */
#define GAANS_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int gaans_encode_symbols_noalloc(void* stream, const int32_t* symbols_dev,
                                 const int32_t* indexes_dev, const gaans_tables* tables,
                                 int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                                 uint8_t* out_dev, int64_t out_bytes, uint64_t* info_out);

/* ---- decode ------------------------------------------------------------- */

/* Decode a payload into int32 symbols [B, N].  The last block writes the
 * OR of all GAANS_ST_* bits (0 when the payload decoded cleanly) to
 * status_out[0] (device or pinned host memory), and the completion word
 * status_out[1] = 1 | status << 1 (status_out holds 2 u32).
 * Reference: decode_with_indexes_warp_cuda, warp_ans_kernel.cu:477-544. */
int gaans_decode_symbols(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                         const int32_t* indexes_dev, const gaans_tables* tables,
                         int64_t B, int64_t N, int64_t C, int64_t P, int32_t segments,
                         int32_t* out_dev, void* ctrl_dev, uint32_t* status_out);

/* Decode with CompressAI's dequantize fused in: y_hat = fp32(symbol) +
 * medians[c], written as [B, C, HW] fp32. */
int gaans_decode_latents(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                         const int32_t* indexes_dev, const gaans_tables* tables,
                         const float* medians_dev, int64_t B, int64_t N, int64_t C,
                         int64_t P, int32_t segments, float* y_hat_dev, void* ctrl_dev,
                         uint32_t* status_out);

/* Decode a gaans_encode_gaussian payload with the same scales, means and
 * scale table, dequantize fused: y_hat = fp32(symbol) + mean (fp32(symbol)
 * when means_dev is NULL), written as [B, C, HW] fp32.  Replaces CompressAI's
 * GaussianConditional.decompress (build_indexes + RansDecoder + dequantize). */
int gaans_decode_gaussian(void* stream, const uint8_t* payload_dev, int64_t payload_bytes,
                          const float* scales_dev, const float* means_dev,
                          const float* scale_table_dev, int32_t n_scales, float scale_bound,
                          const gaans_tables* tables, int64_t B, int64_t N, int64_t C,
                          int64_t P, int32_t segments, float* y_hat_dev, void* ctrl_dev,
                          uint32_t* status_out);

/* ---- CompressAI Rans64 bitstreams ------------------------------------------ */

/* Decode B CompressAI Rans64 streams (what RansEncoder.encode_with_indexes
 * writes for one image: 64-bit state, 32-bit words, 16-bit CDFs, escapes as
 * 4-bit bypass groups), one stream per batch row, into int32 symbols [B, N].
 * The streams lie back to back in streams_dev (streams_bytes bytes); stream b
 * is bytes [offsets_dev[b], offsets_dev[b + 1]) (B + 1 int64 offsets in device
 * memory, multiples of 4).  indexes_dev [B, N], or NULL: position i uses table
 * i / (N / C) (EntropyBottleneck).  tables: gaans_tables_prepare of the same
 * CDFs.  Status (as in gaans_decode_symbols): GAANS_ST_CORRUPT when a stream
 * is too short, ends early or holds an impossible escape, GAANS_ST_INDEX for
 * an index >= M.  One lane decodes one stream (a stream is one serial chain).
 * Replaces CompressAI's RansDecoder.decode_with_indexes as the reference's
 * coder="rans" path calls it (src/fast_compressai/coders/compressai_ans.py:51-87)
 * and the reference's per-chunk GPU decode loop
 * (src/fast_compressai/coders/cuda/ans_gpu_kernel.cu:295-394). */
int gaans_rans64_decode(void* stream, const uint8_t* streams_dev, int64_t streams_bytes,
                        const int64_t* offsets_dev, const int32_t* indexes_dev,
                        const gaans_tables* tables, int64_t B, int64_t N, int64_t C,
                        int32_t* out_dev, void* ctrl_dev, uint32_t* status_out);

/* The same CompressAI Rans64 streams decoded on the host CPU, for batches too
 * small to fill the GPU: host pointers only (streams: B concatenated byte
 * strings, stream b at bytes [stream_offsets[b], stream_offsets[b + 1]);
 * indexes int32 [B, N] or NULL for table = channel; CompressAI's tables cdfs
 * [M, Lmax], cdf_sizes [M], offsets [M]).  Streams are shared out over
 * `threads` threads (<= 0: one per hardware thread).  out: int32 [B, N];
 * *status: the OR of GAANS_ST_CORRUPT (short stream, impossible escape,
 * value outside int32) and GAANS_ST_INDEX over the streams (a stream stops at
 * its first error).  Returns GAANS_ETABLE for tables that are not 16-bit
 * quantized CDFs.  Replaces CompressAI's RansDecoder.decode_with_indexes on
 * the reference's CPU path (src/fast_compressai/coders/compressai_ans.py:51-87). */
int gaans_rans64_decode_host(const uint8_t* streams, const int64_t* stream_offsets,
                             const int32_t* indexes, const int32_t* cdfs,
                             const int32_t* cdf_sizes, const int32_t* offsets, int32_t M,
                             int32_t Lmax, int64_t B, int64_t N, int64_t C, int32_t threads,
                             int32_t* out, uint32_t* status);

/* ---- completion ------------------------------------------------------------ */

/* Wait on the host for a launch's completion word (encode: low half of
 * info_out[2]; decode: status_out[1]) in pinned host memory that the caller
 * set to 0 before the launch.  Returns GAANS_OK once the word is nonzero; the
 * word itself carries the size and status (info_out[0..1] and status_out[0]
 * are only guaranteed after the stream has finished).  The packing (the fused
 * encode kernel's own, or the pack kernel) may still run, and later work is
 * ordered after it on `stream` as usual.  Returns
 * GAANS_EHIP when the stream reports an error or drains without setting the
 * word.  Replaces the stream synchronisations of the reference's host code
 * (warp_ans_kernel_v2.cu:275-276, warp_div.py:63-65). */
int gaans_wait_host_word(void* stream, const uint32_t* word);

/* ---- call plans: repeated calls of one shape --------------------------------- */

/* A plan is the shape-dependent part of an encode (coding + pack launch) or
 * decode launch -- layout, LDS staging plan, kernel variant, launch geometry
 * and argument block -- computed once by gaans_plan_encode / gaans_plan_decode
 * with the device it will run on current.  gaans_run_encode / gaans_run_decode
 * then only set the call's pointers, enqueue and wait: the same bytes as the
 * gaans_encode_* + gaans_encode_pack + gaans_wait_host_word and
 * gaans_decode_* + gaans_wait_host_word sequences (the encode in one fused
 * kernel instead of two), without recomputing the
 * plan or converting a long argument list on every call.  A plan refers to
 * the table blob at tables->dev: the blob must outlive every run of the plan.
 * A plan is plain bytes owned by the caller; runs only read it, so one plan
 * may serve several streams (each with its own control block).  No
 * counterpart in the reference, whose host code recomputes its launch on
 * every call (warp_ans_kernel_v2.cu:183-306, warp_ans_kernel.cu:477-544). */
#define GAANS_PLAN_BYTES 1536
typedef struct gaans_plan {
  uint64_t opaque[GAANS_PLAN_BYTES / 8];
} gaans_plan;

/* plan modes: the inputs a run takes (see gaans_run_encode / _decode) */
#define GAANS_MODE_SYMBOLS 0  /* int32 symbols (gaans_encode_symbols / gaans_decode_symbols) */
#define GAANS_MODE_LATENTS 1  /* fp32 latents + medians (gaans_encode_latents / _decode_latents) */
#define GAANS_MODE_GAUSSIAN 2 /* GaussianConditional (gaans_encode_gaussian / _decode_gaussian) */

/* Plan an encode of B x N symbols (C channels, P per chunk, `segments` per
 * chunk) with `tables`.  explicit_indexes: runs pass an indexes array (0:
 * table = channel; ignored for GAANS_MODE_GAUSSIAN).  n_scales and
 * scale_bound: the Gaussian scale table's length and CompressAI's lower scale
 * bound (ignored for the other modes). */
int gaans_plan_encode(const gaans_tables* tables, int32_t mode, int32_t explicit_indexes,
                      int32_t n_scales, float scale_bound, int64_t B, int64_t N, int64_t C,
                      int64_t P, int32_t segments, gaans_plan* plan);

/* Plan a decode; arguments as for gaans_plan_encode. */
int gaans_plan_decode(const gaans_tables* tables, int32_t mode, int32_t explicit_indexes,
                      int32_t n_scales, float scale_bound, int64_t B, int64_t N, int64_t C,
                      int64_t P, int32_t segments, gaans_plan* plan);

/* Encode with a plan: enqueue one kernel on `stream` that codes every unit
 * and packs the payload into out_dev (at least the layout's
 * max_payload_bytes), then wait for the completion word info_host[2]
 * (pinned host memory, 3 u64; the run clears it before the launch).  On
 * return info_host[2] = 1 | status << 1 | payload bytes << 16, as for
 * gaans_encode_symbols; the kernel may still be writing other units' words,
 * ordered on `stream` before any later work.  The pack is fused: each unit
 * takes its number from a ticket counter in the control block, publishes its
 * size, finds its payload offset by a decoupled look-back over the units
 * before it (workspace words at layout->ws_look, which must be zero before
 * the first such launch on a workspace; every launch leaves them zero) and
 * writes its own part of the payload.  Device inputs by mode:
 *   GAANS_MODE_SYMBOLS:  in0 symbols int32 [B, N], in1 indexes int32 [B, N]
 *                        (NULL for a table = channel plan)
 *   GAANS_MODE_LATENTS:  in0 y fp32 [B, N], in1 medians fp32 [C], in2 indexes
 *                        (as above)
 *   GAANS_MODE_GAUSSIAN: in0 y, in1 means (or NULL), in2 scales, all fp32
 *                        [B, N]; in3 the scale table (n_scales fp32)
 * Unused inputs are ignored.  Reference: encode_with_indexes_warp_v2_cuda
 * (warp_ans_kernel_v2.cu:183-306: six launches and two host syncs). */
int gaans_run_encode(const gaans_plan* plan, void* stream, const void* in0, const void* in1,
                     const void* in2, const void* in3, void* workspace_dev,
                     int64_t workspace_bytes, void* ctrl_dev, uint8_t* out_dev,
                     int64_t out_bytes, uint64_t* info_host);

/* gaans_run_encode without the wait: enqueue the fused encode kernel and
 * return.  info_out (3 u64, device or pinned host memory) receives the
 * payload size, status and completion word as for gaans_encode_symbols.  For
 * callers that order their own work after the encode (graph capture,
 * pipelines, kernel timing).  No counterpart in the reference. */
int gaans_enqueue_encode(const gaans_plan* plan, void* stream, const void* in0, const void* in1,
                         const void* in2, const void* in3, void* workspace_dev,
                         int64_t workspace_bytes, void* ctrl_dev, uint8_t* out_dev,
                         int64_t out_bytes, uint64_t* info_out);

/* Decode with a plan into out_dev (int32 symbols for GAANS_MODE_SYMBOLS, fp32
 * y_hat otherwise, [B, N]) and wait for the completion word status_host[1]
 * (pinned host memory, 2 u32; cleared by the run); status_host[0] and the
 * word's status bits as for gaans_decode_symbols.  Device inputs by mode:
 *   GAANS_MODE_SYMBOLS:  in0 indexes (NULL for a table = channel plan)
 *   GAANS_MODE_LATENTS:  in0 medians fp32 [C], in1 indexes (as above)
 *   GAANS_MODE_GAUSSIAN: in0 scales, in1 means (or NULL), in2 the scale table */
int gaans_run_decode(const gaans_plan* plan, void* stream, const uint8_t* payload_dev,
                     int64_t payload_bytes, const void* in0, const void* in1, const void* in2,
                     void* out_dev, void* ctrl_dev, uint32_t* status_host);

/* gaans_run_decode without the wait: enqueue the decode kernel and return;
 * status_out (2 u32, device or pinned host memory) as for
 * gaans_decode_symbols.  No counterpart in the reference. */
int gaans_enqueue_decode(const gaans_plan* plan, void* stream, const uint8_t* payload_dev,
                         int64_t payload_bytes, const void* in0, const void* in1,
                         const void* in2, void* out_dev, void* ctrl_dev, uint32_t* status_out);

/* gaans_run_encode / gaans_run_decode with their arguments in one struct
 * (same meaning, same behaviour): for bindings whose per-call cost is the
 * argument conversion itself (ctypes converts each argument on every call),
 * which keep one struct per plan and stream, set the fields that change
 * (inputs, output, workspace) and pass its address.  No counterpart in the
 * reference (its binding is a pybind11 module, ans_gpu.cpp:25-30). */
typedef struct gaans_encode_call {
  const gaans_plan* plan;
  void* stream;
  const void* in[4];
  void* workspace_dev;
  int64_t workspace_bytes;
  void* ctrl_dev;
  uint8_t* out_dev;
  int64_t out_bytes;
  uint64_t* info_host;
} gaans_encode_call;

typedef struct gaans_decode_call {
  const gaans_plan* plan;
  void* stream;
  const uint8_t* payload_dev;
  int64_t payload_bytes;
  const void* in[3];
  void* out_dev;
  void* ctrl_dev;
  uint32_t* status_host;
} gaans_decode_call;

int gaans_run_encode_call(const gaans_encode_call* call);
int gaans_run_decode_call(const gaans_decode_call* call);

/* ---- measurement ------------------------------------------------------------ */

/* Phase timestamps of later encode and decode launches (measurement only; a
 * library built with GAANS_PHASE_TIMES defined -- the default build returns
 * GAANS_EINVAL for a non-NULL buffer and its kernels record nothing):
 * with buffer_dev set (device memory of GAANS_PHASE_SLOTS u64 per coding
 * unit, `units` units), unit u < units of every later gaans_encode_* /
 * gaans_decode_* / gaans_run_* launch writes slots of buffer_dev[16u ..
 * 16u + 15]: the device's constant-rate real-time counter
 * (hipDeviceAttributeWallClockRate) at 0 kernel entry, 1 the unit's first
 * loads returned (payload header, table header and metadata; the mark
 * waits for them), 2 tables staged,
 * 3 the first coding step (first block ready), 4 after the last step,
 * 5 before and 6 after the unit's completion-counter atomic (fused encode:
 * its look-back), 7 (the unit that wrote the completion word) after it; the
 * fused encode's pack at 8 (the unit's payload offset known), 9 (the word
 * stores issued) and 10 (its stores completed); the shader clock at 12 the
 * first and 13 after the last step, 14 the shader cycles the coder wave spent
 * in its block barriers, and 15 the coder wave's XCC_ID << 32 | HW_ID.
 * Other slots are not written.  NULL (or
 * units <= 0) turns it off; a launch picks the setting up when it is bound,
 * so it is process-wide and not for concurrent callers.  The points are taken
 * in scalar registers and stored once per unit.  wall_clock_khz (may be NULL) receives the real-time
 * counter's rate on the current device.  No counterpart in the reference. */
#define GAANS_PHASE_SLOTS 16
int gaans_debug_phases(void* buffer_dev, int64_t units, int32_t* wall_clock_khz);

/* ---- host self test ------------------------------------------------------- */

/* Checks the host-computed division constants the kernels use; returns 0
 * when every check passes (no GPU needed). */
int gaans_host_selftest(void);

#ifdef __cplusplus
}
#endif
#endif
