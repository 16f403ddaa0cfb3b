/* tritonkv_amd -- C ABI of the MI355X (gfx950) quantized-KV decode-attention kernels.
 *
 * Every entry point is extern "C", takes plain device pointers and sizes,
 * enqueues work on the given hipStream_t, never allocates and never
 * synchronises (so a caller may capture it in a HIP graph), and returns
 *     0            success
 *     < 0          TKV_E* argument error (nothing was launched)
 *     > 0          the hipError_t of a failed launch
 *
 * Data layout is the reference's contract (quantize.py:40-54, :73-146):
 *   packed  uint8  (B, HKV, S, D/P)    P = 8/nbits codes per byte, split-P:
 *                                      bits [p*nbits,(p+1)*nbits) of byte j hold dim j + p*D/P
 *   scale   fp16   (B, HKV, S, D/gs)
 *   zero    fp16   (B, HKV, S, D/gs)
 *   q       fp16 or fp32 (B, HQ, D);  out fp32 (B, HQ, D)
 *   partials acc fp32 (B, HQ, num_splits, D), maxs/sums fp32 (B, HQ, num_splits)
 * All tensors are contiguous row-major.  fp16 values are passed as uint16_t
 * bit patterns.
 */
#ifndef TKV_H_
#define TKV_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *tkv_stream_t; /* == hipStream_t */

enum {
  TKV_OK = 0,
  TKV_EINVAL = -1,       /* inconsistent or out-of-range argument */
  TKV_EUNSUPPORTED = -2, /* valid but not compiled: D, nbits, group size combination,
                            or a cache block past the 32-bit buffer range (below) */
  TKV_ENODEVICE = -3,    /* no HIP device visible */
  TKV_ESCRATCH = -4      /* split partials larger than TKV_NOALLOC_SCRATCH_BYTES */
};

/* Bytes of device memory tkv_fused_decode_attention_noalloc keeps per GPU for
 * the split partials of one call (16 MiB: B*HQ*num_splits*(D + 2)*4 bytes must
 * fit, e.g. 32768 partial rows at D = 128). */
#define TKV_NOALLOC_SCRATCH_BYTES (16u << 20)

/* Arguments of one decode step.  For the quantized path k/v are the packed
 * codes and k_scale/k_zero/v_scale/v_zero the fp16 metadata; for the fp16
 * control path k/v are fp16 (B, HKV, S, D) and the metadata pointers are unused.
 *
 * Buffer range limit: the split kernels address each (b, kv-head) block of a
 * tensor -- each (page, kv-head) slab of a paged pool -- through a buffer
 * resource with a 32-bit byte range, so one block must span less than 2^32
 * bytes: rows * D * nbits / 8 (codes) and rows * (D / group_size) * 2 (scale,
 * zero) on the quantized path, rows * D * 2 on the fp16 control, with rows = S
 * (page_size for a paged pool).  Larger blocks return TKV_EUNSUPPORTED before
 * anything is launched (e.g. 4-bit at D = 128: S < 2^26; the fp16 control at
 * D = 128: S < 2^24).  The quantize / append entry points use 64-bit offsets
 * and have no such limit.
 *
 * S is the token capacity of each (b, kv-head) block.  If seq_lens is NULL every
 * row attends to all S tokens; otherwise row b attends to its first seq_lens[b]
 * tokens (1 <= seq_lens[b] <= S) -- an extension the reference does not have
 * (it uses one S for the whole batch, kernels/fused_decode_attn.py:469).
 *
 * The history [0, S) is cut into num_splits ranges of split_size tokens
 * (the last one ragged).  If num_splits == 1 the kernel writes out directly and
 * acc/maxs/sums may be NULL; otherwise it writes the partials and a combine
 * pass writes out:
 *   counters == NULL   a separate combine kernel (tkv_*_attention) merges them;
 *   counters != NULL   the split kernel's last workgroup of each (b, kv head,
 *                      block of 16 query heads) merges them itself, found by an
 *                      atomic ticket in counters[(b*HKV + kv)*ceil(G/16) + blk].
 *                      The caller zero-fills the B*HKV*ceil(G/16) int32 counters
 *                      once; every call leaves them zero again.  Calls that
 *                      share a counters buffer must not overlap in time.
 * waves: workgroup size in 64-lane waves, 4, 8 or 12 (0 = 4).  12 runs
 *        12 waves where the library has such a kernel (quantized, head_dim
 *        128, contiguous caches, 2-bit gs32 with at most 4 query heads per
 *        KV head, or gs128 with equal K/V bits) and 8 otherwise. */
typedef struct tkv_decode_args {
  const void *q;
  int32_t q_is_fp32;
  const void *k, *k_scale, *k_zero;
  const void *v, *v_scale, *v_zero;
  const int32_t *seq_lens;
  float *acc, *maxs, *sums;
  float *out;
  int32_t B, HQ, HKV, S, D;
  int32_t k_nbits, v_nbits; /* 2 or 4 (K and V may differ); ignored by the fp16 path */
  int32_t group_size;       /* 16, 32, 64 or 128, <= D; ignored by the fp16 path */
  float sm_scale;
  int32_t split_size, num_splits;
  int32_t *counters;
  int32_t waves;
  /* Paged caches (quantized path only): page_size > 0 makes k, k_scale, k_zero,
   * v, v_scale, v_zero pools laid out (num_pages, HKV, page_size, ...), and
   * logical page p of batch row b is pool page block_table[b * block_table_stride + p]
   * (entries outside [0, num_pages) are clamped into the pool).  page_size must
   * be a multiple of 32 and S == block_table_stride * page_size.  page_size == 0:
   * contiguous (B, HKV, S, ...) caches and the block table is unused. */
  const int32_t *block_table;
  int32_t block_table_stride, page_size, num_pages;
  /* Fused append (quantized path only): if k_new != NULL, the step first puts
   * one new token per (b, kv head) into the cache -- k_new/v_new laid out
   * (B, HKV, D), fp16 (new_is_fp32 == 0) or fp32 -- at position L_b - 1, where
   * L_b = seq_lens[b] (or S), quantized exactly as tkv_quantize_pack /
   * tkv_paged_quantize_pack would, and then attends over [0, L_b) including
   * it.  The same result and the same cache bits as that append followed by
   * the decode, in one launch.  A paged token whose table entry lies outside
   * [0, num_pages) is not stored.  No counterpart in the reference (it has no
   * GPU append). */
  const void *k_new, *v_new;
  int32_t new_is_fp32;
  /* Per-channel keys (quantized path only): key_block == 32 makes k_scale /
   * k_zero (B, HKV, S/32, D) -- one fp16 scale and zero per (32-token block,
   * channel), as tkv_quantize_keys_channel writes them -- instead of per-token
   * groups; V keeps its per-token groups, whose group_size must then be 16 or
   * 32.  Contiguous caches only, no fused append, S a multiple of 32.
   * key_block == 0: per-token key groups.  The reference plans this format
   * (docs/future_work.md:229-293) and has no implementation of it. */
  int32_t key_block;
  /* Partials placement: this launch's num_splits splits are partial rows
   * split_base .. split_base + num_splits - 1 of num_splits_total per (b, head)
   * (num_splits_total == 0 means num_splits), so that two launches -- e.g. a
   * quantized history and an fp16 residual window -- fill one set of partials
   * for one combine.  num_splits_total == 1 writes out directly.  The
   * *_attention entry points need split_base == 0 and num_splits_total equal
   * to num_splits (or 0); counters likewise. */
  int32_t split_base, num_splits_total;
  /* Dispatch order (quantized path only; NULL: the natural order).  A caller
   * buffer of 2 * B * HKV * num_splits int32 (8-byte aligned) that the call
   * fills, with one small launch ahead of the split kernel, with a
   * longest-piece-first order of the split workgroups: piece (b, s), tokens
   * [s * split_size, (s + 1) * split_size) of row b, ranked by its length
   * under seq_lens, longest first; each slot holds the workgroup's
   * s * B * HKV + unit and its row's length.
   * The split kernel then takes its (unit, split) from that order, so in a
   * ragged batch the short pieces fill the end of the launch instead of a full
   * piece of a long row starting last.  Every (unit, split) still runs once and
   * writes its own partial row (or, unsplit, its own rows of out), so out is
   * bit-identical to work_order == NULL.  The order launch costs O(B) per
   * piece (B * num_splits pieces).  The fp16 path returns TKV_EUNSUPPORTED and
   * the _noalloc entry TKV_EINVAL for a non-NULL work_order.  No counterpart
   * in the reference (its Triton grid runs splits in program-id order). */
  int32_t *work_order;
} tkv_decode_args;

/* Fused 2/4-bit split-P decode attention: the split kernel, then (if
 * num_splits > 1 and counters == NULL) the log-sum-exp combine kernel.
 * Replaces the two Triton launches of kernels/fused_decode_attn.py:525-568
 * (_fused_decode_attn_split :155-353 and _combine_splits :355-395). */
int tkv_fused_decode_attention(const tkv_decode_args *args, tkv_stream_t stream);

/* fp16 control: identical split, softmax and combine; K/V read as fp16.
 * Replaces kernels/fp16_decode_attn.py:207-239 (_fp16_decode_attn_split :47-135). */
int tkv_fp16_decode_attention(const tkv_decode_args *args, tkv_stream_t stream);

/* tkv_fused_decode_attention that allocates nothing and takes no workspace:
 * the split partials go to a static device array of TKV_NOALLOC_SCRATCH_BYTES
 * that each GPU holds from the library's load until the process ends (its
 * address is looked up once per device, on the first call there).  For callers
 * that cannot call hipMalloc: code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation.  No counterpart in the reference.
 * args->acc, maxs, sums and counters must be NULL; the partials of
 * B * HQ * num_splits rows must fit the scratch (else TKV_ESCRATCH, nothing
 * launched).  Inputs and out are the caller's, exactly as for
 * tkv_fused_decode_attention, and the result is bit-identical to it.  All
 * calls on one GPU share the array, which keeps the last call's contents:
 * calls that overlap in time on one GPU (e.g. on two streams) race. */
int tkv_fused_decode_attention_noalloc(const tkv_decode_args *args, tkv_stream_t stream);

/* The split kernels alone (no combine launch): with num_splits == 1 they write
 * out; otherwise the partials acc/maxs/sums, merged into out by the last
 * workgroup when counters != NULL.  Replace the single launches
 * kernels/fused_decode_attn.py:525-556 and kernels/fp16_decode_attn.py:207-227;
 * used to time the split kernel by itself. */
int tkv_fused_decode_split(const tkv_decode_args *args, tkv_stream_t stream);
int tkv_fp16_decode_split(const tkv_decode_args *args, tkv_stream_t stream);

/* Read-ceiling probe of the quantized split kernel: the same grid, waves,
 * chunk order, two-stage ring and direct-to-LDS loads over the same
 * contiguous caches (args as for tkv_fused_decode_split; no paged caches,
 * fused append or per-channel keys), with no arithmetic behind them, so its
 * duration gives the bandwidth that access pattern can stream.  Writes nothing
 * the caller reads (out[blockIdx.x] only on a sentinel sum).  The measurement
 * counterpart, for this kernel's reads, of the reference's device-copy
 * bandwidth probe (benchmark.py:1160-1222). */
int tkv_read_probe(const tkv_decode_args *args, tkv_stream_t stream);

/* Log-sum-exp merge of split partials into out, as _combine_splits
 * (kernels/fused_decode_attn.py:355-395, launched at :558-568). */
int tkv_combine_splits(const float *acc, const float *maxs, const float *sums, float *out,
                       int32_t B, int32_t HQ, int32_t num_splits, int32_t D,
                       tkv_stream_t stream);

/* Group-wise asymmetric quantize + split-P pack of N new tokens per
 * (b, kv-head), written into a cache at token positions.
 *   x: (B, HKV, N, D) fp16 (x_is_fp32 == 0) or fp32
 *   positions: NULL (write tokens [0, N)) or B int32 start positions; the
 *              tokens of batch row b land at [positions[b], positions[b] + N)
 *   packed/scale/zero: caches of capacity S_cap tokens per (b, kv-head)
 * Bit-exact with quantize_groupwise + pack_codes (quantize.py:186-236,
 * :149-169); used for one-token decode appends and for whole-cache setup. */
int tkv_quantize_pack(const void *x, int32_t x_is_fp32, int32_t B, int32_t HKV, int32_t N,
                      int32_t D, int32_t nbits, int32_t group_size, const int32_t *positions,
                      int32_t S_cap, uint8_t *packed, uint16_t *scale, uint16_t *zero,
                      tkv_stream_t stream);

/* tkv_quantize_pack into a paged cache: row b's N tokens go to logical
 * positions [positions[b], positions[b] + N), i.e. pool page
 * block_table[b * block_table_stride + t / page_size], slot t % page_size, of
 * pools laid out (num_pages, HKV, page_size, ...).  Positions past
 * block_table_stride * page_size, and table entries outside [0, num_pages),
 * are not written.  No counterpart in the reference (its caches are
 * contiguous); the paged form of the decode-step append. */
int tkv_paged_quantize_pack(const void *x, int32_t x_is_fp32, int32_t B, int32_t HKV, int32_t N,
                            int32_t D, int32_t nbits, int32_t group_size,
                            const int32_t *positions, const int32_t *block_table,
                            int32_t block_table_stride, int32_t page_size, int32_t num_pages,
                            uint8_t *packed, uint16_t *scale, uint16_t *zero,
                            tkv_stream_t stream);

/* Decode over per-channel quantized keys plus an fp16 residual window, the
 * format the reference plans (docs/future_work.md:229-293: "the fp16 residual
 * tail goes through the existing fp16 control kernel as one more split, and
 * the existing combine kernel merges it").  args describes the quantized
 * history: key_block == 32, seq_lens (or S) its per-row lengths, num_splits
 * its splits; acc/maxs/sums must hold num_splits + 1 partial rows per
 * (b, head); split_base / num_splits_total / counters are ignored.  k_res,
 * v_res: fp16 (B, HKV, res_cap, D), the window; row b attends to its first
 * res_lens[b] window tokens (0 <= res_lens[b] <= res_cap; NULL = res_cap)
 * after its quantized ones.  Two launches when res_cap <= 32: the quantized
 * split kernel (partial rows 0 .. num_splits-1), then the combine, which
 * attends to the window itself and merges it as one more split.  A longer
 * window takes a third launch, the fp16 split kernel over the window
 * (partial row num_splits), before the combine. */
int tkv_channel_decode_attention(const tkv_decode_args *args, const void *k_res,
                                 const void *v_res, const int32_t *res_lens, int32_t res_cap,
                                 tkv_stream_t stream);

/* Per-channel (KIVI-style) key quantization: x (B, HKV, N, D) fp16/fp32 with
 * N a multiple of 32 is cut into 32-token blocks; within a block every
 * channel is one group (the group-wise arithmetic of quantize_groupwise,
 * quantize.py:209-226, along the token axis).  Codes go to packed
 * (B, HKV, S_cap, D/P) in the split-P row layout, fp16 scale and zero to
 * (B, HKV, S_cap/32, D).  Row b's blocks land at tokens positions[b] + 32k
 * (positions NULL = 0); a block that does not start on a 32-token boundary
 * or does not fit [0, S_cap) is not written.  The reference plans this format
 * (docs/future_work.md:229-293) and has no implementation of it. */
int tkv_quantize_keys_channel(const void *x, int32_t x_is_fp32, int32_t B, int32_t HKV,
                              int32_t N, int32_t D, int32_t nbits, const int32_t *positions,
                              int32_t S_cap, uint8_t *packed, uint16_t *scale, uint16_t *zero,
                              tkv_stream_t stream);

/* The fp16 window of per-channel keys, as two launches per decode step that
 * keep every length on the device (so a captured step replays correctly for
 * any window fill).  k_res / v_res: fp16 (B, HKV, res_cap, D) with res_cap
 * == 32; res_lens / q_lens: int32 (B,) window fills and quantized lengths.
 *
 * tkv_channel_window_append: token (B, HKV, D) fp16 of k_new / v_new goes to
 * window row res_lens[b], which then grows by one (a full window is left
 * unchanged: flush it first).
 *
 * tkv_channel_window_flush: for each row whose window holds 32 tokens, the
 * window is quantized into the history at token q_lens[b] -- keys per channel
 * exactly as tkv_quantize_keys_channel, values per token exactly as
 * tkv_quantize_pack (V group_size 16 or 32) -- then q_lens[b] += 32 and
 * res_lens[b] = 0.  Other rows are untouched.  A full window that does not
 * fit the history (q_lens[b] + 32 > S_cap) is not written and no length
 * moves: res_lens[b] becomes 33, a device-side overflow mark that the append
 * treats as full and the decode clamps to the window's 32 tokens.  No counterpart in the
 * reference (it plans the format, docs/future_work.md:229-293). */
int tkv_channel_window_append(const void *k_new, const void *v_new, int32_t B, int32_t HKV,
                              int32_t D, void *k_res, void *v_res, int32_t res_cap,
                              int32_t *res_lens, tkv_stream_t stream);
int tkv_channel_window_flush(const void *k_res, const void *v_res, int32_t B, int32_t HKV,
                             int32_t D, int32_t k_nbits, int32_t v_nbits, int32_t group_size,
                             int32_t res_cap, int32_t *q_lens, int32_t *res_lens, int32_t S_cap,
                             uint8_t *k_packed, uint16_t *k_scale, uint16_t *k_zero,
                             uint8_t *v_packed, uint16_t *v_scale, uint16_t *v_zero,
                             tkv_stream_t stream);

/* Split-P pack of uint8 codes (rows, D) -> (rows, D/P), as pack_codes
 * (quantize.py:149-169). */
int tkv_pack_codes(const uint8_t *codes, int64_t rows, int32_t D, int32_t nbits,
                   uint8_t *packed, tkv_stream_t stream);

/* Unpack + fp32 dequantize rows of a quantized cache, through the same
 * register unpack the decode kernel uses (path 0: the K-operand extraction,
 * path 1: the transposed V-operand extraction).  codes_out (rows, D) uint8
 * and/or values_out (rows, D) fp32 = code * scale + zero; either may be NULL.
 * As unpack_codes / dequantize_groupwise (quantize.py:172-183, :239-246). */
int tkv_unpack_dequant(const uint8_t *packed, const uint16_t *scale, const uint16_t *zero,
                       int64_t rows, int32_t D, int32_t nbits, int32_t group_size,
                       int32_t path, uint8_t *codes_out, float *values_out,
                       tkv_stream_t stream);

typedef struct tkv_device_info_t {
  int32_t device;
  int32_t compute_units;
  int32_t warp_size;
  int32_t l2_bytes;
  int64_t global_mem_bytes;
  int32_t clock_khz;
  int32_t mem_clock_khz;
  int32_t mem_bus_bits;
  char gcn_arch[64];
} tkv_device_info_t;

/* Properties of the current device (the one the calling thread has selected). */
int tkv_device_info(tkv_device_info_t *info);

/* Human-readable text for a status code returned by any tkv_ function. */
const char *tkv_status_string(int status);

/* ABI version of this library (bumped on any incompatible change; 3 added the
 * paged-cache fields of tkv_decode_args and tkv_paged_quantize_pack, 4 the
 * fused-append fields, 5 the per-channel key and partials-placement fields,
 * tkv_quantize_keys_channel, tkv_channel_decode_attention and the
 * tkv_channel_window_* calls, 6 tkv_fused_decode_attention_noalloc,
 * TKV_ESCRATCH and tkv_read_probe, 7 the work_order field). */
int tkv_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TKV_H_ */
