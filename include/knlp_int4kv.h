/*
 * knlp_int4kv.h -- C ABI of the MI355X (gfx950) INT4/INT8 KV-cache
 * quantize-on-append and split-K decode-attention library.
 *
 * Every entry point takes raw device pointers, element strides, sizes and a
 * hipStream_t (passed as void*), launches onto that stream, allocates nothing
 * and never synchronises, so the calls are safe inside HIP graph capture.
 * Return value: KNLP_OK (0) or a negative KNLP_ERR_* status; nothing is
 * launched when the status is negative.
 *
 * Cache layouts are the reference's (mcgrof/knlp,
 * fused-quant/fused_int4.v0.1.0.py = "F"):
 *   packed INT4 codes  uint8 [num_blocks, block_size, num_kv_heads, D/2]
 *                      low nibble = element 2i, high nibble = 2i+1 (F:359)
 *   INT8 codes         int8  [num_blocks, block_size, num_kv_heads, D]
 *   fp16 cache         fp16  [num_blocks, block_size, num_kv_heads, D]
 *   scales / zeros     fp16  [num_blocks, block_size, num_kv_heads, D/G]
 *   slot = block * block_size + offset; slot < 0 is skipped (F:266-271).
 */
#ifndef KNLP_INT4KV_H
#define KNLP_INT4KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KNLP_ABI_VERSION 1

enum knlp_status {
  KNLP_OK = 0,
  KNLP_ERR_SHAPE = -1,      /* unsupported or inconsistent sizes */
  KNLP_ERR_DTYPE = -2,      /* unsupported element type / format */
  KNLP_ERR_ALIGN = -3,      /* pointer or stride alignment violated */
  KNLP_ERR_WORKSPACE = -4,  /* workspace missing or too small */
  KNLP_ERR_LAUNCH = -5,     /* the HIP launch itself failed */
  KNLP_ERR_ARG = -6         /* null pointer or invalid scalar argument */
};

/* element types of query / key / value / output tensors and index arrays */
enum knlp_dtype {
  KNLP_DT_F16 = 0,
  KNLP_DT_BF16 = 1,
  KNLP_DT_I32 = 2,
  KNLP_DT_I64 = 3
};

/* storage format of one cache plane (K or V) */
enum knlp_kv_format {
  KNLP_KV_INT4_SYM = 0,   /* codes (n-8)*scale, F:328-357 */
  KNLP_KV_INT4_ASYM = 1,  /* codes n*scale + zero, F:308-327 */
  KNLP_KV_INT8_SYM = 2,   /* int8 n*scale, F:1270-1284 */
  KNLP_KV_FP16 = 3        /* plain fp16 cache, no scales */
};

/*
 * One paged cache plane: codes plus per-group fp16 scale (and zero-point for
 * KNLP_KV_INT4_ASYM).  Strides are in elements of the respective array
 * (bytes for uint8/int8 codes, halves for fp16 arrays) over the
 * (block, page-offset, head) axes; the last axis must be contiguous.
 * The reference passes the same numbers as separate Triton kernel arguments
 * (F:226-250, F:676-697).
 */
typedef struct knlp_kv_plane {
  void* data;
  void* scales;             /* NULL for KNLP_KV_FP16 */
  void* zeros;              /* used only by KNLP_KV_INT4_ASYM */
  int64_t stride_block, stride_page, stride_head;
  int64_t s_stride_block, s_stride_page, s_stride_head;
  int64_t z_stride_block, z_stride_page, z_stride_head;
  int32_t format;           /* enum knlp_kv_format */
  int32_t group_size;       /* elements per scale group along head_dim; not
                               read for KNLP_KV_FP16 planes (no scales: any
                               value, 0 included, is taken as head_size) */
} knlp_kv_plane;

int knlp_abi_version(void);
const char* knlp_status_string(int status);

/*
 * Quantize-on-append.  Replaces reshape_and_cache_int4 (F:418-472),
 * reshape_and_cache_v_only_int4 (F:603-647, key == NULL),
 * reshape_and_cache_k_int8 (F:1287-1312, key plane format INT8, value NULL)
 * and reshape_and_cache_v_int8 (F:1619-1650, value plane format INT8).
 * key / value: [num_tokens, num_heads, head_size] fp16 or bf16 (src_dtype),
 * last axis contiguous.  clip_ratio is the symmetric INT4 trimmed-mean clip
 * (F:70-72); 0 disables it.  slot_mapping: [num_tokens] int32 or int64.
 */
int knlp_kv_append(const void* key, const void* value, int32_t src_dtype,
                   int64_t num_tokens, int32_t num_heads, int32_t head_size,
                   int64_t key_stride_token, int64_t key_stride_head,
                   int64_t value_stride_token, int64_t value_stride_head,
                   const knlp_kv_plane* key_cache,
                   const knlp_kv_plane* value_cache,
                   const void* slot_mapping, int32_t slot_dtype,
                   int32_t block_size, float clip_ratio, void* stream);

/*
 * Split-K plan: tokens per split for a batch of num_seqs sequences taken at
 * max_context each (= block-table width * block_size; no device read-back),
 * for K/V planes of the given knlp_kv_format values, taking one scale per
 * row for INT8 planes and group size 32 for INT4 planes (the reference's
 * default GROUP_SIZE, F:55); knlp_kv_decode_plan takes the group sizes and
 * the batch's total context.  Returns the split length in tokens (> 0) or a
 * negative status.
 */
int32_t knlp_kv_decode_split_tokens(int32_t num_seqs, int32_t num_kv_heads,
                                    int32_t num_q_heads, int32_t head_size,
                                    int32_t max_context, int32_t k_format,
                                    int32_t v_format);

/*
 * Split-K plan with everything the dispatch looks at: group sizes decide
 * which decode kernel runs (and so how many workgroups a CU holds), and
 * total_context -- the sum of the batch's sequence lengths, when the caller
 * knows it on the host (vLLM's metadata does) -- sizes the splits of a
 * variable-length batch from its real work; total_context <= 0 means
 * unknown.  Returns the split length in tokens (> 0, a multiple of 64), 0
 * for the stream schedule (below), or a negative status.  0 is returned,
 * when the cooperative matrix-core kernel takes the planes (Hkv % 8 == 0,
 * INT4/INT8 K, at most 1024 sequences, max_context <= 2^25), for
 * variable-length batches (total context at most 90 % of num_seqs *
 * max_context) and for batches of several sequences whose total is unknown
 * (the stream schedule's equal shares hold for any mix of lengths; splits
 * sized for every sequence at max_context leave a long sequence among short
 * ones to a few workgroups).  No counterpart in the reference (it has
 * no split-K).
 *
 * Stream schedule (split_tokens = 0 in the calls below): one workgroup per
 * CU, each taking an equal share of all (sequence, group of 8 kv heads)
 * rows' 32-token tiles laid end to end, so sequences of any mix of lengths
 * keep every CU busy to the end (in large batches each row a workgroup
 * starts after its first counts as 6 tiles of its share: the row's start-up
 * costs about that); the merge folds each row's per-workgroup partials.  Its workspace depends on num_seqs, not max_context.  Planes the
 * cooperative kernel cannot take (fp16 K, Hkv % 8 != 0, a sparse layout)
 * run split-K inside that workspace instead.  More than 1024 sequences or
 * max_context > 2^25 with split_tokens = 0 is KNLP_ERR_SHAPE.
 */
int32_t knlp_kv_decode_plan(int32_t num_seqs, int32_t num_kv_heads,
                            int32_t num_q_heads, int32_t head_size,
                            int32_t max_context, int64_t total_context,
                            int32_t k_format, int32_t k_group_size,
                            int32_t v_format, int32_t v_group_size);

/* Bytes of fp32 workspace decode needs for this shape and split length
 * (split_tokens = 0: the stream schedule's). */
int64_t knlp_kv_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                       int32_t head_size, int32_t max_context,
                                       int32_t split_tokens);

/*
 * Stage 2: split-K decode attention over paged caches.  Replaces the launch
 * in fused_int4_decode (F:901-979), kint8_vint4_decode (F:1496-1554) and the
 * other precision variants (F:1159-1225, F:1796-1848, F:1975-2028): the
 * reference runs one program per (sequence, q head) over the whole context;
 * here one wave per (sequence, kv head, split) serves all q heads of the GQA
 * group and writes an unnormalised partial (acc, max, sum) per split into the
 * caller's fp32 workspace.
 * query: [num_seqs, num_q_heads, head_size] fp16/bf16; block_table int32
 * [num_seqs, >= ceil(max_context / block_size)]; seq_lens int32 [num_seqs].
 * softmax_scale multiplies q.k (the reference fixes it to 1/sqrt(head_size),
 * F:924).
 */
int knlp_kv_decode_partial(const void* query, int32_t q_dtype,
                           int64_t q_stride_seq, int64_t q_stride_head,
                           int32_t num_seqs, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_size,
                           const knlp_kv_plane* key_cache,
                           const knlp_kv_plane* value_cache,
                           const int32_t* block_table, int64_t bt_stride_seq,
                           const int32_t* seq_lens, int32_t block_size,
                           int32_t max_context, float softmax_scale,
                           int32_t split_tokens, void* workspace,
                           int64_t workspace_bytes, void* stream);

/*
 * Stage 3: merge the per-split partial softmax states (log-sum-exp combine)
 * and write the output [num_seqs, num_q_heads, head_size] in out_dtype
 * (fp32 -> fp16 rounding, then bf16 when out_dtype is bf16, as F:891-894 and
 * the reference's store into empty_like(query) do).  A sequence with
 * seq_len == 0 yields NaN, as the reference's 0/0 does (F:886-887).
 * No counterpart in the reference (it has no split-K).
 */
int knlp_kv_decode_merge(const void* workspace, int64_t workspace_bytes,
                         const int32_t* seq_lens, int32_t num_seqs,
                         int32_t num_q_heads, int32_t head_size,
                         int32_t max_context, int32_t split_tokens,
                         void* out, int32_t out_dtype, int64_t o_stride_seq,
                         int64_t o_stride_head, void* stream);

/* knlp_kv_decode_partial followed by knlp_kv_decode_merge on one stream. */
int knlp_kv_decode(const void* query, int32_t q_dtype, int64_t q_stride_seq,
                   int64_t q_stride_head, int32_t num_seqs, int32_t num_q_heads,
                   int32_t num_kv_heads, int32_t head_size,
                   const knlp_kv_plane* key_cache,
                   const knlp_kv_plane* value_cache,
                   const int32_t* block_table, int64_t bt_stride_seq,
                   const int32_t* seq_lens, int32_t block_size,
                   int32_t max_context, float softmax_scale,
                   int32_t split_tokens, void* workspace,
                   int64_t workspace_bytes, void* out, int32_t out_dtype,
                   int64_t o_stride_seq, int64_t o_stride_head, void* stream);

/*
 * Fused append + decode for one new token per sequence: quantise the token
 * being decoded (key / value: [num_seqs, num_kv_heads, head_size] fp16 or
 * bf16, src_dtype) into the caches at slot_mapping[seq] and run
 * knlp_kv_decode_partial + knlp_kv_decode_merge, in the same two launches as
 * knlp_kv_decode.  No counterpart function in the reference: it replaces
 * the separate reshape_and_cache_* launch (F:418-472, F:603-647,
 * F:1287-1312, F:1619-1650) that F's backend issues before every decode
 * (F:2600-2689), the fusion docs/fused-quant/latency.md:41 proposes.
 * Contract: seq_lens[seq] already counts the new token, and slot_mapping[seq]
 * is the slot of position seq_lens[seq] - 1 of that sequence (or < 0: no
 * write); the workgroup whose split holds that position writes the row
 * before it reads the page, and no other workgroup reads that slot.  The
 * codes are bit-identical to knlp_kv_append's; key or value may be NULL.
 */
int knlp_kv_append_decode(const void* query, int32_t q_dtype, int64_t q_stride_seq,
                          int64_t q_stride_head, int32_t num_seqs, int32_t num_q_heads,
                          int32_t num_kv_heads, int32_t head_size, const void* key,
                          const void* value, int32_t src_dtype, int64_t key_stride_seq,
                          int64_t key_stride_head, int64_t value_stride_seq,
                          int64_t value_stride_head, const void* slot_mapping,
                          int32_t slot_dtype, float clip_ratio,
                          const knlp_kv_plane* key_cache, const knlp_kv_plane* value_cache,
                          const int32_t* block_table, int64_t bt_stride_seq,
                          const int32_t* seq_lens, int32_t block_size, int32_t max_context,
                          float softmax_scale, int32_t split_tokens, void* workspace,
                          int64_t workspace_bytes, void* out, int32_t out_dtype,
                          int64_t o_stride_seq, int64_t o_stride_head, void* stream);

/*
 * Packed INT4 codes in the two's-complement nibble form of the reference's
 * gpt2 compression path (gpt2/compression/kv_plugin.py:212-257: t in [-7, 7]
 * stored as t & 0xF, element 2i in the low nibble) re-encoded in this
 * library's offset form (n = t + 8, decoded as (n - 8) * scale, F:359), so
 * such caches can be decoded as KNLP_KV_INT4_SYM planes with that path's
 * per-row scale (group size = head size).  Byte matrix [rows, row_bytes],
 * row_bytes % 4 == 0, row strides in bytes; dst == src converts in place.
 * No counterpart function in the reference (its expand kernel,
 * kernels/triton_kernels.py:62-232, sign-extends in registers instead).
 */
int knlp_int4_twos_to_offset(const void* src, int64_t src_stride_row, void* dst,
                             int64_t dst_stride_row, int64_t rows, int64_t row_bytes,
                             void* stream);

/*
 * Measurement utility (no counterpart function in the reference; its
 * benchmark keeps a STREAM kernel for the same purpose,
 * scripts/v35_h100_bench.py:99-139): read `bytes` (a multiple of 16) of
 * device memory at `src` once, `blocks` workgroups each streaming one
 * contiguous slice with 16-byte loads, and (almost never) write one word per
 * workgroup into `sink` [blocks] uint32, which keeps the loads live.  Timing
 * it over the decode kernel's byte count gives the sustained-read ceiling the
 * decode is compared with.
 */
int knlp_hbm_read_probe(const void* src, int64_t bytes, void* sink, int32_t blocks,
                        void* stream);

/* Which decode kernel a shape dispatches to: 1 = MFMA path, 0 = VALU path,
 * negative = unsupported (status).  Lets tests and the bench report it.  The
 * MFMA path's INT8-K, INT8-V (with INT4 or INT8 K) and more-than-16-row
 * shapes need num_kv_heads % 8 == 0 (reported as 0 otherwise) and densely
 * packed heads (stride_head = one head's row, assumed here); other layouts
 * of those shapes run on the VALU kernel, which serves at most 8 query heads
 * per kv head (more return KNLP_ERR_SHAPE at decode time).  Group sizes of
 * fp16 planes are not read. */
int knlp_kv_decode_kernel_kind(int32_t num_q_heads, int32_t num_kv_heads,
                               int32_t head_size, int32_t k_format,
                               int32_t k_group_size, int32_t v_format,
                               int32_t v_group_size, int32_t q_dtype);

/*
 * knlp_kv_decode without a workspace argument and without any allocation:
 * the split partials go to a 16 MiB array of device memory that the library
 * holds on each GPU it runs on, from its load until the process ends.  No
 * counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The caller passes inputs and output as for knlp_kv_decode.
 * A shape whose partials need more than 16 MiB
 * (num_seqs * num_q_heads * ceil(max_context / split_tokens) * (head_size +
 * 2) * 4 bytes) returns KNLP_ERR_WORKSPACE.  All calls on one GPU share that
 * GPU's array: calls that overlap on one GPU (two streams, two threads) race
 * and must be serialised by the caller.  Nothing in the array needs to start
 * at zero (every partial the merge reads is written first).
 */
int knlp_kv_decode_noalloc(const void* query, int32_t q_dtype, int64_t q_stride_seq,
                           int64_t q_stride_head, int32_t num_seqs, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_size,
                           const knlp_kv_plane* key_cache,
                           const knlp_kv_plane* value_cache,
                           const int32_t* block_table, int64_t bt_stride_seq,
                           const int32_t* seq_lens, int32_t block_size,
                           int32_t max_context, float softmax_scale,
                           int32_t split_tokens, void* out, int32_t out_dtype,
                           int64_t o_stride_seq, int64_t o_stride_head, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KNLP_INT4KV_H */
