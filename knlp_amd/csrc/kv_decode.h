// Shared declarations of the split-K decode kernels (gfx950).
#pragma once

#include "kv_quant.h"

namespace knlp {

// Storage class of a plane inside the decode kernels.
enum : int { kInt4 = 0, kInt8 = 1, kFp16 = 2 };

__host__ __device__ constexpr int storage_of(int format) {
  return format == KNLP_KV_FP16 ? kFp16 : (format == KNLP_KV_INT8_SYM ? kInt8 : kInt4);
}

// The token being decoded, appended by the decode launch itself: one fp16 /
// bf16 K and V row per sequence, written at slot_mapping[seq] (slot < 0:
// nothing to write).  key == value == nullptr: no append.
struct AppendArgs {
  const uint16_t* key;      // [num_seqs, Hkv, D]
  const uint16_t* value;
  int64_t kst, ksh, vst, vsh;
  const void* slots;
  int slots64;
  int src_bf16;
  float clip_ratio;
};

// Everything a decode-partial launch needs; passed by value as a kernel arg.
struct DecodeArgs {
  const uint16_t* q;        // [num_seqs, Hq, D] fp16 or bf16 bits
  int64_t q_stride_seq, q_stride_head;
  int q_bf16;
  int num_seqs, num_q_heads, num_kv_heads, group;   // group = Hq / Hkv
  knlp_kv_plane kp, vp;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* seq_lens;
  int block_size;
  int block_shift;          // log2(block_size) when it is a power of two, else -1
  int split_tokens, num_splits;
  int max_context;          // block-table width * block_size; longer seq_lens are clamped
  float scale_log2;         // softmax_scale * log2(e)
  float* part_o;            // [num_seqs, Hq, num_splits, D]
  float* part_ml;           // [num_seqs, Hq, num_splits, 2]  (max in log2 units, sum)
  // stream schedule (split_tokens == 0): one block per CU over the flattened
  // tiles of all (sequence, head group) rows; partial entry
  // (block + row) * HG + head-in-group, HG = 8 * group; row_meta[seq * hq +
  // q head] = (its first entry, entry count); stream_hdr[0] = HG, the stride
  // of a q head's entries (read by the merge)
  int stream;               // the block count P of the stream schedule, else 0
  // tiles of work charged for each row a stream block starts (its first
  // loads and pipeline fill): shares are equal in tiles + charges
  int stream_row_cost;
  int32_t* row_meta;
  int32_t* stream_hdr;
  AppendArgs app;
};

// Stream schedule workspace: header (4 int32), per-(sequence, q head) records
// of the partials (first entry, count), then the partials of at most
// (blocks + num_seqs) * hq entries.  Rows are (sequence, group of 8 kv heads)
// pairs.  The records are per q head so that the merge can load a record, the
// header and the sequence length together, without one depending on another.
struct StreamViews {
  int32_t* hdr;
  int32_t* meta;
  float* part_ml;
  float* part_o;
};

inline int64_t stream_entries(int num_seqs, int hq, int blocks) {
  return (static_cast<int64_t>(blocks) + num_seqs) * hq;
}

inline int64_t stream_meta_ints(int num_seqs, int hq) {
  return (2 * static_cast<int64_t>(num_seqs) * hq + 3) / 4 * 4;
}

inline int64_t stream_workspace_bytes(int num_seqs, int hq, int d, int blocks) {
  return 16 + 4 * stream_meta_ints(num_seqs, hq) + stream_entries(num_seqs, hq, blocks) * (d + 2) * 4;
}

// Header of a stream workspace: hdr[0] = query heads per row (> 0) when the
// stream schedule ran; hdr[0] = 0 when the planes sent the call to split-K
// instead, with hdr[1] = split_tokens and hdr[2] = splits, the partials then
// [num_seqs, hq, splits] over the entries.  One small kernel writes it (no
// memset: the call may be captured in a graph).
int launch_stream_header(int32_t* hdr, int h0, int h1, int h2, hipStream_t stream);

inline StreamViews stream_views(void* ws, int num_seqs, int hq, int d, int blocks) {
  StreamViews v;
  v.hdr = static_cast<int32_t*>(ws);
  v.meta = v.hdr + 4;
  v.part_ml = reinterpret_cast<float*>(v.meta + stream_meta_ints(num_seqs, hq));
  v.part_o = v.part_ml + 2 * stream_entries(num_seqs, hq, blocks);
  (void)d;
  return v;
}

// Fused append: the workgroup whose split holds position seq_len - 1 (the
// token being decoded, whose slot the caller passes) quantises that token's
// K and V row of kv head `kvh` into the caches before it reads any page.
// Called by whole waves; returns after this wave's stores have completed
// (s_waitcnt vmcnt(0)), so a later load of the same rows by this wave, or by
// a wave of the same workgroup after a barrier, sees them (one CU, one
// write-through L1).  No other workgroup reads that position.
template <int D>
__device__ __forceinline__ void decode_append_if(const DecodeArgs& a, int seq, int kvh,
                                                 bool holds_last, int lane) {
  const AppendArgs& p = a.app;
  if ((p.key == nullptr && p.value == nullptr) || !holds_last) return;
  const int64_t slot = load_slot(p.slots, p.slots64, seq);
  if (slot < 0) return;
  const int64_t blk = slot / a.block_size;
  const int64_t off = slot % a.block_size;
  // D/2 lanes per row; D = 256 takes two passes over 128-element halves
#pragma unroll
  for (int pass = 0; pass < (D / 2 + kWave - 1) / kWave; ++pass) {
    const int l = lane + kWave * pass;
    if (l < D / 2) {
      if (p.key != nullptr)
        quant_row(p.key + seq * p.kst + kvh * p.ksh, p.src_bf16 != 0, a.kp, blk, off, kvh, l,
                  p.clip_ratio);
      if (p.value != nullptr)
        quant_row(p.value + seq * p.vst + kvh * p.vsh, p.src_bf16 != 0, a.vp, blk, off, kvh, l,
                  p.clip_ratio);
    }
  }
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));   // vmcnt(0): the stores have landed
}

template <int D>
__device__ __forceinline__ void decode_append(const DecodeArgs& a, int seq, int kvh, int split,
                                              int seq_len, int lane) {
  decode_append_if<D>(a, seq, kvh, seq_len > 0 && split == (seq_len - 1) / a.split_tokens, lane);
}

// Workspace split into the two partial arrays.
inline void workspace_views(void* ws, int num_seqs, int hq, int d, int num_splits, float** o,
                            float** ml) {
  *o = static_cast<float*>(ws);
  *ml = *o + static_cast<int64_t>(num_seqs) * hq * num_splits * d;
}

inline int64_t workspace_floats(int num_seqs, int hq, int d, int num_splits) {
  return static_cast<int64_t>(num_seqs) * hq * num_splits * (d + 2);
}

int launch_decode_valu(const DecodeArgs& a, int head_size, int heads_per_block,
                       hipStream_t stream);
int launch_decode_mfma(const DecodeArgs& a, int head_size, hipStream_t stream);
bool mfma_supported(int group, int head_size, int k_format, int k_gs, int v_format, int v_gs,
                    int q_bf16);
int launch_merge(const float* part_o, const float* part_ml, const int32_t* seq_lens,
                 int num_seqs, int hq, int head_size, int max_context, int split_tokens,
                 int num_splits,
                 void* out, int out_bf16, int64_t o_stride_seq, int64_t o_stride_head,
                 hipStream_t stream, const int32_t* stream_meta = nullptr,
                 const int32_t* stream_hdr = nullptr);
// launches the stream schedule (one block per CU) when a.stream is set; false
// if this shape has no cooperative kernel (the stream schedule needs it)
bool stream_supported(const DecodeArgs& a, int head_size);

}  // namespace knlp
