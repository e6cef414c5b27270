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
  AppendArgs app;
};

// Fused append: the workgroup whose split holds position seq_len - 1 (the
// token being decoded, whose slot the caller passes) quantises that token's
// K and V row of kv head `kvh` into the caches before it reads any page.
// Called by whole waves; returns after this wave's stores have completed
// (s_waitcnt vmcnt(0)), so a later load of the same rows by this wave, or by
// a wave of the same workgroup after a barrier, sees them (one CU, one
// write-through L1).  No other workgroup reads that position.
template <int D>
__device__ __forceinline__ void decode_append(const DecodeArgs& a, int seq, int kvh, int split,
                                              int seq_len, int lane) {
  const AppendArgs& p = a.app;
  if ((p.key == nullptr && p.value == nullptr) || seq_len <= 0 ||
      split != (seq_len - 1) / a.split_tokens)
    return;
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
                 hipStream_t stream);

}  // namespace knlp
