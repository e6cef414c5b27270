// Shared declarations of the split-K decode kernels (gfx950).
#pragma once

#include "kv_common.h"

namespace knlp {

// Storage class of a plane inside the decode kernels.
enum : int { kInt4 = 0, kInt8 = 1, kFp16 = 2 };

__host__ __device__ constexpr int storage_of(int format) {
  return format == KNLP_KV_FP16 ? kFp16 : (format == KNLP_KV_INT8_SYM ? kInt8 : kInt4);
}

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
};

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
