// Stage 2 (matrix-core path), host side: which shapes the matrix-core
// kernels take and which of the three kernel families a launch goes to.  The
// kernels themselves are in kv_decode_mfma.h, instantiated by
// kv_decode_mfma_perhead.hip, kv_decode_mfma_coop.hip and
// kv_decode_mfma_stream.hip.
#include "kv_decode_mfma.h"

namespace knlp {

// Shapes the matrix-core path takes: INT4 V with 1, 2 or 4 scale groups
// (or, at D = 128, INT8 V with 1 or 4; or fp16 K with INT4 or INT8 V and one
// head set, on the per-head kernel),
// fp16 or bf16 q, D = 64 or 128, K packed INT4 with V's groups or (D = 128) INT8 with
// one scale per row or V's groups, and at most two head sets of 16 rows.  The
// per-head kernel covers INT4 K with one head set; the other shapes need the
// cooperative kernel's dense layout and otherwise run on the VALU kernel.
bool mfma_supported(int group, int head_size, int k_format, int k_gs, int v_format, int v_gs,
                    int q_bf16) {
  const auto int4 = [](int f) { return f == KNLP_KV_INT4_SYM || f == KNLP_KV_INT4_ASYM; };
  (void)q_bf16;        // bf16 q is converted exactly in init_wave
  const bool v8 = v_format == KNLP_KV_INT8_SYM;
  // fp16 K and V: per-head kernel, one head set (the rows are the q heads)
  if (v_format == KNLP_KV_FP16)
    return k_format == KNLP_KV_FP16 && (head_size == 64 || head_size == 128) && group >= 1 &&
           group <= 16;
  if (!(int4(v_format) || v8) || v_gs <= 0) return false;
  if (head_size != 64 && head_size != 128) return false;
  if (head_size % v_gs) return false;
  const int ng = head_size / v_gs;
  if (ng != 1 && ng != 2 && ng != 4) return false;
  // INT8 V: D = 128 with one scale per row or g32 (cooperative kernel only)
  if (v8 && (head_size != 128 || (ng != 1 && ng != 4))) return false;
  if (int4(k_format)) {
    if (k_gs != v_gs) return false;
  } else if (k_format == KNLP_KV_INT8_SYM) {
    if (head_size != 128 || (k_gs != head_size && k_gs != v_gs)) return false;
  } else if (k_format == KNLP_KV_FP16) {
    // fp16 K on the per-head kernel: INT4 or INT8 V, one head set
    return group >= 1 && group * ng <= 16;
  } else {
    return false;
  }
  return group >= 1 && group * ng <= 32;
}

// Heads densely packed in a token row, 16-byte aligned rows, Hkv a multiple
// of the kv heads per block (`heads`: 8, or 4 for fp16 K): the cooperative
// kernel can fetch a block's heads' rows as one contiguous run.
static bool coop_layout_ok(const knlp_kv_plane& P, int head_size, int num_kv_heads, int heads) {
  const bool f16 = P.format == KNLP_KV_FP16;
  const int64_t eb = f16 ? 2 : 1;                         // strides are in elements
  const int64_t ng = f16 ? 1 : head_size / P.group_size;
  const int64_t row = f16 || P.format == KNLP_KV_INT8_SYM ? head_size : head_size / 2;
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (num_kv_heads % heads != 0) return false;
  if (!a16(P.data) || P.stride_head != row || (eb * P.stride_block) % 16 != 0 ||
      (eb * P.stride_page) % 16 != 0 || eb * P.stride_block >= (1LL << 31) ||
      eb * P.stride_page >= (1LL << 31))
    return false;
  if (f16) return true;                                   // no scales or zero-points
  const auto scales_ok = [&](const void* p, int64_t sb, int64_t sp, int64_t sh) {
    return a16(p) && sh == ng && (2 * sb) % 16 == 0 && (2 * sp) % 16 == 0 &&
           2 * sb < (1LL << 31) && 2 * sp < (1LL << 31);
  };
  if (!scales_ok(P.scales, P.s_stride_block, P.s_stride_page, P.s_stride_head)) return false;
  if (P.format == KNLP_KV_INT4_ASYM &&
      !scales_ok(P.zeros, P.z_stride_block, P.z_stride_page, P.z_stride_head))
    return false;
  return true;
}

// fp16 K on the cooperative loader: D = 128, 4 kv heads per block, dense
// layouts (the shapes mfma_supported admits for fp16 K: one head set), V in
// fp16 or with 2 or 4 scale groups (with one scale per row, 4 heads' V
// scales of a token are 8 bytes, less than the 16-byte chunk a lane copies).
static bool coop16_ok(const DecodeArgs& a, int head_size) {
  const bool vrows_ok = a.vp.format == KNLP_KV_FP16 || head_size / a.vp.group_size >= 2;
  return a.kp.format == KNLP_KV_FP16 && head_size == 128 && vrows_ok &&
         coop_layout_ok(a.kp, head_size, a.num_kv_heads, 4) &&
         coop_layout_ok(a.vp, head_size, a.num_kv_heads, 4);
}

bool stream_supported(const DecodeArgs& a, int head_size) {
  if (!mfma_supported(a.group, head_size, a.kp.format, a.kp.group_size, a.vp.format,
                      a.vp.group_size, a.q_bf16))
    return false;
  if (a.kp.format == KNLP_KV_FP16) return coop16_ok(a, head_size);
  return coop_layout_ok(a.kp, head_size, a.num_kv_heads, 8) &&
         coop_layout_ok(a.vp, head_size, a.num_kv_heads, 8);
}

int launch_decode_mfma(const DecodeArgs& a, int head_size, hipStream_t stream) {
  const int ng = head_size / a.vp.group_size;
  const bool k8 = a.kp.format == KNLP_KV_INT8_SYM;
  const bool v8 = a.vp.format == KNLP_KV_INT8_SYM;
  const bool k16 = a.kp.format == KNLP_KV_FP16;
  const int nset = (a.group * ng + 15) / 16;
  if (k16) {
    // fp16 K: the cooperative loader (4 kv heads per block) on dense layouts
    // at D = 128, else the per-head kernel (any kv-head count, split only)
    if (coop16_ok(a, head_size))
      return a.stream ? launch_mfma_coop_stream(a, head_size, stream)
                      : launch_mfma_coop_split(a, head_size, stream);
    if (a.stream) return KNLP_ERR_SHAPE;
    return launch_mfma_perhead(a, head_size, stream);
  }
  const bool coop = coop_layout_ok(a.kp, head_size, a.num_kv_heads, 8) &&
                    coop_layout_ok(a.vp, head_size, a.num_kv_heads, 8);
  // only the cooperative kernel has these (the per-head kernel takes INT8 V
  // with fp16 K only)
  if (!coop && (k8 || v8 || nset > 1))
    return launch_decode_valu(a, head_size, heads_per_block_mfma(a.num_kv_heads), stream);
  if (a.stream && !coop) return KNLP_ERR_SHAPE;   // the stream schedule is the cooperative kernel's
  // INT4 K and V without the cooperative kernel's dense layout: per-head kernel
  if (!coop) return launch_mfma_perhead(a, head_size, stream);
  return a.stream ? launch_mfma_coop_stream(a, head_size, stream)
                  : launch_mfma_coop_split(a, head_size, stream);
}

}  // namespace knlp
