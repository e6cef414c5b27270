// Stage 1: quantize-on-append into the paged INT4 / INT8 caches (gfx950).
//
// Replaces the reference's _reshape_and_cache_int4_kernel (F:210-415),
// _reshape_and_cache_v_only_int4_kernel (F:481-600),
// _reshape_and_cache_k_int8_kernel (F:1231-1284) and
// _reshape_and_cache_v_int8_kernel (F:1563-1616); F = fused-quant/fused_int4.v0.1.0.py.
//
// Layout of the work: one (token, head) row of D elements is handled by D/2
// consecutive lanes, two elements per lane, so a wave reads 256 contiguous
// bytes of fp16 source and writes 64 contiguous bytes of packed codes.  The
// row quantisers themselves live in kv_quant.h (shared with the decode
// kernels' fused append).
#include "kv_quant.h"

namespace knlp {

// One (token, head) row per D/2 lanes; 256 threads per block.
template <int D>
__global__ __launch_bounds__(256) void kv_append_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value, int src_bf16,
    int64_t num_tokens, int num_heads, int64_t kst, int64_t ksh, int64_t vst, int64_t vsh,
    knlp_kv_plane KP, knlp_kv_plane VP, const void* __restrict__ slots, int slots64,
    int block_size, float clip_ratio) {
  constexpr int L = D / 2;
  constexpr int IPB = 256 / L;
  const int lane = threadIdx.x % L;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * IPB + threadIdx.x / L;
  if (item >= num_tokens * num_heads) return;
  const int64_t tok = item / num_heads;
  const int head = static_cast<int>(item % num_heads);
  const int64_t slot = load_slot(slots, slots64, tok);
  if (slot < 0) return;                               // padding token, F:266-268
  const int64_t blk = slot / block_size;
  const int64_t off = slot % block_size;
  if (key != nullptr)
    quant_row(key + tok * kst + head * ksh, src_bf16 != 0, KP, blk, off, head, lane, clip_ratio);
  if (value != nullptr)
    quant_row(value + tok * vst + head * vsh, src_bf16 != 0, VP, blk, off, head, lane,
              clip_ratio);
}

int launch_append(const void* key, const void* value, int src_bf16, int64_t num_tokens,
                  int num_heads, int head_size, int64_t kst, int64_t ksh, int64_t vst,
                  int64_t vsh, const knlp_kv_plane& KP, const knlp_kv_plane& VP,
                  const void* slots, int slots64, int block_size, float clip_ratio,
                  hipStream_t stream) {
  const int64_t items = num_tokens * num_heads;
  const int ipb = 256 / (head_size / 2);
  const int64_t blocks = (items + ipb - 1) / ipb;
  if (blocks == 0) return KNLP_OK;
  if (blocks > 0x7FFFFFFF) return KNLP_ERR_SHAPE;
  const auto* k = static_cast<const uint16_t*>(key);
  const auto* v = static_cast<const uint16_t*>(value);
  switch (head_size) {
#define KNLP_APPEND_D(D)                                                              \
  case D:                                                                             \
    hipLaunchKernelGGL(kv_append_kernel<D>, dim3(static_cast<uint32_t>(blocks)),      \
                       dim3(256), 0, stream, k, v, src_bf16, num_tokens, num_heads,   \
                       kst, ksh, vst, vsh, KP, VP, slots, slots64, block_size,        \
                       clip_ratio);                                                   \
    break;
    KNLP_APPEND_D(32)
    KNLP_APPEND_D(64)
    KNLP_APPEND_D(128)
    KNLP_APPEND_D(256)
#undef KNLP_APPEND_D
    default:
      return KNLP_ERR_SHAPE;
  }
  return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
}

}  // namespace knlp
