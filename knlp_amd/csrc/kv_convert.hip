// Re-encoding of packed INT4 codes from the two's-complement nibble form of
// the reference's gpt2 compression path into this library's offset form.
//
// gpt2/compression/kv_plugin.py:212-257 packs t in [-7, 7] as (t & 0xF),
// element 2i in the low nibble; this library (and F:359) packs n = t + 8 in
// [0, 15] in the same nibble order and decodes (n - 8) * scale.  For a 4-bit
// two's-complement value, (t & 0xF) ^ 8 == t + 8, so the conversion is an
// xor of every byte with 0x88: one read and one write of the packed bytes,
// in place or into another buffer.  The per-row scale of that format is an
// fp16 [..., 1] array, usable as-is as a scale plane with group size D.
#include "kv_common.h"

namespace knlp {

// One dword per lane over a [rows, row_bytes] byte matrix (row_bytes % 4 == 0,
// 4-byte aligned rows): dst = src ^ 0x88888888.
__global__ __launch_bounds__(256) void twos_to_offset_kernel(const uint8_t* __restrict__ src,
                                                             int64_t src_stride,
                                                             uint8_t* __restrict__ dst,
                                                             int64_t dst_stride, int64_t rows,
                                                             int64_t row_dwords) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * row_dwords) return;
  const int64_t r = i / row_dwords;
  const int64_t c = i % row_dwords;
  const uint32_t w = reinterpret_cast<const uint32_t*>(src + r * src_stride)[c];
  reinterpret_cast<uint32_t*>(dst + r * dst_stride)[c] = w ^ 0x88888888u;
}

int launch_twos_to_offset(const void* src, int64_t src_stride, void* dst, int64_t dst_stride,
                          int64_t rows, int64_t row_bytes, hipStream_t stream) {
  const int64_t items = rows * (row_bytes / 4);
  const int64_t blocks = (items + 255) / 256;
  if (blocks == 0) return KNLP_OK;
  if (blocks > 0x7FFFFFFF) return KNLP_ERR_SHAPE;
  hipLaunchKernelGGL(twos_to_offset_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     stream, static_cast<const uint8_t*>(src), src_stride,
                     static_cast<uint8_t*>(dst), dst_stride, rows, row_bytes / 4);
  return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
}

}  // namespace knlp
