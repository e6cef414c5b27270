// Sustained-read probe: how fast this GPU streams a buffer of a given size
// from HBM when nothing else is in the way.  It gives the decode kernel's
// bandwidth a measured ceiling next to the data-sheet peak (the reference's
// benchmark keeps a STREAM kernel for the same purpose,
// scripts/v35_h100_bench.py:99-139).
//
// Each workgroup reads one contiguous slice of the buffer with 16-byte loads,
// NLOAD loads in flight per lane, and folds the words with xor; a store that
// only fires for one 32-bit value keeps every load live without writing
// anything in practice.  Reads each byte once: algorithmic bytes = traffic.
#include "kv_common.h"

namespace knlp {

using vu4 = unsigned int __attribute__((ext_vector_type(4)));

template <int NLOAD>
__global__ __launch_bounds__(512) void hbm_read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                       int64_t per_block,
                                                       uint32_t* __restrict__ sink) {
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * per_block;
  const int64_t end = min(n16, begin + per_block);
  uint32_t acc = 0;
  const int64_t stride = static_cast<int64_t>(NLOAD) * blockDim.x;
  for (int64_t i = begin + threadIdx.x; i < end; i += stride) {
    uint4 v[NLOAD];
#pragma unroll
    for (int k = 0; k < NLOAD; ++k) {
      const int64_t j = i + static_cast<int64_t>(k) * blockDim.x;
      if (j < end) {
        // non-temporal, like the decode kernel's tile copies: streamed once
        const vu4 w = __builtin_nontemporal_load(reinterpret_cast<const vu4*>(src) + j);
        v[k] = make_uint4(w.x, w.y, w.z, w.w);
      } else {
        v[k] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int k = 0; k < NLOAD; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

int launch_hbm_read_probe(const void* src, int64_t bytes, void* sink, int blocks,
                          hipStream_t stream) {
  const int64_t n16 = bytes / 16;
  const int64_t per_block = (n16 + blocks - 1) / blocks;
  hipLaunchKernelGGL(hbm_read_kernel<8>, dim3(blocks), dim3(512), 0, stream,
                     static_cast<const uint4*>(src), n16, per_block,
                     static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
}

}  // namespace knlp
