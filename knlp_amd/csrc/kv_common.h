// Device helpers shared by the append, decode and merge kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/knlp_int4kv.h"

namespace knlp {

constexpr int kWave = 64;

// Round half away from zero with the +-0.5 added in fp32, exactly as the
// reference's _triton_round (F:198-202): floor(t + 0.5) for t >= 0, else
// ceil(t - 0.5).  t = 0.49999997f therefore rounds to 1.
__device__ __forceinline__ float round_half_away(float t) {
#pragma clang fp contract(off)
  return t >= 0.0f ? floorf(t + 0.5f) : ceilf(t - 0.5f);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  // v_cvt_f16_f32: round to nearest even, subnormals kept.
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  // round to nearest even (inputs here are finite fp16 values)
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(r >> 16);
}

// Load one element of a fp16 / bf16 tensor as fp32 (exact widening).
__device__ __forceinline__ float load_src(const uint16_t* p, bool is_bf16) {
  uint16_t b = *p;
  return is_bf16 ? bf16_bits_to_float(b) : half_bits_to_float(b);
}

// Cross-lane xor exchange inside a wavefront (ds_swizzle/bpermute under the
// hood); only used where the lane pattern is not a DPP row pattern.
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}
__device__ __forceinline__ int shfl_xor(int v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// Row of a slot mapping (int32 or int64 entries).
__device__ __forceinline__ int64_t load_slot(const void* slots, int is64, int64_t i) {
  return is64 ? static_cast<const int64_t*>(slots)[i]
              : static_cast<int64_t>(static_cast<const int32_t*>(slots)[i]);
}

}  // namespace knlp
