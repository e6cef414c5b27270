// Row quantisers shared by the append kernel and the decode kernels' fused
// append (gfx950).  One (token, head) row of D elements is handled by D/2
// consecutive lanes, two elements per lane; a scale group of GS elements
// spans GS/2 aligned lanes and its min/max/sum are xor-butterfly reductions
// over those lanes.  The butterfly order is also the fixed summation order of
// the symmetric trimmed mean (element i adds element i + GS/2, then + GS/4,
// ...), which the CPU oracle restates.
//
// All quantisation arithmetic is IEEE fp32 without contraction: correctly
// rounded subtraction and division, floor/ceil rounding of F:198-202, and
// round-to-nearest-even fp32 -> fp16 for the stored scale / zero-point.  The
// codes are computed from the fp32 scale; the fp16 scale is what is stored.
// F = fused-quant/fused_int4.v0.1.0.py.
#pragma once

#include "kv_common.h"

namespace knlp {

struct RowDst {
  uint8_t* codes;       // start of this (block, offset, head) row of codes
  uint16_t* scales;     // start of its scale row
  uint16_t* zeros;      // start of its zero-point row (asymmetric only)
};

__device__ __forceinline__ RowDst row_dst(const knlp_kv_plane& P, int64_t blk, int64_t off,
                                          int head) {
  RowDst r;
  const int64_t eb = P.format == KNLP_KV_FP16 ? 2 : 1;   // strides are in elements
  r.codes = static_cast<uint8_t*>(P.data) +
            eb * (blk * P.stride_block + off * P.stride_page + head * P.stride_head);
  r.scales = static_cast<uint16_t*>(P.scales) + blk * P.s_stride_block +
             off * P.s_stride_page + head * P.s_stride_head;
  r.zeros = static_cast<uint16_t*>(P.zeros) + blk * P.z_stride_block + off * P.z_stride_page +
            head * P.z_stride_head;
  return r;
}

// One group of GS elements; this lane holds elements d0 = 2*lane, d0 + 1 of
// the row (x0, x1).  Lanes of one group are GS/2 aligned consecutive lanes.
template <int GS>
__device__ __forceinline__ void quant_int4_asym(float x0, float x1, int lane, const RowDst& r) {
#pragma clang fp contract(off)
  float mn = fminf(x0, x1), mx = fmaxf(x0, x1);
#pragma unroll
  for (int o = GS / 4; o >= 1; o >>= 1) {
    mn = fminf(mn, shfl_xor(mn, o));
    mx = fmaxf(mx, shfl_xor(mx, o));
  }
  const float rng = fmaxf(mx - mn, 1e-8f);          // F:314
  const float scale = rng / 15.0f;                   // F:315
  const float q0 = fmaxf(fminf(round_half_away((x0 - mn) / scale), 15.0f), 0.0f);
  const float q1 = fmaxf(fminf(round_half_away((x1 - mn) / scale), 15.0f), 0.0f);
  r.codes[lane] = static_cast<uint8_t>(static_cast<uint32_t>(q0) |
                                       (static_cast<uint32_t>(q1) << 4));
  const int d0 = 2 * lane;
  if ((d0 % GS) == 0) {
    r.scales[d0 / GS] = float_to_half_bits(scale);
    r.zeros[d0 / GS] = float_to_half_bits(mn);
  }
}

template <int GS>
__device__ __forceinline__ void quant_int4_sym(float x0, float x1, int lane, float clip_ratio,
                                               const RowDst& r) {
#pragma clang fp contract(off)
  const float a0 = fabsf(x0), a1 = fabsf(x1);
  float amax = fmaxf(a0, a1);
#pragma unroll
  for (int o = GS / 4; o >= 1; o >>= 1) amax = fmaxf(amax, shfl_xor(amax, o));
  amax = fmaxf(amax, 1e-8f);                         // F:336
  if (clip_ratio > 0.0f) {                           // F:342-347
    float b0 = a0 < amax ? a0 : 0.0f;
    float b1 = a1 < amax ? a1 : 0.0f;
    int c = static_cast<int>(a0 < amax) + static_cast<int>(a1 < amax);
#pragma unroll
    for (int o = GS / 4; o >= 1; o >>= 1) {
      b0 = b0 + shfl_xor(b0, o);
      b1 = b1 + shfl_xor(b1, o);
      c += shfl_xor(c, o);
    }
    const float sum = b0 + b1;
    const float cnt = fmaxf(static_cast<float>(c), 1.0f);
    const float tmean = sum / cnt;
    const float clip = tmean * clip_ratio;
    amax = fminf(amax, fmaxf(clip, 1e-8f));
  }
  const float scale = amax / 7.0f;                   // F:348
  const float q0 = fmaxf(fminf(round_half_away(x0 / scale), 7.0f), -8.0f) + 8.0f;
  const float q1 = fmaxf(fminf(round_half_away(x1 / scale), 7.0f), -8.0f) + 8.0f;
  r.codes[lane] = static_cast<uint8_t>(static_cast<uint32_t>(q0) |
                                       (static_cast<uint32_t>(q1) << 4));
  const int d0 = 2 * lane;
  if ((d0 % GS) == 0) r.scales[d0 / GS] = float_to_half_bits(scale);
}

template <int GS>
__device__ __forceinline__ void quant_int8(float x0, float x1, int lane, const RowDst& r) {
#pragma clang fp contract(off)
  float amax = fmaxf(fabsf(x0), fabsf(x1));
#pragma unroll
  for (int o = GS / 4; o >= 1; o >>= 1) amax = fmaxf(amax, shfl_xor(amax, o));
  amax = fmaxf(amax, 1e-8f);                         // F:1276
  const float scale = amax / 127.0f;                 // F:1277
  const float q0 = fmaxf(fminf(round_half_away(x0 / scale), 127.0f), -128.0f);
  const float q1 = fmaxf(fminf(round_half_away(x1 / scale), 127.0f), -128.0f);
  const uint32_t b0 = static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(q0)));
  const uint32_t b1 = static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(q1)));
  reinterpret_cast<uint16_t*>(r.codes)[lane] = static_cast<uint16_t>(b0 | (b1 << 8));
  const int d0 = 2 * lane;
  if ((d0 % GS) == 0) r.scales[d0 / GS] = float_to_half_bits(scale);
}

__device__ __forceinline__ void quant_row(const uint16_t* src, bool bf16, const knlp_kv_plane& P,
                                          int64_t blk, int64_t off, int head, int lane,
                                          float clip_ratio) {
  const RowDst r = row_dst(P, blk, off, head);
  if (P.format == KNLP_KV_FP16) {                    // plain copy (fp16 source only)
    reinterpret_cast<uint32_t*>(r.codes)[lane] = reinterpret_cast<const uint32_t*>(src)[lane];
    return;
  }
  const float x0 = load_src(src + 2 * lane, bf16);
  const float x1 = load_src(src + 2 * lane + 1, bf16);
#define KNLP_QUANT_GS(GS)                                                   \
  case GS:                                                                  \
    if (P.format == KNLP_KV_INT4_ASYM) quant_int4_asym<GS>(x0, x1, lane, r);          \
    else if (P.format == KNLP_KV_INT4_SYM) quant_int4_sym<GS>(x0, x1, lane, clip_ratio, r); \
    else quant_int8<GS>(x0, x1, lane, r);                                   \
    break;
  switch (P.group_size) {
    KNLP_QUANT_GS(16)
    KNLP_QUANT_GS(32)
    KNLP_QUANT_GS(64)
    KNLP_QUANT_GS(128)
    default: break;
  }
#undef KNLP_QUANT_GS
}

}  // namespace knlp
