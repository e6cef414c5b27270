// Stage 2 (general shapes): split-K decode attention on the vector ALUs.
//
// Replaces the single-pass Triton kernels of the reference
// (_fused_int4_decode_kernel F:656-894, _kint8_vint4_decode_kernel
// F:1318-1493, _kfp16_vint4_decode_kernel F:987-1156, and the INT8-V variants
// F:1652-1793, F:1850-1972).  Differences in structure, not in arithmetic:
//   * one wave per (sequence, kv head, split) serves all G = Hq/Hkv query
//     heads of the GQA group, so every KV byte is read once (the reference
//     runs one program per query head and re-reads KV G times);
//   * the context is cut into splits of split_tokens tokens; each wave writes
//     an unnormalised partial (acc, running max, running sum) that the merge
//     kernel combines (the reference has no split-K);
//   * the per-group scale and zero-point are applied outside the code dot
//     product: q.k = s * (q.n) + z * sum(q) over the group (scale placement of
//     docs/fused-quant/fp8-attention-hardware-notes.md:108-113), and
//     p.v = (p*s).n + p*z for V.
//   * softmax runs in base 2 with softmax_scale*log2(e) folded into q.
// This kernel covers every format pair and G <= 8; the MFMA kernel
// (kv_decode_mfma.hip) takes the shapes it supports.
//
// Lane layout: a token row of D elements is spread over TPT = D/8 lanes, 8
// consecutive elements per lane (4 bytes of INT4, 8 of INT8, 16 of fp16); a
// wave covers TOK = 64/TPT tokens per step.  A lane's 8 elements always lie
// in one scale group (group sizes >= 16).
#include "kv_decode.h"

namespace knlp {

template <int S>
struct RowLoad {
  float x[8];
  float s, z;   // group scale and zero-point (z folds the -8 offset of INT4 sym)
};

// Raw bits of one lane's slice of a row: loaded a step ahead of their use,
// converted by to_row8 when the step computes.
template <int S>
struct RawRow;
template <>
struct RawRow<kInt4> {
  uint32_t w;
  uint16_t s, z;
};
template <>
struct RawRow<kInt8> {
  uint2 w;
  uint16_t s, z;
};
template <>
struct RawRow<kFp16> {
  uint4 w;
};

template <int S>
__device__ __forceinline__ void load_raw(const knlp_kv_plane& P, int64_t page, int64_t off,
                                         int head, int c, int grp, RawRow<S>& r) {
  const int64_t base = page * P.stride_block + off * P.stride_page + head * P.stride_head;
  if constexpr (S == kInt4) {
    r.w = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(P.data) + base + 4 * c);
  } else if constexpr (S == kInt8) {
    r.w = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(P.data) + base + 8 * c);
  } else {
    r.w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(P.data) + base + 8 * c);
  }
  if constexpr (S != kFp16) {
    r.s = (static_cast<const uint16_t*>(P.scales) + page * P.s_stride_block +
           off * P.s_stride_page + head * P.s_stride_head)[grp];
    r.z = P.format == KNLP_KV_INT4_ASYM
              ? (static_cast<const uint16_t*>(P.zeros) + page * P.z_stride_block +
                 off * P.z_stride_page + head * P.z_stride_head)[grp]
              : static_cast<uint16_t>(0);
  }
}

// Raw bits -> the lane's 8 elements as exact floats, and the group's scale and
// zero-point (the symmetric INT4 zero is the -8 offset times the scale).
template <int S>
__device__ __forceinline__ void to_row8(const knlp_kv_plane& P, const RawRow<S>& w,
                                        RowLoad<S>& r) {
  if constexpr (S == kInt4) {
#pragma unroll
    for (int e = 0; e < 8; ++e) r.x[e] = static_cast<float>((w.w >> (4 * e)) & 0xFu);
  } else if constexpr (S == kInt8) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r.x[e] = static_cast<float>(static_cast<int8_t>((w.w.x >> (8 * e)) & 0xFFu));
      r.x[4 + e] = static_cast<float>(static_cast<int8_t>((w.w.y >> (8 * e)) & 0xFFu));
    }
  } else {
    const uint32_t ws[4] = {w.w.x, w.w.y, w.w.z, w.w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r.x[2 * e] = half_bits_to_float(static_cast<uint16_t>(ws[e] & 0xFFFFu));
      r.x[2 * e + 1] = half_bits_to_float(static_cast<uint16_t>(ws[e] >> 16));
    }
  }
  if constexpr (S != kFp16) {
    r.s = half_bits_to_float(w.s);
    r.z = P.format == KNLP_KV_INT4_ASYM ? half_bits_to_float(w.z)
        : P.format == KNLP_KV_INT4_SYM ? -8.0f * r.s : 0.0f;
  } else {
    r.s = 1.0f;
    r.z = 0.0f;
  }
}

template <int D, int GB, int KS, int VS>
__global__ __launch_bounds__(512) void decode_valu_kernel(DecodeArgs a) {
  constexpr int TPT = D / 8;
  constexpr int TOK = kWave / TPT;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int hpb = blockDim.x / kWave;
  const int split = blockIdx.x;
  const int seq = blockIdx.y;
  const int kvh = blockIdx.z * hpb + wave;
  if (kvh >= a.num_kv_heads) return;
  const int seq_len = min(a.seq_lens[seq], a.max_context);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= seq_len) return;                   // split past the end: no partial
  const int t_end = min(seq_len, t_begin + a.split_tokens);
  // the token being decoded, when the caller fused its append into this launch
  decode_append<D>(a, seq, kvh, split, seq_len, lane);
  const int tk = lane / TPT;
  const int c = lane % TPT;
  const int G = a.group;

  float q[GB][8];
  float qs[GB];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    qs[g] = 0.0f;
    const int h = kvh * G + g;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = 0.0f;
      if (g < G) {
        const uint16_t b = a.q[seq * a.q_stride_seq + h * a.q_stride_head + 8 * c + e];
        v = (a.q_bf16 ? bf16_bits_to_float(b) : half_bits_to_float(b)) * a.scale_log2;
      }
      q[g][e] = v;
      qs[g] += v;
    }
  }
  const int kgrp = KS == kFp16 ? 0 : (8 * c) / a.kp.group_size;
  const int vgrp = VS == kFp16 ? 0 : (8 * c) / a.vp.group_size;

  float m[GB], l[GB], zacc[GB], acc[GB][8];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
    zacc[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
  }
  const int32_t* bt = a.block_table + seq * a.bt_stride;
  const int bs = a.block_size;

  // Software pipeline over token steps: the block-table entry of step i + 2
  // and the K / V rows of step i + 1 are loaded while step i computes.  The
  // pure fp16 pair keeps the unpipelined order, which measured faster for it
  // (its rows are 4x larger: the second register set costs occupancy).
  constexpr bool PIPE = !(KS == kFp16 && VS == kFp16);
  auto token_of = [&](int t0) {
    const int t = t0 + tk;
    return t < t_end ? t : t_begin;
  };
  int32_t page1 = 0, page2 = 0;                      // pages of steps i + 1, i + 2
  RawRow<KS> kraw, kraw1;
  RawRow<VS> vraw, vraw1;
  {
    const int tt = token_of(t_begin);
    const int64_t page = bt[tt / bs];
    load_raw<KS>(a.kp, page, tt % bs, kvh, c, kgrp, kraw);
    load_raw<VS>(a.vp, page, tt % bs, kvh, c, vgrp, vraw);
    if (PIPE && t_begin + TOK < t_end) page1 = bt[token_of(t_begin + TOK) / bs];
  }
  for (int t0 = t_begin; t0 < t_end; t0 += TOK) {
    const bool valid = t0 + tk < t_end;
    if constexpr (PIPE) {
      if (t0 + 2 * TOK < t_end) page2 = bt[token_of(t0 + 2 * TOK) / bs];
      if (t0 + TOK < t_end) {
        const int tt = token_of(t0 + TOK);
        load_raw<KS>(a.kp, page1, tt % bs, kvh, c, kgrp, kraw1);
        load_raw<VS>(a.vp, page1, tt % bs, kvh, c, vgrp, vraw1);
      }
    } else if (t0 != t_begin) {
      const int tt = token_of(t0);
      const int64_t page = bt[tt / bs];
      load_raw<KS>(a.kp, page, tt % bs, kvh, c, kgrp, kraw);
      load_raw<VS>(a.vp, page, tt % bs, kvh, c, vgrp, vraw);
    }

    RowLoad<KS> kr;
    to_row8<KS>(a.kp, kraw, kr);
    float part[GB];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s = fmaf(q[g][e], kr.x[e], s);
      part[g] = KS == kFp16 ? s : fmaf(kr.s, s, kr.z * qs[g]);
    }
#pragma unroll
    for (int o = TPT / 2; o >= 1; o >>= 1) {
#pragma unroll
      for (int g = 0; g < GB; ++g) part[g] += shfl_xor(part[g], o);
    }
    float mt[GB];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      part[g] = valid ? part[g] : -INFINITY;
      mt[g] = part[g];
    }
#pragma unroll
    for (int o = TPT; o < kWave; o <<= 1) {
#pragma unroll
      for (int g = 0; g < GB; ++g) mt[g] = fmaxf(mt[g], shfl_xor(mt[g], o));
    }
    bool grow = false;
#pragma unroll
    for (int g = 0; g < GB; ++g) grow |= mt[g] > m[g];
    if (grow) {                                      // wave-uniform
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        const float mn = fmaxf(m[g], mt[g]);
        const float alpha = exp2f(m[g] - mn);
        m[g] = mn;
        l[g] *= alpha;
        zacc[g] *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
      }
    }
    RowLoad<VS> vr;
    to_row8<VS>(a.vp, vraw, vr);
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      const float p = exp2f(part[g] - m[g]);         // invalid token: exp2(-inf) = 0
      if (c == 0) l[g] += p;
      const float pv = VS == kFp16 ? p : p * vr.s;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pv, vr.x[e], acc[g][e]);
      zacc[g] = fmaf(p, vr.z, zacc[g]);
    }
    if constexpr (PIPE) {
      kraw = kraw1;
      vraw = vraw1;
      page1 = page2;
    }
  }

#pragma unroll
  for (int o = TPT; o < kWave; o <<= 1) {
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      l[g] += shfl_xor(l[g], o);
      zacc[g] += shfl_xor(zacc[g], o);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] += shfl_xor(acc[g][e], o);
    }
  }
  if (tk == 0) {
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      if (g >= G) break;
      const int h = kvh * G + g;
      const int64_t row = (static_cast<int64_t>(seq) * a.num_q_heads + h) * a.num_splits + split;
      float4* dst = reinterpret_cast<float4*>(a.part_o + row * D + 8 * c);
      dst[0] = make_float4(acc[g][0] + zacc[g], acc[g][1] + zacc[g], acc[g][2] + zacc[g],
                           acc[g][3] + zacc[g]);
      dst[1] = make_float4(acc[g][4] + zacc[g], acc[g][5] + zacc[g], acc[g][6] + zacc[g],
                           acc[g][7] + zacc[g]);
      if (c == 0) {
        a.part_ml[2 * row] = m[g];
        a.part_ml[2 * row + 1] = l[g];
      }
    }
  }
}

template <int D, int GB>
static int launch_formats(const DecodeArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  const int ks = storage_of(a.kp.format), vs = storage_of(a.vp.format);
#define KNLP_FMT(K, V)                                                                   \
  if (ks == K && vs == V) {                                                              \
    hipLaunchKernelGGL((decode_valu_kernel<D, GB, K, V>), grid, block, 0, stream, a);    \
    return KNLP_OK;                                                                      \
  }
  KNLP_FMT(kInt4, kInt4)
  KNLP_FMT(kInt8, kInt4)
  KNLP_FMT(kFp16, kInt4)
  KNLP_FMT(kInt8, kInt8)
  KNLP_FMT(kFp16, kInt8)
  KNLP_FMT(kFp16, kFp16)
  KNLP_FMT(kInt4, kInt8)
  KNLP_FMT(kInt4, kFp16)
  KNLP_FMT(kInt8, kFp16)
#undef KNLP_FMT
  return KNLP_ERR_DTYPE;
}

template <int D>
static int launch_gb(const DecodeArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  if (a.group <= 1) return launch_formats<D, 1>(a, grid, block, stream);
  if (a.group <= 2) return launch_formats<D, 2>(a, grid, block, stream);
  if (a.group <= 4) return launch_formats<D, 4>(a, grid, block, stream);
  if (a.group <= 8) return launch_formats<D, 8>(a, grid, block, stream);
  return KNLP_ERR_SHAPE;
}

int launch_decode_valu(const DecodeArgs& a, int head_size, int heads_per_block,
                       hipStream_t stream) {
  const dim3 grid(a.num_splits, a.num_seqs,
                  (a.num_kv_heads + heads_per_block - 1) / heads_per_block);
  const dim3 block(kWave * heads_per_block);
  int st;
  switch (head_size) {
    case 32: st = launch_gb<32>(a, grid, block, stream); break;
    case 64: st = launch_gb<64>(a, grid, block, stream); break;
    case 128: st = launch_gb<128>(a, grid, block, stream); break;
    case 256: st = launch_gb<256>(a, grid, block, stream); break;
    default: return KNLP_ERR_SHAPE;
  }
  if (st != KNLP_OK) return st;
  return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
}

}  // namespace knlp
