// Stage 2 (matrix-core path): split-K decode attention over packed INT4 K/V
// for gfx950, used for the GQA shapes of the benchmark configurations.
//
// Same contract as decode_valu_kernel (kv_decode_valu.hip): one wave per
// (sequence, kv head, split), unnormalised partials (acc, max, sum) in the
// workspace, softmax in base 2.  Replaces the reference's
// _fused_int4_decode_kernel (F:656-894) for these shapes.
//
// Work per wave and 32-token tile (two 16-token sub-tiles); lane l has
// col = l % 16, blk = l / 16.  "Slot (blk, e)" is element e of lane block blk
// of an MFMA A/B operand: the contraction index k of that element.  Slots are
// assigned freely, as long as A and B agree.
//
// QK  v_mfma_f32_16x16x32_f16.  Rows r = g*NG + kg are (q head g, K scale
//     group kg) pairs, where NG = D / group_size.  Columns are the 16 tokens.
//     A = q masked to group kg (built once per wave).  B = the K nibbles of
//     the token, as exact fp16 16 + n.  The lane's 16-byte load (D = 128)
//     holds 32 nibbles; dword c goes to chunk c.  The accumulator starts at
//     -16 * sum(q over the group), which cancels the bias.  The output lane
//     (token col, rows 4blk..4blk+3) then holds sum(q.n) per group, and the
//     score is  sum_kg s[t,kg] * S + z[t,kg] * sum(q)  in fp32.  This is the
//     scale placement of docs/fused-quant/fp8-attention-hardware-notes.md:108-113.
// PV  The V scale depends on the token, which is the contraction index, so
//     it goes into the probabilities: P'[(g,vg), t] = p[g,t] * s_v[t,vg], split
//     into fp16 hi + lo (about 22 significant bits).  B = V nibbles as 16 + n;
//     the bias and the zero-point fold into a per-row term
//     sum_t p * (z - 16 s), accumulated in fp32.  Output rows are (g, vg)
//     pairs and columns are head_dim elements; a column's value is kept only
//     in the row whose vg is the column's group.
// Both operands of PV need "lane = row/column, registers = tokens", but
// they arrive as "lane = token".  The transposes run on the matrix cores
// instead of through LDS:
//   * V: v_mfma_i32_16x16x32_i8 with A = the nibbles as bytes, B = 64 * a
//     selection matrix, C = 0x4C00.  Each int32 output is then the fp16 bit
//     pattern of 16 + n for one (token, column).
//   * P': v_mfma_f32_16x16x16_f16 against the identity.
// Output layout assumed for 16x16 MFMAs (all shapes used here): lane l holds
// D[4*(l/16) + i][l % 16] in register i.
//
// Online softmax: a row's running max is raised only when a tile's max
// exceeds it by more than 2 (log2 units).  Then p <= 4 and |P'| <= 4 * s_v,
// which stays inside fp16 range for any finite fp16 K/V input (s_v < 9400).
#include "kv_decode.h"

namespace knlp {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr float kRescaleLog2 = 2.0f;
// slot e of a converted K dword -> nibble index within the dword
__device__ constexpr int kNibK[8] = {0, 4, 1, 5, 2, 6, 3, 7};

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Reductions over the 16 lanes of a DPP row (lanes with the same blk).
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp<0xB1>(x));    // quad_perm [1,0,3,2]
  x = fmaxf(x, dpp<0x4E>(x));    // quad_perm [2,3,0,1]
  x = fmaxf(x, dpp<0x141>(x));   // row_half_mirror
  x = fmaxf(x, dpp<0x140>(x));   // row_mirror
  return x;
}
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  x += dpp<0x140>(x);
  return x;
}

// 8 nibbles (one dword, element 2i in the low nibble of byte i) -> 8 exact
// fp16 values 16 + n in slot order kNibK.  fp16 0x4C00 is 16.0; the nibble
// goes to mantissa bits 6..9.
__device__ __forceinline__ h8 nibbles_to_h8_b16(uint32_t w) {
  const uint32_t m = 0x03C003C0u, c = 0x4C004C00u;
  u4 o;
  o[0] = ((w << 6) & m) | c;   // n0, n4
  o[1] = ((w << 2) & m) | c;   // n1, n5
  o[2] = ((w >> 2) & m) | c;   // n2, n6
  o[3] = ((w >> 6) & m) | c;   // n3, n7
  return __builtin_bit_cast(h8, o);
}

// nibbles of one dword as 8 int8 slots: [n0 n2 n4 n6 | n1 n3 n5 n7]
__device__ __forceinline__ long nibbles_to_i8x8(uint32_t w) {
  const uint64_t lo = w & 0x0F0F0F0Fu;
  const uint64_t hi = (w >> 4) & 0x0F0F0F0Fu;
  return static_cast<long>(lo | (hi << 32));
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

template <int NG>
struct Halves;   // NG consecutive fp16 values of one (block, page, head) row
template <>
struct Halves<4> {
  uint2 v;
  __device__ float get(int i) const { return h2f((i < 2 ? v.x : v.y) >> (16 * (i & 1))); }
  __device__ void load(const uint16_t* p) { v = *reinterpret_cast<const uint2*>(p); }
};
template <>
struct Halves<2> {
  uint32_t v;
  __device__ float get(int i) const { return h2f(v >> (16 * i)); }
  __device__ void load(const uint16_t* p) { v = *reinterpret_cast<const uint32_t*>(p); }
};
template <>
struct Halves<1> {
  uint32_t v;
  __device__ float get(int) const { return h2f(v); }
  __device__ void load(const uint16_t* p) { v = *p; }
};

template <int NCH>
struct Codes;    // NCH dwords of packed nibbles (D/8 bytes) per lane and token
template <>
struct Codes<4> {
  uint4 v;
  __device__ uint32_t dw(int c) const { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }
  __device__ void load(const uint8_t* p) { v = *reinterpret_cast<const uint4*>(p); }
};
template <>
struct Codes<2> {
  uint2 v;
  __device__ uint32_t dw(int c) const { return c == 0 ? v.x : v.y; }
  __device__ void load(const uint8_t* p) { v = *reinterpret_cast<const uint2*>(p); }
};

template <int NCH, int NG>
struct SubTile {
  Codes<NCH> k, v;
  Halves<NG> ks, kz, vs, vz;
  bool valid;    // this lane's token is inside [t_begin, t_end)
};

template <int D, int NG>
__device__ __forceinline__ void load_sub(const DecodeArgs& a, const int32_t* bt, int kvh,
                                         int base, int t_first, int t_end, int col, int blk,
                                         bool kasym, bool vasym, SubTile<D / 32, NG>& st) {
  constexpr int LB = D / 8;      // bytes of codes per lane per token
  // a sub-tile wholly past the end re-reads the split's first page (masked)
  const bool sub_valid = base < t_end;
  const int pbase = sub_valid ? base : t_first;
  const int64_t page = bt[pbase / a.block_size];
  const int64_t off = pbase % a.block_size + col;
  st.valid = sub_valid && (base + col) < t_end;
  const knlp_kv_plane& K = a.kp;
  const knlp_kv_plane& V = a.vp;
  st.k.load(static_cast<const uint8_t*>(K.data) + page * K.stride_block + off * K.stride_page +
            kvh * K.stride_head + LB * blk);
  st.v.load(static_cast<const uint8_t*>(V.data) + page * V.stride_block + off * V.stride_page +
            kvh * V.stride_head + LB * blk);
  st.ks.load(static_cast<const uint16_t*>(K.scales) + page * K.s_stride_block +
             off * K.s_stride_page + kvh * K.s_stride_head);
  st.vs.load(static_cast<const uint16_t*>(V.scales) + page * V.s_stride_block +
             off * V.s_stride_page + kvh * V.s_stride_head);
  if (kasym)
    st.kz.load(static_cast<const uint16_t*>(K.zeros) + page * K.z_stride_block +
               off * K.z_stride_page + kvh * K.z_stride_head);
  if (vasym)
    st.vz.load(static_cast<const uint16_t*>(V.zeros) + page * V.z_stride_block +
               off * V.z_stride_page + kvh * V.z_stride_head);
}

template <int D, int NG>
__global__ __launch_bounds__(512) void decode_mfma_kernel(DecodeArgs a) {
  constexpr int NCH = D / 32;    // K-chunks of 32 along head_dim = dwords per lane
  constexpr int GPL = 4 / NG;    // q heads per lane (rows 4blk..4blk+3)
  const int lane = threadIdx.x & (kWave - 1);
  const int col = lane & 15;
  const int blk = lane >> 4;
  const int wave = threadIdx.x / kWave;
  const int hpb = blockDim.x / kWave;
  const int split = blockIdx.x;
  const int seq = blockIdx.y;
  const int kvh = blockIdx.z * hpb + wave;
  if (kvh >= a.num_kv_heads) return;
  const int seq_len = min(a.seq_lens[seq], a.max_context);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= seq_len) return;
  const int t_end = min(seq_len, t_begin + a.split_tokens);
  const int G = a.group;
  const int gs = a.kp.group_size;
  const int rows = G * NG;
  const bool kasym = a.kp.format == KNLP_KV_INT4_ASYM;
  const bool vasym = a.vp.format == KNLP_KV_INT4_ASYM;

  // ---- masked q: A operands of QK; row r = col ------------------------------
  h8 aq[NCH];
  float qpart = 0.0f;
  {
    const int r = col;
    const bool rv = r < rows;
    const int g = rv ? r / NG : 0;
    const int kg = r % NG;
    const uint16_t* qrow = a.q + seq * a.q_stride_seq + (kvh * G + g) * a.q_stride_head;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = (D / 4) * blk + 8 * c + kNibK[e];
        _Float16 v = 0;
        if (rv && d / gs == kg) v = __builtin_bit_cast(_Float16, qrow[d]);
        aq[c][e] = v;
        qpart += static_cast<float>(v);
      }
    }
  }
  // sum of q over row r's group, then spread so lane (t, blk) has rows 4blk+i
  qpart += __shfl_xor(qpart, 16, kWave);
  qpart += __shfl_xor(qpart, 32, kWave);
  float qsum[4];
  f4 cinit;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qsum[i] = __shfl(qpart, 4 * blk + i, kWave);
    cinit[i] = -16.0f * qsum[i];
  }
  // identity (P' transpose) and 64 * selection (V transpose) operands
  h4 eye;
#pragma unroll
  for (int e = 0; e < 4; ++e) eye[e] = (blk == col / 4 && e == col % 4) ? 1.0f : 0.0f;
  long vsel[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    vsel[h] = blk == col / 4 ? static_cast<long>(64ull << (8 * (4 * h + col % 4))) : 0l;
  const i4 vinit = {0x4C00, 0x4C00, 0x4C00, 0x4C00};

  f4 acc[NCH][2];
#pragma unroll
  for (int c = 0; c < NCH; ++c) acc[c][0] = acc[c][1] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run[GPL], lsum[GPL], zacc[4];
#pragma unroll
  for (int i = 0; i < GPL; ++i) {
    m_run[i] = -INFINITY;
    lsum[i] = 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) zacc[e] = 0.0f;

  const int32_t* bt = a.block_table + seq * a.bt_stride;
  const float sl2 = a.scale_log2;

  SubTile<NCH, NG> cur[2], nxt[2];
  load_sub<D, NG>(a, bt, kvh, t_begin, t_begin, t_end, col, blk, kasym, vasym, cur[0]);
  load_sub<D, NG>(a, bt, kvh, t_begin + 16, t_begin, t_end, col, blk, kasym, vasym, cur[1]);

  for (int t0 = t_begin; t0 < t_end; t0 += 32) {
    const bool more = t0 + 32 < t_end;
    if (more) {
      load_sub<D, NG>(a, bt, kvh, t0 + 32, t_begin, t_end, col, blk, kasym, vasym, nxt[0]);
      load_sub<D, NG>(a, bt, kvh, t0 + 48, t_begin, t_end, col, blk, kasym, vasym, nxt[1]);
    }

    // ---- scores ---------------------------------------------------------------
    float score[2][GPL];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      f4 S = cinit;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        S = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[c], nibbles_to_h8_b16(cur[x].k.dw(c)), S,
                                                   0, 0, 0);
#pragma unroll
      for (int gi = 0; gi < GPL; ++gi) {
        float sc = 0.0f;
#pragma unroll
        for (int kg = 0; kg < NG; ++kg) {
          const int i = gi * NG + kg;
          const float s = cur[x].ks.get(kg);
          const float z = kasym ? cur[x].kz.get(kg) : -8.0f * s;
          sc = fmaf(s, S[i], fmaf(z, qsum[i], sc));
        }
        score[x][gi] = cur[x].valid ? sc * sl2 : -INFINITY;
      }
    }

    // ---- online softmax (lazy max) -------------------------------------------
    float alpha[GPL];
    bool need = false;
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) {
      const float tmax = row_max16(fmaxf(score[0][gi], score[1][gi]));
      const bool up = tmax > m_run[gi] + kRescaleLog2;
      alpha[gi] = up ? exp2f(m_run[gi] - tmax) : 1.0f;
      m_run[gi] = up ? tmax : m_run[gi];
      need |= up;
    }
    if (__any(need)) {
#pragma unroll
      for (int gi = 0; gi < GPL; ++gi) lsum[gi] *= alpha[gi];
#pragma unroll
      for (int e = 0; e < 4; ++e) zacc[e] *= alpha[e / NG];
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[c][h][i] *= alpha[i / NG];
    }

    // ---- P' = p * s_v (hi + lo), zero-point term, transposes -----------------
    h8 ahi, alo;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      float p[GPL];
#pragma unroll
      for (int gi = 0; gi < GPL; ++gi) {
        p[gi] = exp2f(score[x][gi] - m_run[gi]);
        lsum[gi] += p[gi];
      }
      h4 xhi, xlo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int vg = e % NG;
        const float sv = cur[x].vs.get(vg);
        const float zv = vasym ? cur[x].vz.get(vg) : -8.0f * sv;
        const float pe = p[e / NG];
        const float P = cur[x].valid ? pe * sv : 0.0f;
        const _Float16 hi = static_cast<_Float16>(P);
        xhi[e] = hi;
        xlo[e] = static_cast<_Float16>(P - static_cast<float>(hi));
        zacc[e] = cur[x].valid ? fmaf(pe, fmaf(-16.0f, sv, zv), zacc[e]) : zacc[e];
      }
      const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
      const f4 thi = __builtin_amdgcn_mfma_f32_16x16x16f16(xhi, eye, zero4, 0, 0, 0);
      const f4 tlo = __builtin_amdgcn_mfma_f32_16x16x16f16(xlo, eye, zero4, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ahi[4 * x + r] = static_cast<_Float16>(thi[r]);
        alo[4 * x + r] = static_cast<_Float16>(tlo[r]);
      }
    }

    // ---- V transposes and PV ---------------------------------------------------
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const long va = nibbles_to_i8x8(cur[0].v.dw(c));
      const long vb = nibbles_to_i8x8(cur[1].v.dw(c));
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const i4 ta = __builtin_amdgcn_mfma_i32_16x16x32_i8(va, vsel[h], vinit, 0, 0, 0);
        const i4 tb = __builtin_amdgcn_mfma_i32_16x16x32_i8(vb, vsel[h], vinit, 0, 0, 0);
        u4 bw;
        bw[0] = static_cast<uint32_t>(ta[0]) | (static_cast<uint32_t>(ta[1]) << 16);
        bw[1] = static_cast<uint32_t>(ta[2]) | (static_cast<uint32_t>(ta[3]) << 16);
        bw[2] = static_cast<uint32_t>(tb[0]) | (static_cast<uint32_t>(tb[1]) << 16);
        bw[3] = static_cast<uint32_t>(tb[2]) | (static_cast<uint32_t>(tb[3]) << 16);
        const h8 bv = __builtin_bit_cast(h8, bw);
        acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bv, acc[c][h], 0, 0, 0);
        acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bv, acc[c][h], 0, 0, 0);
      }
    }
    if (more) {
      cur[0] = nxt[0];
      cur[1] = nxt[1];
    }
  }

  // ---- reduce over tokens and write the partial ---------------------------------
#pragma unroll
  for (int gi = 0; gi < GPL; ++gi) lsum[gi] = row_sum16(lsum[gi]);
#pragma unroll
  for (int e = 0; e < 4; ++e) zacc[e] = row_sum16(zacc[e]);
  const int64_t row0 = static_cast<int64_t>(seq) * a.num_q_heads + kvh * G;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int d = (D / 4) * (col / 4) + 8 * c + 2 * (col % 4) + h;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * blk + i;
        const int g = r / NG;
        if (g < G && d / gs == r % NG) {
          const int64_t row = (row0 + g) * a.num_splits + split;
          a.part_o[row * D + d] = acc[c][h][i] + zacc[i];
        }
      }
    }
  }
  if (col == 0) {
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) {
      const int g = (4 * blk) / NG + gi;
      if (g < G) {
        const int64_t row = (row0 + g) * a.num_splits + split;
        a.part_ml[2 * row] = m_run[gi];
        a.part_ml[2 * row + 1] = lsum[gi];
      }
    }
  }
}

int heads_per_block_mfma(int num_kv_heads) {
  for (int h = 8; h >= 1; h >>= 1)
    if (num_kv_heads % h == 0) return h;
  return 1;
}

}  // namespace

bool mfma_supported(int group, int head_size, int k_format, int k_gs, int v_format, int v_gs,
                    int q_bf16) {
  const bool int4 = (k_format == KNLP_KV_INT4_SYM || k_format == KNLP_KV_INT4_ASYM) &&
                    (v_format == KNLP_KV_INT4_SYM || v_format == KNLP_KV_INT4_ASYM);
  if (!int4 || q_bf16 || k_gs != v_gs || k_gs <= 0) return false;
  if (head_size != 64 && head_size != 128) return false;
  const int ng = head_size / k_gs;
  if (ng != 1 && ng != 2 && ng != 4) return false;
  return group >= 1 && group * ng <= 16;
}

int launch_decode_mfma(const DecodeArgs& a, int head_size, hipStream_t stream) {
  const int hpb = heads_per_block_mfma(a.num_kv_heads);
  const dim3 grid(a.num_splits, a.num_seqs, a.num_kv_heads / hpb);
  const dim3 block(kWave * hpb);
  const int ng = head_size / a.kp.group_size;
#define KNLP_MFMA(D, NG)                                                               \
  if (head_size == D && ng == NG) {                                                    \
    hipLaunchKernelGGL((decode_mfma_kernel<D, NG>), grid, block, 0, stream, a);        \
    return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;                \
  }
  KNLP_MFMA(128, 4)
  KNLP_MFMA(128, 2)
  KNLP_MFMA(128, 1)
  KNLP_MFMA(64, 4)
  KNLP_MFMA(64, 2)
  KNLP_MFMA(64, 1)
#undef KNLP_MFMA
  return KNLP_ERR_SHAPE;
}

}  // namespace knlp
