// Stage 2 (matrix-core path): split-K decode attention over packed INT4 K/V
// for gfx950, used for the GQA shapes of the benchmark configurations.
//
// Same contract as decode_valu_kernel (kv_decode_valu.hip): unnormalised
// partials (acc, max, sum) per (sequence, q head, split) in the workspace,
// softmax in base 2.  Replaces the reference's _fused_int4_decode_kernel
// (F:656-894) for these shapes.  Three kernels share the per-wave arithmetic:
// decode_mfma_kernel (one wave per (sequence, kv head, split), loads straight
// into VGPRs), decode_mfma_coop_kernel (8 waves stage whole pages of 8 kv
// heads through LDS; described further down) and decode_mfma_coop_stream_kernel
// (the same block, one per CU, over equal shares of all rows' tiles).
//
// Work per wave and 32-token tile (two 16-token sub-tiles); lane l has
// col = l % 16, blk = l / 16.  "Slot (blk, e)" is element e of lane block blk
// of an MFMA A/B operand: the contraction index k of that element.  Slots are
// assigned freely, as long as A and B agree.
//
// Code encoding: a nibble n enters the matrix cores as the fp16 whose bit
// pattern is n, the exact subnormal n * 2^-24, so a dword of 8 nibbles
// becomes 8 fp16 operands with one shift and one mask per pair.  The
// matrix cores keep fp16 subnormal inputs, and a product with an fp16 q or P'
// lands far above the fp32 subnormal range, so nothing is lost; the factor
// 2^24 is folded into the softmax scale and the final accumulator.
//
// QK  v_mfma_f32_16x16x32_f16.  Rows r = g*NG + kg are (q head g, K scale
//     group kg) pairs, where NG = D / group_size.  Columns are the 16 tokens.
//     A = q masked to group kg (built once per wave), B = the token's K codes.
//     Symmetric K starts the accumulator at -8 * 2^-24 * sum(q over the
//     group).  The output lane (token col, rows 4blk..4blk+3) then holds
//     2^-24 * sum(q.n) per group, and the score is
//     sum_kg s[t,kg] * S + z[t,kg] * 2^-24 * sum(q)  in fp32.  This is the
//     scale placement of docs/fused-quant/fp8-attention-hardware-notes.md:108-113.
// PV  The V scale depends on the token, which is the contraction index, so
//     it goes into the probabilities: P'[(g,vg), t] = p[g,t] * s_v[t,vg], split
//     into fp16 hi + lo.  B = the V codes; the zero-point (asymmetric) or
//     -8 s (symmetric; -128 s for the biased INT8 codes) folds into a per-row
//     term sum_t p * z, accumulated in fp32.  Output rows are (g, vg) pairs and
//     columns are head_dim elements; a column's value is kept only in the row
//     whose vg is the column's group, and hi and lo take one product each.
//     Group pairs (cooperative kernel, one head set, INT4 V in four groups at
//     D = 128): a lane reads V as two 16-bit halves per token, so that each
//     product's 16 columns lie in groups {0, 1} or {2, 3}; the A operand of
//     a pair has rows (g, group of the pair, hi / lo), and a column sums its
//     hi and lo rows when the partial is written: half the PV products.
//     Precision of P': p carries a per-wave power of two 2^k chosen from the
//     largest V scale seen so far (k lowered, with the accumulators rescaled,
//     when a larger one arrives), so that max_t P' lies near 2^12..2^14 however
//     small the V scales are.  The dominant terms then have a normal fp16 hi
//     and lo, P' keeps about 22 significant bits, and fp16's absolute floor
//     (2^-24) sits 2^-36 or more below the largest V scale.  hi is rounded
//     toward zero by one explicit conversion and lo is the exact product minus
//     that same hi, so the matrix cores see hi + lo = p * s_v to 2^-22 and the
//     symmetric bias term (computed from p * s_v in fp32) cancels against it.
// Both operands of PV need "lane = row/column, registers = tokens", but
// they arrive as "lane = token".  P' is transposed on the matrix cores
// (v_mfma_f32_16x16x16_f16 against the identity).  V is transposed either
// on the matrix cores (per-head kernel: v_mfma_i32_16x16x32_i8 with A = the
// nibbles as bytes and B = a selection matrix, each int32 output then being
// the code of one (token, column)), or for free by reading the staged tile
// from LDS in column order (cooperative kernel, pv_columns).
// Output layout assumed for 16x16 MFMAs (all shapes used here): lane l holds
// D[4*(l/16) + i][l % 16] in register i.
//
// Online softmax: a row's running max is raised only when a tile's max
// exceeds it by more than 2 (log2 units).  Then p <= 4 * 2^k and
// |P'| <= 4 * 2^k * s_v <= 2^14, inside fp16 range for any finite input.

// Matrix-core decode kernels for gfx950: the device code shared by the
// translation units that instantiate them (kv_decode_mfma_perhead.hip,
// kv_decode_mfma_coop.hip, kv_decode_mfma_stream.hip, compiled in parallel)
// and the host dispatch in kv_decode_mfma.hip.
#pragma once
#include <type_traits>

#include "kv_decode.h"

namespace knlp {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// Raw buffer resource over [base, base + 4 GiB): every cache load is
// "scalar descriptor + 32-bit lane byte offset", so the address arithmetic of
// a load is scalar.  Word 3 is the gfx9-family raw-buffer format
// (0x00020000, as composable_kernel's CK_BUFFER_RESOURCE_3RD_DWORD).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(0xFFFFFFFFu), 0x00020000);
}

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

// Masks that pick one nibble per fp16 half of a dword: at bits 0-3 (value n)
// or at bits 4-7 (value 16 n); both stay inside the fp16 mantissa, so the
// half is the exact subnormal n * 2^-24 or 16 n * 2^-24.
constexpr uint32_t kNib1 = 0x000F000Fu;
constexpr uint32_t kNib16 = 0x00F000F0u;

// 8 nibbles (one dword, element 2i in the low nibble of byte i) -> 8 fp16
// values in slot order kNibK: even nibbles as n * 2^-24, odd nibbles as
// 16 n * 2^-24 (slots e with e & 2).  Five VALU ops per dword; the q slots
// that meet the odd nibbles hold q / 16.
__device__ __forceinline__ h8 nibbles_to_h8_sub(uint32_t w) {
  const uint32_t t = w >> 8;
  u4 o;
  o[0] = w & kNib1;     // n0, n4
  o[1] = w & kNib16;    // 16 n1, 16 n5
  o[2] = t & kNib1;     // n2, n6
  o[3] = t & kNib16;    // 16 n3, 16 n7
  return __builtin_bit_cast(h8, o);
}

// slot e of a converted INT8 dword pair -> byte index within the pair
__device__ constexpr int kByteK8[8] = {0, 2, 1, 3, 4, 6, 5, 7};

// 8 int8 codes (two dwords, element i in byte i) -> 8 fp16 values in slot
// order kByteK8 whose bit patterns are the codes biased by 128 (the xor with
// 0x80 flips the sign bit): the exact subnormals (n + 128) * 2^-24, all below
// 2^-14.  Four VALU ops per dword; the bias leaves 128 * sum(q) per row, which
// the accumulator's start value cancels.
__device__ __forceinline__ h8 bytes_to_h8_sub(uint32_t w0, uint32_t w1) {
  constexpr uint32_t m = 0x00FF00FFu;
  const uint32_t a = w0 ^ 0x80808080u, b = w1 ^ 0x80808080u;
  u4 o;
  o[0] = a & m;           // bytes 0, 2
  o[1] = (a >> 8) & m;    // bytes 1, 3
  o[2] = b & m;           // bytes 4, 6
  o[3] = (b >> 8) & m;    // bytes 5, 7
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
  __device__ _Float16 geth(int i) const {
    return __builtin_bit_cast(_Float16,
                              static_cast<uint16_t>((i < 2 ? v.x : v.y) >> (16 * (i & 1))));
  }
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
  }
};
template <>
struct Halves<2> {
  uint32_t v;
  __device__ float get(int i) const { return h2f(v >> (16 * i)); }
  __device__ _Float16 geth(int i) const {
    return __builtin_bit_cast(_Float16, static_cast<uint16_t>(v >> (16 * i)));
  }
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  }
};
template <>
struct Halves<1> {
  uint32_t v;
  __device__ float get(int) const { return h2f(v); }
  __device__ _Float16 geth(int) const { return __builtin_bit_cast(_Float16, static_cast<uint16_t>(v)); }
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
  }
};

template <int NCH>
struct Codes;    // NCH dwords of codes per lane and token
template <>
struct Codes<16> {   // 64 bytes: a quarter of an fp16 K row at D = 128
  uint4 v[4];
  __device__ uint32_t dw(int c) const {
    const uint4& u = v[c >> 2];
    const int i = c & 3;
    return i == 0 ? u.x : i == 1 ? u.y : i == 2 ? u.z : u.w;
  }
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      v[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * k, 0, 0));
  }
};
template <>
struct Codes<8> {
  uint4 v, w;
  __device__ uint32_t dw(int c) const {
    const uint4& u = c < 4 ? v : w;
    const int i = c & 3;
    return i == 0 ? u.x : i == 1 ? u.y : i == 2 ? u.z : u.w;
  }
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0));
  }
};
template <>
struct Codes<4> {
  uint4 v;
  __device__ uint32_t dw(int c) const { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  }
};
template <>
struct Codes<2> {
  uint2 v;
  __device__ uint32_t dw(int c) const { return c == 0 ? v.x : v.y; }
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
  }
};

// fp16 V in the PV B-operand order: r[i] holds the 2 NCH halves of head-dim
// columns 2 NCH col .. 2 NCH col + 2 NCH - 1 (NCH = D / 32 dwords) of token
// 4 blk + i of the sub-tile, so each load of a 16-lane group covers one
// token's head row (2 D bytes).
template <int NCH>
struct RowsH {
  uint32_t r[4][NCH];
  __device__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t stride) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (NCH == 4) {
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + i * stride, 0, 0));
        r[i][0] = v.x; r[i][1] = v.y; r[i][2] = v.z; r[i][3] = v.w;
      } else {
        static_assert(NCH == 2, "fp16 V rows for D = 64 or 128");
        const uint2 v = __builtin_bit_cast(
            uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, off + i * stride, 0, 0));
        r[i][0] = v.x; r[i][1] = v.y;
      }
    }
  }
};

// One 16-token sub-tile in the per-lane layout.  K: KCH code dwords and NGK
// scale halves per row (packed INT4: KCH = NCH, NGK = NG; INT8: KCH = 2 NCH
// and NGK scale groups, 1 for one scale per row; fp16: KCH = 4 NCH, no
// scales); V: VCH code dwords (packed INT4: NCH, INT8: 2 NCH), or VCH = 0 for
// fp16 V rows (RowsH, no scales).
template <int NCH, int NG, int KCH = NCH, int NGK = NG, int VCH = NCH>
struct SubTile {
  using VCodes = typename std::conditional<VCH == 0, RowsH<NCH>, Codes<VCH == 0 ? 4 : VCH>>::type;
  Codes<KCH> k;
  VCodes v;
  Halves<NGK> ks;
  Halves<NG> kz, vs, vz;
};

// Per-wave addressing: uniform bases (this kv head folded in) plus
// loop-invariant per-lane offsets, so every load is "scalar base + vector
// offset" and the per-tile work is one scalar page lookup.
struct Addr {
  const uint8_t* kc;
  const uint8_t* vc;
  const uint16_t* ks;
  const uint16_t* kz;
  const uint16_t* vs;
  const uint16_t* vz;
  int64_t kc_b, kc_p, vc_b, vc_p;       // bytes per block / per page slot
  int64_t ks_b, ks_p, kz_b, kz_p, vs_b, vs_p, vz_b, vz_p;   // halves
  uint32_t lkc, lvc;                    // lane byte offsets of the codes
  uint32_t vrow;                        // fp16 V: bytes from one token row to the next
  uint32_t lks, lkz, lvs, lvz;          // lane byte offsets of scales / zeros
  const int32_t* bt;
  int bs_shift;
};

// Page lookup: lane l of `win` holds block_table[seq, win_first + l]; the
// sub-tile's page is read back with v_readlane into an SGPR, so all address
// arithmetic of a load is scalar.  The window is refilled every 64 pages.
struct PageWindow {
  int win;          // per lane
  int first;        // uniform: block-table index held by lane 0
  int last;         // uniform: last block-table index this split touches
  __device__ __forceinline__ void fill(const int32_t* bt, int lane, int first_idx) {
    first = first_idx;
    const int idx = first_idx + lane;
    win = idx <= last ? bt[idx] : 0;
    // wait here, inside the (rare) refill, so that the compiler does not put
    // a vector-memory wait in front of every lookup; in the cooperative
    // kernel such a wait would also drain the tile copies in flight
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));   // vmcnt(0)
  }
  __device__ __forceinline__ int64_t page(const int32_t* bt, int lane, int idx) {
    if (idx - first >= kWave) fill(bt, lane, idx);      // uniform branch
    return static_cast<int64_t>(__builtin_amdgcn_readlane(win, idx - first));
  }
};

template <int NCH, int NG, bool KASYM, bool VASYM, int KCH = NCH, int VCH = NCH>
__device__ __forceinline__ void load_sub(const Addr& A, PageWindow& P, int lane, int pbase,
                                         SubTile<NCH, NG, KCH, NG, VCH>& st) {
  const int64_t page = P.page(A.bt, lane, pbase >> A.bs_shift);
  const int64_t off0 = pbase & ((1 << A.bs_shift) - 1);
  st.k.load(rsrc_of(A.kc + (page * A.kc_b + off0 * A.kc_p)), A.lkc);
  if constexpr (VCH == 0)         // fp16 V rows, no scales
    st.v.load(rsrc_of(A.vc + (page * A.vc_b + off0 * A.vc_p)), A.lvc, A.vrow);
  else
    st.v.load(rsrc_of(A.vc + (page * A.vc_b + off0 * A.vc_p)), A.lvc);
  if constexpr (KCH != 4 * NCH)   // fp16 K has no scales
    st.ks.load(rsrc_of(A.ks + (page * A.ks_b + off0 * A.ks_p)), A.lks);
  if constexpr (VCH != 0) st.vs.load(rsrc_of(A.vs + (page * A.vs_b + off0 * A.vs_p)), A.lvs);
  if constexpr (KASYM) st.kz.load(rsrc_of(A.kz + (page * A.kz_b + off0 * A.kz_p)), A.lkz);
  if constexpr (VASYM) st.vz.load(rsrc_of(A.vz + (page * A.vz_b + off0 * A.vz_p)), A.lvz);
}

// Running state of one wave.
//
// Tiles normally take the fast path: scores, a per-lane test that no row's
// tile max exceeds its running max by more than the threshold, then
// accumulate.  A tile that would raise a max (or the partial last tile) takes
// the general path: masked scores, raise_max, masked accumulate.  Both paths
// do the same arithmetic on rows whose max does not move, so the result does
// not depend on which path a tile took.
template <int NCH, int NG, bool KASYM, bool VASYM, int KCH = NCH, int NGK = NG, bool V8 = false,
          bool V16 = false>
struct WaveState {
  static constexpr int GPL = 4 / NG;
  static constexpr int NGV = NG;       // V scale groups per token
  // V codes: packed INT4 (one dword of 8 nibble-columns per token and lane in
  // pv_columns) or INT8 (V8: 8 bytes)
  // fp16 V (V16, cooperative kernel): 16 bytes, the 8 halves of columns
  // 8 col .. 8 col + 7 of one token (D = 128)
  using VWord = typename std::conditional<V16, uint4,
                                          typename std::conditional<V8, uint2, uint32_t>::type>::type;
  // INT8 K codes: two dwords per QK chunk, one scale per NG / NGK row groups
  static constexpr bool K8 = KCH == 2 * NCH;
  // fp16 K: four dwords of halves per QK chunk, used as they are (no scale)
  static constexpr bool K16 = KCH == 4 * NCH;
  // fp16 V (V16): no scales or zero-points, values used as they are
  using ST = SubTile<NCH, NG, KCH, NGK, V16 ? 0 : V8 ? 2 * NCH : NCH>;
  static constexpr bool KZ_USED = KASYM;
  static constexpr bool VZ_USED = VASYM;
  // Group-pair PV (cooperative kernel, INT4 V in four groups at D = 128):
  // each product's 16 columns lie in V groups {0, 1} or {2, 3}, and its A
  // rows are (head, group of the pair, hi / lo), so hi and lo of P' share
  // one product (8 PV products per tile instead of 16).
  static constexpr bool PAIRS_OK = !V8 && !V16 && NG == 4 && NCH == 4;
  static_assert(NG % NGK == 0 && (K8 || K16 || NGK == NG),
                "K scale groups nest in the row groups");
  h8 aq[NCH];          // masked q, A operands of QK (row = col)
  float qsum24[4];     // 2^-24 * sum of q over the group of rows 4blk..4blk+3
  f4 cinit;            // QK accumulator start: 0 for asymmetric INT4 K, else -bias * qsum24
                       // (bias 8 for symmetric INT4, 128 for the biased INT8 codes)
  h4 eye;              // identity, B operand of the P' transpose
  long vsel[2];        // selection, B operand of the V transpose
  f4 acc[NCH][2];      // PV accumulators (units of 2^-24), rows (g, vg) x columns d
  float m_run[GPL];    // running max per q head (score units of 2^-24)
  float lsum[GPL];     // per-lane partial softmax sums
  float zacc[4];       // per-lane zero-point term, rows 4blk + e
  float sl2[GPL];      // softmax_scale * log2(e) * 2^24 / (the row's q scale)
  float thr[GPL];      // rescale threshold 2 / sl2 (score units)
  float kexp;          // k: p, lsum, zacc and acc carry the factor 2^k (wave-uniform)
  float svlim;         // 2^(12 - k): a V scale above it takes the slow path

  // Scores of the two sub-tiles in units of 2^-24:
  //   sum_kg s[t,kg] * S[(g,kg),t] + z[t,kg] * qsum24[(g,kg)].
  template <bool MASK>
  __device__ __forceinline__ void scores(const ST (&st)[2], const bool (&valid)[2],
                                         float (&score)[2][GPL]) const {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      f4 S = KASYM ? f4{0.f, 0.f, 0.f, 0.f} : cinit;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        S = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            aq[c],
            K16  ? __builtin_bit_cast(h8, u4{st[x].k.dw(4 * c), st[x].k.dw(4 * c + 1),
                                             st[x].k.dw(4 * c + 2), st[x].k.dw(4 * c + 3)})
            : K8 ? bytes_to_h8_sub(st[x].k.dw(2 * c), st[x].k.dw(2 * c + 1))
                 : nibbles_to_h8_sub(st[x].k.dw(c)),
            S, 0, 0, 0);
#pragma unroll
      for (int gi = 0; gi < GPL; ++gi) {
        float sc = 0.0f;
#pragma unroll
        for (int kg = 0; kg < NG; ++kg) {
          const int i = gi * NG + kg;
          if constexpr (KASYM) sc = fmaf(st[x].kz.get(kg), qsum24[i], sc);
          if constexpr (K16)
            sc += S[i];
          else
            sc = fmaf(st[x].ks.get(kg * NGK / NG), S[i], sc);
        }
        score[x][gi] = (MASK && !valid[x]) ? -INFINITY : sc;
      }
    }
  }

  // V scales of the two sub-tiles, kept in fp16 (the fp32 products below take
  // them as mixed-precision operands, so they are never converted), and their
  // largest value; tokens past the end read 0 (their bytes are stale).
  template <bool MASK>
  __device__ __forceinline__ float vscales(const ST (&st)[2], const bool (&valid)[2],
                                           _Float16 (&sv)[2][NG]) const {
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        sv[x][g] = V16 ? static_cast<_Float16>(1.0f) : st[x].vs.geth(g);
        if constexpr (MASK) sv[x][g] = valid[x] ? sv[x][g] : static_cast<_Float16>(0.0f);
      }
    if constexpr (V16) {
      return 1.0f;
    } else if constexpr (MASK) {
      float m = 0.0f;
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int g = 0; g < NG; ++g) m = fmaxf(m, static_cast<float>(sv[x][g]));
      return m;
    } else {
      // Scales are non-negative, and non-negative fp16 values order like
      // their bit patterns: a packed unsigned 16-bit max on the scale words.
      const auto w = [](uint32_t u) { return __builtin_bit_cast(u16x2, u); };
      u16x2 m;
      if constexpr (NG == 4)
        m = __builtin_elementwise_max(__builtin_elementwise_max(w(st[0].vs.v.x), w(st[0].vs.v.y)),
                                      __builtin_elementwise_max(w(st[1].vs.v.x), w(st[1].vs.v.y)));
      else if constexpr (NG == 2)
        m = __builtin_elementwise_max(w(st[0].vs.v), w(st[1].vs.v));
      else
        m = u16x2{static_cast<uint16_t>(st[0].vs.v), static_cast<uint16_t>(st[1].vs.v)};
      return static_cast<float>(
          __builtin_bit_cast(_Float16, static_cast<uint16_t>(m[0] > m[1] ? m[0] : m[1])));
    }
  }

  // Does any row's tile max exceed its running max by more than thr, or any
  // V scale exceed svlim?  No cross-lane reduction: lane-wise tests and one
  // ballot.
  __device__ __forceinline__ bool slow_tile(const float (&score)[2][GPL], float svmax) const {
    bool up = svmax > svlim;
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) up |= fmaxf(score[0][gi], score[1][gi]) > m_run[gi] + thr[gi];
    return __any(up);
  }

  // Raise the running max of the rows whose tile max exceeds it by more than
  // thr, lower k when a V scale of the tile exceeds svlim, and rescale the
  // accumulators by both factors (powers of two for k, so exact).
  __device__ __forceinline__ void slow_step(const float (&score)[2][GPL], float svmax) {
    // k from the largest V scale of the tile over the wave: s <= 2^e, and
    // 2^k * s <= 2^12.  k only decreases (it starts at 40, far above any
    // fp16 scale's need: fp16 scales are at least 2^-24).
    float smax = row_max16(svmax);
    smax = fmaxf(smax, __shfl_xor(smax, 16, kWave));
    smax = fmaxf(smax, __shfl_xor(smax, 32, kWave));
    int e = 0;
    frexpf(smax, &e);                                // smax = 0 gives e = 0
    const float knew = fminf(kexp, static_cast<float>(12 - e));
    const float kscale = ldexpf(1.0f, static_cast<int>(knew - kexp));   // 2^(knew - k) <= 1
    kexp = knew;
    svlim = ldexpf(1.0f, 12 - static_cast<int>(knew));
    float alpha[GPL];
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) {
      const float tmax = row_max16(fmaxf(score[0][gi], score[1][gi]));
      const bool up = tmax > m_run[gi] + thr[gi];
      alpha[gi] = (up ? __builtin_amdgcn_exp2f((m_run[gi] - tmax) * sl2[gi]) : 1.0f) * kscale;
      m_run[gi] = up ? tmax : m_run[gi];
    }
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) lsum[gi] *= alpha[gi];
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) zacc[e4] *= alpha[e4 / NG];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[c][h][i] *= alpha[i / NG];
  }

  // Probabilities p (times 2^k), P' = p * s_v split into fp16 hi + lo and
  // transposed to the PV A operand (lane = row (g, vg), slots = tokens), and
  // the zero-point term, for the two sub-tiles.
  template <bool MASK, bool PAIRS = false>
  __device__ __forceinline__ void probs(const ST (&st)[2], const bool (&valid)[2],
                                        const float (&score)[2][GPL],
                                        const _Float16 (&svt)[2][NG],
                                        h8& ahi, h8& alo) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      float p[GPL];
#pragma unroll
      for (int gi = 0; gi < GPL; ++gi) {
        // (score - max) first: the token that sets the max gets p = 2^k exactly
        p[gi] = __builtin_amdgcn_exp2f(fmaf(score[x][gi] - m_run[gi], sl2[gi], kexp));
        lsum[gi] += p[gi];                                    // 0 when masked
      }
      float sv[4], P[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sv[e] = static_cast<float>(svt[x][e % NG]);
        // the exact product rounded once, as p * s_v: an fma with the fp16
        // scale as a mixed operand needs no conversion
        P[e] = fmaf(p[e / NG], sv[e], 0.0f);
        if constexpr (V16) {
          // fp16 V: no zero-point term
        } else if constexpr (VASYM) {
          float zv = st[x].vz.get(e % NG);
          if constexpr (MASK) zv = valid[x] ? zv : 0.0f;
          zacc[e] = fmaf(p[e / NG], zv, zacc[e]);
        } else {
          // symmetric: zero = -8 s (INT4) or -128 s (INT8 codes biased by 128)
          zacc[e] = fmaf(V8 ? -128.0f : -8.0f, P[e], zacc[e]);
        }
      }
      // hi by one explicit conversion (toward zero), lo = p * s_v - hi exactly
      // rounded: both halves derive from the same hi bits
      const h2 hi01 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(P[0], P[1]));
      const h2 hi23 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(P[2], P[3]));
      const float r0 = fmaf(p[0 / NG], sv[0], -static_cast<float>(hi01[0]));
      const float r1 = fmaf(p[1 / NG], sv[1], -static_cast<float>(hi01[1]));
      const float r2 = fmaf(p[2 / NG], sv[2], -static_cast<float>(hi23[0]));
      const float r3 = fmaf(p[3 / NG], sv[3], -static_cast<float>(hi23[1]));
      const h2 lo01 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(r0, r1));
      const h2 lo23 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(r2, r3));
      // PAIRS: "hi" carries rows (g, vg 0 / 1, hi / lo), "lo" rows (g, vg 2 / 3, hi / lo)
      const h4 xhi = PAIRS ? h4{hi01[0], lo01[0], hi01[1], lo01[1]}
                           : h4{hi01[0], hi01[1], hi23[0], hi23[1]};
      const h4 xlo = PAIRS ? h4{hi23[0], lo23[0], hi23[1], lo23[1]}
                           : h4{lo01[0], lo01[1], lo23[0], lo23[1]};
      const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
      const f4 thi = __builtin_amdgcn_mfma_f32_16x16x16f16(xhi, eye, zero4, 0, 0, 0);
      const f4 tlo = __builtin_amdgcn_mfma_f32_16x16x16f16(xlo, eye, zero4, 0, 0, 0);
      const h2 h01 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(thi[0], thi[1]));
      const h2 h23 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(thi[2], thi[3]));
      const h2 l01 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(tlo[0], tlo[1]));
      const h2 l23 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(tlo[2], tlo[3]));
      ahi[4 * x + 0] = h01[0]; ahi[4 * x + 1] = h01[1];
      ahi[4 * x + 2] = h23[0]; ahi[4 * x + 3] = h23[1];
      alo[4 * x + 0] = l01[0]; alo[4 * x + 1] = l01[1];
      alo[4 * x + 2] = l23[0]; alo[4 * x + 3] = l23[1];
    }
  }

  // PV with V transposed on the matrix cores (V arrives as lane = token):
  // accumulator (c, h) holds column d = (D/4)(col/4) + 8c + 2(col%4) + h.
  // INT8 V (V8): the 8 bytes of chunk c, elements in the nibble order of
  // nibbles_to_i8x8 ([e0 e2 e4 e6 | e1 e3 e5 e7]), go through the same
  // transpose with the accumulator started at 128, so each output is the
  // biased code n + 128: the fp16 subnormal (n + 128) 2^-24.
  __device__ __forceinline__ void pv_transposed(const ST (&st)[2], const h8& ahi,
                                                const h8& alo) {
    const i4 vzero = V8 ? i4{128, 128, 128, 128} : i4{0, 0, 0, 0};
    const auto v_i8 = [](const typename ST::VCodes& v, int c) -> long {
      if constexpr (V8) {
        const uint32_t w0 = v.dw(2 * c), w1 = v.dw(2 * c + 1);
        const uint64_t lo = __builtin_amdgcn_perm(w1, w0, 0x06040200u);   // e0 e2 e4 e6
        const uint64_t hi = __builtin_amdgcn_perm(w1, w0, 0x07050301u);   // e1 e3 e5 e7
        return static_cast<long>(lo | (hi << 32));
      } else {
        return nibbles_to_i8x8(v.dw(c));
      }
    };
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const long va = v_i8(st[0].v, c);
      const long vb = v_i8(st[1].v, c);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const i4 ta = __builtin_amdgcn_mfma_i32_16x16x32_i8(va, vsel[h], vzero, 0, 0, 0);
        const i4 tb = __builtin_amdgcn_mfma_i32_16x16x32_i8(vb, vsel[h], vzero, 0, 0, 0);
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
  }

  // PV with fp16 V rows (RowsH): r[i] of sub-tile x holds columns
  // (D/16) col .. (D/16) col + D/16 - 1 of token 16x + 4blk + i, the token of
  // A slot 4x + i.  Accumulator j = 2c + h holds column (D/16) col + j; its B
  // operand takes half j of each token's row, two tokens per dword with one
  // v_perm.  Tokens past the end read 0 (their bytes are stale and could be
  // Inf or NaN, which a zero probability would not cancel).
  template <bool MASK>
  __device__ __forceinline__ void pv_rows16(const ST (&st)[2], const bool (&valid)[2],
                                            int tbase, int t_end, int blk, const h8& ahi,
                                            const h8& alo) {
    uint32_t r[2][4][NCH];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = !MASK || tbase + 16 * x + 4 * blk + i < t_end;
#pragma unroll
        for (int w = 0; w < NCH; ++w) r[x][i][w] = ok ? st[x].v.r[i][w] : 0u;
      }
    (void)valid;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = 2 * c + h;
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        u4 bw;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          bw[q] = __builtin_amdgcn_perm(r[q / 2][2 * (q % 2) + 1][j >> 1],
                                        r[q / 2][2 * (q % 2)][j >> 1], sel);
        const h8 bv = __builtin_bit_cast(h8, bw);
        acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bv, acc[c][h], 0, 0, 0);
        acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bv, acc[c][h], 0, 0, 0);
      }
    }
  }

  // PV with V read from LDS as lane = column: vw[x][i] holds the D/16 nibbles
  // of columns (D/16)*col .. (D/16)*col + D/16 - 1 of token 16x + 4blk + i,
  // the tokens of this lane's A slots 4x + i.  Accumulator j = 2c + h holds
  // column d = (D/16) * col + j.  Token pairs are interleaved by halves with
  // v_perm, then each column's nibble pair is one mask (after one shift per
  // pair of columns): the fp16 subnormal bit patterns of slots (2q, 2q + 1),
  // n * 2^-24 for even j and 16 n * 2^-24 for odd j (h == 1), so the
  // accumulators acc[c][1] carry an extra factor 16.  PAIRS (group-pair
  // layout): vw comes from coop_read_v<PAIRS> already interleaved by token
  // pairs, and accumulator j holds column 64 (j / 4) + 4 col + j % 4.
  template <bool PAIRS = false>
  __device__ __forceinline__ void pv_columns(const uint32_t (&vw)[2][4], const h8& ahi,
                                             const h8& alo) {
    uint32_t u0[4], u1[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = vw[q / 2][2 * (q % 2)];
      const uint32_t b = vw[q / 2][2 * (q % 2) + 1];
      if constexpr (PAIRS) {      // already token pairs (coop_read_v<PAIRS>)
        u0[q] = a;
        u1[q] = b;
      } else {
        u0[q] = __builtin_amdgcn_perm(b, a, 0x05040100u);   // a.lo16 | b.lo16 << 16
        u1[q] = __builtin_amdgcn_perm(b, a, 0x07060302u);   // a.hi16 | b.hi16 << 16
      }
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = 2 * c + h;
        u4 bw;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t u = j < 4 ? u0[q] : u1[q];
          bw[q] = ((j % 4) < 2 ? u : u >> 8) & (j % 2 ? kNib16 : kNib1);
        }
        const h8 bv = __builtin_bit_cast(h8, bw);
        if constexpr (PAIRS) {
          // columns 64 (j / 4) + 4 col + j % 4: groups {0, 1} for j < 4
          acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(j < 4 ? ahi : alo, bv, acc[c][h],
                                                             0, 0, 0);
        } else {
          acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bv, acc[c][h], 0, 0, 0);
          acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bv, acc[c][h], 0, 0, 0);
        }
      }
    }
  }

  // PV with fp16 V rows read from LDS (cooperative kernel): vw[x][i] holds
  // the halves of columns (D/16) col .. (D/16) col + 7 of token 16x + 4blk + i
  // (rows past the end read as 0), the tokens of this lane's A slots 4x + i;
  // accumulator j = 2c + h holds column (D/16) col + j, whose B operand takes
  // half j of each token, two tokens per dword with one v_perm (as pv_rows16).
  __device__ __forceinline__ void pv_columns(const uint4 (&vw)[2][4], const h8& ahi,
                                             const h8& alo) {
    const auto dw = [](const uint4& u, int w) {
      return w == 0 ? u.x : w == 1 ? u.y : w == 2 ? u.z : u.w;
    };
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = 2 * c + h;
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        u4 bw;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          bw[q] = __builtin_amdgcn_perm(dw(vw[q / 2][2 * (q % 2) + 1], j >> 1),
                                        dw(vw[q / 2][2 * (q % 2)], j >> 1), sel);
        const h8 bv = __builtin_bit_cast(h8, bw);
        acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bv, acc[c][h], 0, 0, 0);
        acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bv, acc[c][h], 0, 0, 0);
      }
    }
  }

  // PV with INT8 V codes read from LDS as lane = column: vw[x][i] holds the
  // 8 bytes of columns 8 col .. 8 col + 7 of token 16x + 4blk + i.  The codes
  // are biased by 128 (xor 0x80), then column j takes byte j of a token pair
  // into the two halves of a dword with one v_perm: the fp16 subnormals
  // (n + 128) 2^-24 of slots (2q, 2q + 1); the bias returns through zacc.
  // Accumulator j = 2c + h holds column 8 col + j.
  __device__ __forceinline__ void pv_columns(const uint2 (&vw)[2][4], const h8& ahi,
                                             const h8& alo) {
    uint32_t w[2][2][4];      // [column half][x][i], biased
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[0][x][i] = vw[x][i].x ^ 0x80808080u;
        w[1][x][i] = vw[x][i].y ^ 0x80808080u;
      }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = 2 * c + h;
        const uint32_t sel = static_cast<uint32_t>(j % 4) | (0x0Cu << 8) |
                             (static_cast<uint32_t>(4 + j % 4) << 16) | (0x0Cu << 24);
        u4 bw;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          bw[q] = __builtin_amdgcn_perm(w[j / 4][q / 2][2 * (q % 2) + 1],
                                        w[j / 4][q / 2][2 * (q % 2)], sel);
        const h8 bv = __builtin_bit_cast(h8, bw);
        acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bv, acc[c][h], 0, 0, 0);
        acc[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bv, acc[c][h], 0, 0, 0);
      }
    }
  }

  // General step: any tile, masked or not, max moving or not.
  template <bool MASK>
  __device__ __forceinline__ void step(const ST (&st)[2], int tbase, int t_end,
                                       int col) {
    bool valid[2] = {true, true};
    if constexpr (MASK) {
      valid[0] = tbase + col < t_end;
      valid[1] = tbase + 16 + col < t_end;
    }
    float score[2][GPL];
    scores<MASK>(st, valid, score);
    _Float16 sv[2][NG];
    const float svmax = vscales<MASK>(st, valid, sv);
    if (slow_tile(score, svmax)) slow_step(score, svmax);
    h8 ahi, alo;
    probs<MASK>(st, valid, score, sv, ahi, alo);
    if constexpr (V16)
      pv_rows16<MASK>(st, valid, tbase, t_end, static_cast<int>((threadIdx.x & (kWave - 1)) >> 4),
                      ahi, alo);
    else
      pv_transposed(st, ahi, alo);
  }

};

// Query heads per head set: a set fills the 16 rows of one 16x16 MFMA.
template <int NG>
__host__ __device__ constexpr int heads_per_set() { return 16 / NG; }

// q, constants and accumulators of the wave serving kv head `kvh`, for the
// head set whose first query head (within the kv head's group) is `hs`.
// This lane's D/4 consecutive q elements (row r = col of the head set whose
// first query head is `hs`), as raw 16-bit words; loaded apart from
// init_wave so that a kernel can issue these loads next to its other first
// loads and wait once for all of them.
template <int D, int NG>
__device__ __forceinline__ void load_q(uint4 (&qw)[D / 32], const DecodeArgs& a, int seq,
                                       int kvh, int col, int blk, int hs = 0) {
  const int nh = min(heads_per_set<NG>(), a.group - hs);
  const int rows = nh * NG;
  const int g = col < rows ? col / NG : 0;
  const uint16_t* qp =
      a.q + seq * a.q_stride_seq + (kvh * a.group + hs + g) * a.q_stride_head + (D / 4) * blk;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) qw[i] = reinterpret_cast<const uint4*>(qp)[i];
}

template <int D, int NG, bool KASYM, bool VASYM, int KCH = D / 32, int NGK = NG, bool V8 = false,
          bool V16 = false>
__device__ __forceinline__ void init_wave(WaveState<D / 32, NG, KASYM, VASYM, KCH, NGK, V8, V16>& W,
                                          const uint4 (&qw)[D / 32], const DecodeArgs& a,
                                          int col, int blk, int hs = 0) {
  constexpr int NCH = D / 32;
  constexpr int GPL = 4 / NG;
  constexpr bool K8 = KCH == 2 * NCH;
  constexpr bool K16 = KCH == 4 * NCH;
  const int G = a.group;
  const int nh = min(heads_per_set<NG>(), G - hs);
  // rows (g, kg): kg is a K scale group for INT4 K; for INT8 K the NG row
  // groups split the head dim in equal parts that share the K scale(s)
  const int gs = K8 || K16 ? D / NG : a.kp.group_size;
  const int rows = nh * NG;
  // ---- masked q (row r = col): this lane's D/4 consecutive elements ----------
  // A bf16 q enters the fp16 A operand scaled by a power of two per head,
  // qscale = 2^(14 - e) with max|q_head| < 2^e: exact for every element down
  // to 2^-28 of the head's maximum (fp16 holds bf16's 8-bit mantissa), and
  // the scale leaves the scores through the row's softmax scale.
  // The online softmax below tracks each row's maximum score, which needs a
  // positive scale: a negative softmax scale enters as -q with |scale|
  // (negation is exact), and a zero scale as q = 0 (every score 0, so the
  // weights are uniform over the valid tokens) with any positive scale.
  const bool qneg = a.scale_log2 < 0.0f;
  const bool qzero = a.scale_log2 == 0.0f;
  float qpart = 0.0f;
  float qscale = 1.0f;
  {
    const int r = col;
    const bool on = r < rows && ((D / 4) * blk) / gs == r % NG && !qzero;
    uint16_t qv[D / 4];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const uint4 w = qw[i];
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qv[8 * i + 2 * j] = static_cast<uint16_t>(ws[j]);
        qv[8 * i + 2 * j + 1] = static_cast<uint16_t>(ws[j] >> 16);
      }
    }
    if (a.q_bf16) {
      float mx = 0.0f;
#pragma unroll
      for (int i = 0; i < D / 4; ++i) mx = fmaxf(mx, fabsf(bf16_bits_to_float(qv[i])));
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));   // the four lane blocks hold the head
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      int ex = 0;
      frexpf(mx, &ex);
      qscale = mx > 0.0f ? ldexpf(1.0f, 14 - ex) : 1.0f;
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int el = 8 * c + (K16 ? e : K8 ? kByteK8[e] : kNibK[e]);
        _Float16 v = !on ? _Float16(0)
                     : a.q_bf16 ? static_cast<_Float16>(bf16_bits_to_float(qv[el]) * qscale)
                                : __builtin_bit_cast(_Float16, qv[el]);
        if (qneg) v = -v;
        // odd nibbles arrive as 16 n: their q slot holds q / 16 (exact
        // unless |q| < 2^-10, where the fp16 subnormal keeps an absolute
        // error below 2^-25); INT8 codes arrive as n + 128
        W.aq[c][e] = (!K8 && !K16 && (e & 2)) ? v * static_cast<_Float16>(0.0625f) : v;
        qpart += static_cast<float>(v);
      }
    }
  }
  qpart += __shfl_xor(qpart, 16, kWave);
  qpart += __shfl_xor(qpart, 32, kWave);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // 2^-24 is exact in fp32: K codes enter the QK product as n * 2^-24
    W.qsum24[i] = __shfl(qpart, 4 * blk + i, kWave) * 0x1p-24f;
    if constexpr (K16) W.cinit[i] = 0.0f;
    else if constexpr (K8) W.cinit[i] = -128.0f * W.qsum24[i];
    else if constexpr (!KASYM) W.cinit[i] = -8.0f * W.qsum24[i];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) W.eye[e] = (blk == col / 4 && e == col % 4) ? 1.0f : 0.0f;
#pragma unroll
  for (int h = 0; h < 2; ++h)
    W.vsel[h] = blk == col / 4 ? static_cast<long>(1ull << (8 * (4 * h + col % 4))) : 0l;
#pragma unroll
  for (int c = 0; c < NCH; ++c) W.acc[c][0] = W.acc[c][1] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < GPL; ++i) {
    W.m_run[i] = -INFINITY;
    W.lsum[i] = 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) W.zacc[e] = 0.0f;
  // no V scale seen yet: the first tile sets k (every fp16 scale exceeds 2^-28)
  W.kexp = 40.0f;
  W.svlim = 0x1p-28f;
  // scores are in units of 2^-24 times the row's q scale
#pragma unroll
  for (int gi = 0; gi < GPL; ++gi) {
    const float qs = __shfl(qscale, 4 * blk + gi * NG, kWave);
    // INT4 / INT8 codes enter as n * 2^-24; fp16 K as itself
    W.sl2[gi] = (qzero ? 1.0f : fabsf(a.scale_log2)) * (K16 ? 1.0f : 0x1p24f) / qs;
    W.thr[gi] = kRescaleLog2 / W.sl2[gi];
  }
}

// Reduce over tokens and write the wave's partial (acc, max, sum) for query
// head g of the set at entry base + g * stride of the workspace.  COLS: the
// accumulators follow pv_columns' column order, else pv_transposed's.
template <int D, int NG, bool KASYM, bool VASYM, bool COLS = false, int KCH = D / 32,
          int NGK = NG, bool V8 = false, bool V16 = false, bool PAIRS = false>
__device__ __forceinline__ void write_partials_at(
    WaveState<D / 32, NG, KASYM, VASYM, KCH, NGK, V8, V16>& W, const DecodeArgs& a,
    int64_t base, int64_t stride, int col, int blk, int hs = 0) {
  constexpr int NCH = D / 32;
  constexpr int GPL = 4 / NG;
  const int G = min(heads_per_set<NG>(), a.group - hs);   // heads of this set
  const int gs = a.vp.group_size;
  // acc, zacc and lsum carry 2^k
  const float kinv = ldexpf(1.0f, -static_cast<int>(W.kexp));
#pragma unroll
  for (int gi = 0; gi < GPL; ++gi) W.lsum[gi] = row_sum16(W.lsum[gi]) * kinv;
#pragma unroll
  for (int e = 0; e < 4; ++e) W.zacc[e] = row_sum16(W.zacc[e]);
  // the cooperative kernel's group-pair PV (WaveState::PAIRS_OK, one head set)
  static_assert(!PAIRS || (COLS && !V8 && !V16 && NG == 4 && D == 128), "pair layout shapes");
  if constexpr (PAIRS) {
    const int vgl = col / 8;                 // this lane's group within each pair
    const int g = blk;
    if (g < G) {
      const int64_t row = base + g * stride;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int j = 2 * c + h;
          const int d = 64 * (j / 4) + 4 * col + j % 4;
          // constant indices only (a lane-dependent index would move the
          // accumulators to scratch memory)
          const f4 v = W.acc[c][h];
          const float hl = vgl ? v[2] + v[3] : v[0] + v[1];
          const float z = vgl ? W.zacc[2 * (j / 4) + 1] : W.zacc[2 * (j / 4)];
          // odd columns carry a factor 16 (pv_columns)
          a.part_o[row * D + d] = fmaf(hl, h ? 0x1p20f : 0x1p24f, z) * kinv;
        }
    }
  }
#pragma unroll
  for (int c = 0; c < (PAIRS ? 0 : NCH); ++c) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int d = COLS || V16 ? (D / 16) * col + 2 * c + h
                                : (D / 4) * (col / 4) + 8 * c + 2 * (col % 4) + h;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * blk + i;
        const int g = r / NG;
        if (g < G && d / gs == r % NG) {
          const int64_t row = base + g * stride;
          // pv_columns' odd INT4 columns carry a factor 16
          a.part_o[row * D + d] =
              fmaf(W.acc[c][h][i], V16 ? 1.0f : COLS && h && !V8 ? 0x1p20f : 0x1p24f,
                   W.zacc[i]) * kinv;
        }
      }
    }
  }
  if (col == 0) {
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) {
      const int g = (4 * blk) / NG + gi;
      if (g < G) {
        const int64_t row = base + g * stride;
        a.part_ml[2 * row] = W.m_run[gi] * W.sl2[gi];
        a.part_ml[2 * row + 1] = W.lsum[gi];
      }
    }
  }
}

// The split schedule's entries: [num_seqs, Hq, num_splits].
template <int D, int NG, bool KASYM, bool VASYM, bool COLS = false, int KCH = D / 32,
          int NGK = NG, bool V8 = false, bool V16 = false>
__device__ __forceinline__ void write_partials(WaveState<D / 32, NG, KASYM, VASYM, KCH, NGK, V8, V16>& W,
                                               const DecodeArgs& a, int seq, int kvh,
                                               int split, int col, int blk, int hs = 0) {
  const int64_t row0 = static_cast<int64_t>(seq) * a.num_q_heads + kvh * a.group + hs;
  write_partials_at<D, NG, KASYM, VASYM, COLS, KCH, NGK, V8, V16>(
      W, a, row0 * a.num_splits + split, a.num_splits, col, blk, hs);
}

// Per-head loads: each wave fetches its own kv head's rows (any layout that
// passes the alignment checks).  One wave per (sequence, kv head, split).
// fp16 K and V (V16) keep two 32-token tiles of 256-byte rows per wave in
// registers: 4 waves per block, so each wave may use the whole register file
// of its SIMD lane (VGPRs and AGPRs) without spilling.
template <int D, int NG, bool KASYM, bool VASYM, bool K16 = false, bool V8 = false,
          bool V16 = false>
__global__ __launch_bounds__(V16 ? 256 : 512) void decode_mfma_kernel(DecodeArgs a) {
  constexpr int NCH = D / 32;    // K-chunks of 32 along head_dim = dwords per lane
  constexpr int LB = D / 8;      // bytes of INT4 codes per lane per token
  constexpr int KCH = K16 ? 4 * NCH : NCH;   // fp16 K: D/2 bytes per lane per token
  // INT8 V: D/4 bytes per lane per token; fp16 V: rows (Rows16, VCH = 0)
  constexpr int VCH = V16 ? 0 : V8 ? 2 * NCH : NCH;
  constexpr int KEB = K16 ? 2 : 1;           // K element bytes (its strides are in elements)
  constexpr int VEB = V16 ? 2 : 1;           // V element bytes
  const int lane = threadIdx.x & (kWave - 1);
  const int col = lane & 15;
  const int blk = lane >> 4;
  // the wave index is uniform; readfirstlane lets the compiler keep every
  // per-head base address in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int hpb = blockDim.x / kWave;
  const int split = blockIdx.x;
  const int seq = blockIdx.y;
  const int kvh = blockIdx.z * hpb + wave;
  if (kvh >= a.num_kv_heads) return;
  const int seq_len = min(a.seq_lens[seq], a.max_context);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= seq_len) return;
  const int t_end = min(seq_len, t_begin + a.split_tokens);
  // the token being decoded, when the caller fused its append into this launch
  decode_append<D>(a, seq, kvh, split, seq_len, lane);

  WaveState<NCH, NG, KASYM, VASYM, KCH, NG, V8, V16> W;
  {
    uint4 qw[D / 32];
    load_q<D, NG>(qw, a, seq, kvh, col, blk);
    init_wave<D, NG, KASYM, VASYM, KCH, NG, V8, V16>(W, qw, a, col, blk);
  }

  Addr A;
  {
    const knlp_kv_plane& K = a.kp;
    const knlp_kv_plane& V = a.vp;
    A.kc = static_cast<const uint8_t*>(K.data) + KEB * kvh * K.stride_head;
    A.vc = static_cast<const uint8_t*>(V.data) + VEB * kvh * V.stride_head;
    A.ks = static_cast<const uint16_t*>(K.scales) + kvh * K.s_stride_head;
    A.vs = static_cast<const uint16_t*>(V.scales) + kvh * V.s_stride_head;
    A.kz = KASYM ? static_cast<const uint16_t*>(K.zeros) + kvh * K.z_stride_head : nullptr;
    A.vz = VASYM ? static_cast<const uint16_t*>(V.zeros) + kvh * V.z_stride_head : nullptr;
    A.kc_b = KEB * K.stride_block; A.kc_p = KEB * K.stride_page;
    A.vc_b = VEB * V.stride_block; A.vc_p = VEB * V.stride_page;
    A.ks_b = K.s_stride_block; A.ks_p = K.s_stride_page;
    A.vs_b = V.s_stride_block; A.vs_p = V.s_stride_page;
    A.kz_b = K.z_stride_block; A.kz_p = K.z_stride_page;
    A.vz_b = V.z_stride_block; A.vz_p = V.z_stride_page;
    // a lane holds elements 32 blk .. 32 blk + 31 of its token: D/8 bytes of
    // INT4 codes or D/2 bytes of fp16
    A.lkc = static_cast<uint32_t>(KEB * col * K.stride_page + (K16 ? D / 2 : LB) * blk);
    // fp16 V: token 4 blk + i's columns (D/16) col .. (D/16) col + D/16 - 1 (RowsH)
    A.lvc = V16 ? static_cast<uint32_t>(2 * (4 * blk) * V.stride_page + (D / 8) * col)
                : static_cast<uint32_t>(col * V.stride_page + (V8 ? D / 4 : LB) * blk);
    A.vrow = static_cast<uint32_t>(2 * V.stride_page);
    A.lks = static_cast<uint32_t>(2 * col * K.s_stride_page);
    A.lvs = static_cast<uint32_t>(2 * col * V.s_stride_page);
    A.lkz = static_cast<uint32_t>(2 * col * K.z_stride_page);
    A.lvz = static_cast<uint32_t>(2 * col * V.z_stride_page);
    A.bt = a.block_table + seq * a.bt_stride;
    A.bs_shift = a.block_shift;
  }

  PageWindow PW;
  PW.last = (t_end - 1) >> A.bs_shift;
  PW.fill(A.bt, lane, t_begin >> A.bs_shift);

  // 32-token tiles in order through a two-buffer pipeline: the loads of tile
  // i + 1 are in flight while tile i computes.  Only a sequence's last split
  // can end in a partial tile; that one runs the masked step.  Tiles are
  // visited in increasing order so the page window only moves forward.
  const int ntiles = (t_end - t_begin + 31) / 32;
  using ST = SubTile<NCH, NG, KCH, NG, VCH>;
  ST X[2], Y[2];
  auto load_tile = [&](int tb, ST(&buf)[2]) {
    load_sub<NCH, NG, KASYM, VASYM, KCH, VCH>(A, PW, lane, tb, buf[0]);
    // a second half wholly past the end re-reads the first half's page (masked)
    load_sub<NCH, NG, KASYM, VASYM, KCH, VCH>(A, PW, lane, tb + 16 < t_end ? tb + 16 : tb,
                                              buf[1]);
  };
  auto run_tile = [&](int tb, const ST(&buf)[2]) {
    if (tb + 32 <= t_end)
      W.template step<false>(buf, tb, t_end, col);
    else
      W.template step<true>(buf, tb, t_end, col);
  };
  load_tile(t_begin, X);
  for (int i = 0; i < ntiles; i += 2) {
    const int tb = t_begin + 32 * i;
    if (i + 1 < ntiles) load_tile(tb + 32, Y);
    run_tile(tb, X);
    if (i + 1 >= ntiles) break;
    if (i + 2 < ntiles) load_tile(tb + 64, X);
    run_tile(tb + 32, Y);
  }
  write_partials<D, NG, KASYM, VASYM, false, KCH, NG, V8, V16>(W, a, seq, kvh, split, col, blk);
}

// ---------------------------------------------------------------------------
// Cooperative page staging, for caches whose kv heads are densely packed in a
// token row (stride_head = one head's code bytes and scale halves) and
// Hkv % 8 == 0.
//
// A block is 8 waves serving 8 consecutive kv heads of one (sequence, split),
// so each 16-token sub-tile of each array (codes K and V, scales and zeros) is
// 16 rows of 8 heads' contiguous bytes.  The block copies a 32-token tile
// from HBM straight into LDS with global_load_lds (16 bytes per lane, one
// wave instruction = 1 KB of consecutive rows), NBUF - 1 tiles ahead of the
// compute; after a barrier each wave reads its own head's slice in the lane
// layout of the per-head kernel.  Per-head loads touch 64-byte fragments at a
// 512-byte stride and 8-byte scale fragments at a 64-byte stride, which
// measured 55-59% of HBM peak even without compute; page-contiguous copies
// run as fast as a plain stream.  The direct-to-LDS copy keeps the staging
// out of VGPRs.
//
// K is packed INT4 (NG scale groups, the same as V's) or INT8 (one byte per
// element, NGK scale groups: 1 for one scale per row, or NG).  A wave serves
// the G query heads of its kv head in head sets of 16 / NG heads, one
// WaveState each (G = 5 with g32 V: heads 0-3 and head 4); the sets share the
// staged tile and, after common-subexpression elimination, its K and V
// conversions.
// ---------------------------------------------------------------------------
template <int D, int NG, bool K8 = false, int NGK = NG, bool V8 = false, bool K16 = false,
          bool V16 = false, bool FEW = false>
struct CoopLayout {
  // fp16 K rows (512 bytes per token and kv head with fp16 V) take 4 kv heads
  // per block, so that 32-token tiles of K and V (64 KB) double-buffer in
  // LDS; packed rows take 8
  static constexpr int kHeads = K16 ? 4 : 8;
  // Waves that issue the tile copies: all of them, or with FEW (8 kv heads)
  // waves 0-3 only, one per SIMD.  A CU runs two of the 8 waves per SIMD,
  // and the second wave on a SIMD, which issues after the first, reaches the
  // tile barrier last; with FEW it has no copies to issue.  In interleaved
  // A/B runs that shortened the split-K partials (config 4: 79.0 -> 75.6 us,
  // config 5: 290.2 -> 280.4, config 8: 96.6 -> 92.1, config 6: 51.6 ->
  // 50.0) and the stream schedule's at config 8 (96.6 -> 93.1 us), with
  // config 2 and the ragged config 3 unchanged within the spread; both
  // cooperative kernels use it.
  static constexpr int NCW = (FEW && !K16) ? 4 : kHeads;
  static constexpr bool ALL = NCW == kHeads;       // every wave copies
  static constexpr int WPS = NCW / 2;              // waves copying each sub-tile
  static constexpr int HBK = K16 ? 2 * D : K8 ? D : D / 2;   // K bytes per head and token
  static constexpr int HBV = V16 ? 2 * D : V8 ? D : D / 2;   // V bytes per head and token
  static constexpr int SBK = K16 ? 0 : 2 * NGK;    // K scale bytes per head and token
  static constexpr int SBV = V16 ? 0 : 2 * NG;     // V scale bytes per head and token
  static constexpr int CROWK = kHeads * HBK;       // LDS rows (16 rows per sub-tile)
  static constexpr int CROWV = kHeads * HBV;
  static constexpr int SROWK = kHeads * SBK;
  static constexpr int SROWV = kHeads * SBV;
  static constexpr int CPSK = 16 * CROWK / 1024;   // 1-KB wave copies per code sub-tile
  static constexpr int CPSV = 16 * CROWV / 1024;
  static constexpr int NPWK = CPSK / WPS;          // code parts per wave and tile
  static constexpr int NPWV = CPSV / WPS;
  static constexpr int NJ = NPWK + NPWV;           // code copies per wave and tile
  // scale arrays (K scales, V scales, K zeros, V zeros) per copying wave:
  // four arrays of two sub-tiles over the copying waves
  static constexpr int NSA = NCW == 4 && !K16 ? 2 : 1;
  static constexpr bool HAS_KZ = !K8 && !K16;      // K zero-points (asymmetric INT4 K)
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + 2 * 16 * CROWK;
  static constexpr int KS_OFF = V_OFF + 2 * 16 * CROWV;   // scale arrays, 2 sub-tiles each
  static constexpr int VS_OFF = KS_OFF + 2 * 16 * SROWK;
  static constexpr int KZ_OFF = VS_OFF + 2 * 16 * SROWV;
  static constexpr int VZ_OFF = KZ_OFF + (HAS_KZ ? 2 * 16 * SROWK : 0);
  static constexpr int BYTES = VZ_OFF + 2 * 16 * SROWV;
  // LDS tile buffers at one block per CU (160 KB): copies run NBUF - 1 tiles ahead
  static constexpr int NBUF = 4 * BYTES <= 160 * 1024 ? 4 : 3 * BYTES <= 160 * 1024 ? 3 : 2;
  static_assert(NBUF * BYTES <= 160 * 1024, "tile buffers fit one CU's LDS");
  static_assert(CPSK % WPS == 0 && CPSV % WPS == 0 && NPWK >= 1 && NPWK <= 8 && NPWV >= 1 &&
                    NPWV <= 8,
                "each sub-tile's code parts split evenly over its waves");
  static_assert(16 * SROWK <= 1024 && 16 * SROWV <= 1024, "one wave copy per scale sub-tile");
  // a lane copies one 16-byte chunk of one scale row (the block's heads'
  // scales of one token), so rows must be whole chunks
  static_assert(SROWK % 16 == 0 && SROWV % 16 == 0, "scale rows of whole 16-byte chunks");
  // Scale array j of copying wave w (of its sub-tile w % 2): 8 waves take
  // array w / 2 (0 K scales, 1 V scales, 2 K zeros, 3 V zeros), 4 copying
  // waves of 8 arrays w / 2 and w / 2 + 2; with fp16 K (no K scales or
  // zeros) 4 waves take V scales (w / 2 = 0) and V zeros.
  __host__ __device__ static constexpr int s_array(int wave, int j = 0) {
    return kHeads == 8 ? (wave >> 1) + 2 * j : ((wave >> 1) == 0 ? 1 : 3);
  }
  // scale array a: 0 K scales, 1 V scales, 2 K zeros, 3 V zeros
  __host__ __device__ static constexpr int s_off(int a) {
    return a == 0 ? KS_OFF : a == 1 ? VS_OFF : a == 2 ? KZ_OFF : VZ_OFF;
  }
  __host__ __device__ static constexpr int s_row(int a) { return (a & 1) ? SROWV : SROWK; }
  // Rows are not padded; bank conflicts are avoided by XOR swizzles.  The
  // 16-byte chunk c of code row r (r < 16) lives at chunk c ^ r: the 16 rows a
  // wave reads at one head offset then cover all 64 banks.
  __host__ __device__ static constexpr int code_off(int crow, int r, int byte) {
    return r * crow + ((((byte >> 4) ^ r) << 4) | (byte & 15));
  }
  // The 16-byte chunk c of scale row r lives at chunk c ^ scale_swz(r); the
  // 16 rows' slots of one head then fall in distinct banks.
  __host__ __device__ static constexpr int scale_swz(int srow, int r) {
    return srow >= 32 ? (r * srow / 256) & (srow / 16 - 1) : 0;
  }
  __host__ __device__ static constexpr int scale_off(int srow, int r, int byte) {
    return r * srow + ((((byte >> 4) ^ scale_swz(srow, r)) << 4) | (byte & 15));
  }
};

// Loop-invariant addressing of the cooperative copy.  Strides are in bytes
// and fit 32 bits (the host checks), so a page's address is one 32x32->64
// multiply-add on the scalar unit.  Copying wave w copies sub-tile x = w % 2
// only: code parts w / 2 + WPS k of K and V and the scale chunks of its
// arrays (L::s_array), so each copying wave looks up one page per tile.
struct CoopScale {
  const uint8_t* sp;      // the scale array, head h0
  uint32_t sp_b, sp_p;    // its block and page strides in bytes
  uint32_t ls;            // this lane's byte offset in HBM
  bool on;                // this wave copies it (wave-uniform)
  bool lane_on;           // this lane copies a chunk
  int lds;                // LDS offset of this wave's sub-tile of it
};

struct CoopAddr {
  const uint8_t* kc;      // codes of head h0 (block/page strides below)
  const uint8_t* vc;
  uint32_t kc_b, kc_p, vc_b, vc_p;   // bytes
  uint32_t lk[8], lv[8];  // lane byte offsets in HBM (code parts)
  bool same_kv;           // K and V codes share their strides (one page offset)
  bool copier;            // this wave issues copies (wave-uniform)
  int nsc;                // scale copies per tile of this wave
  int x;                  // sub-tile this wave copies
  CoopScale s0, s1;       // this wave's scale arrays (s1: four copying waves)
  const int32_t* bt;
  int bs_shift;
};

// 16 bytes per lane from global memory (64-bit scalar base + 32-bit lane
// offset) straight into LDS at m0 + 16 * lane, non-temporal (gfx950 cache
// policy NT): each K/V byte is read once per launch, in whole lines, by the
// one workgroup that copies its page, so the lines need not stay in the
// caches.  At config 2 the partial went from 65.6 to 59.4 us with the hint
// (and a plain streaming read of the same bytes from 0.764 to 0.811 of
// 8 TB/s).  The per-head and VALU kernels keep default loads: their waves
// read one head's slice of lines that neighbouring heads' waves read too
// (with the hint their fp16 decode at config 3 took 724 us against 519).
// Written as inline asm so that the compiler does not track these copies:
// its conservative tracking would put a full vector-memory wait before
// every LDS read, serialising the copies of later tiles with the compute of
// this one.  All waits for the copies are explicit (wait_vmcnt) and
// followed by a block barrier before any wave reads the copied bytes.
__device__ __forceinline__ void lds_copy16(const void* base, uint32_t voff, const void* lds_dst) {
  // base and m0 are wave-uniform; readfirstlane makes that explicit so that
  // both are allocated to SGPRs
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  // (readfirstlane returns int: convert through uint32_t, never sign-extend)
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | lo;
  // the low 32 bits of an LDS location's flat address are its LDS offset
  // (the aperture is the high half); an explicit flat -> LDS cast would add a
  // null check
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_dst)));
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt"
               :
               : "v"(voff), "s"(sb), "s"(m0)
               : "memory", "m0");
}

// Issue this wave's copies of the tile at `tb` into `buf`.  The page number
// comes from the lane-held block-table window by v_readlane: no memory wait
// at all, except when the window moves on (every 64 pages), whose refill
// waits for its own load inside the refill.  A second half wholly past the
// end re-reads the first half's page (its tokens are masked).
template <class L>
__device__ __forceinline__ void coop_issue(const CoopAddr& C, PageWindow& PW, int lane,
                                           int wave, int tb, int t_end, uint8_t* buf) {
  if constexpr (!L::ALL) {
    if (!C.copier) return;
  }
  const int pb = (C.x == 0 || tb + 16 < t_end) ? tb + 16 * C.x : tb;
  const uint32_t pg = static_cast<uint32_t>(PW.page(C.bt, lane, pb >> C.bs_shift));
  const uint32_t of = static_cast<uint32_t>(pb & ((1 << C.bs_shift) - 1));
  const uint64_t ok = static_cast<uint64_t>(pg) * C.kc_b + of * C.kc_p;
  const uint64_t ov = C.same_kv ? ok : static_cast<uint64_t>(pg) * C.vc_b + of * C.vc_p;
  // this wave's parts (wave >> 1) + WPS k of each code sub-tile
  const int p0 = (wave >> 1) * 1024;
  uint8_t* dk = buf + L::K_OFF + C.x * 16 * L::CROWK + p0;
  uint8_t* dv = buf + L::V_OFF + C.x * 16 * L::CROWV + p0;
#pragma unroll
  for (int k = 0; k < L::NPWK; ++k) lds_copy16(C.kc + ok, C.lk[k], dk + k * L::WPS * 1024);
#pragma unroll
  for (int k = 0; k < L::NPWV; ++k) lds_copy16(C.vc + ov, C.lv[k], dv + k * L::WPS * 1024);
  const auto scale_copy = [&](const CoopScale& S) {
    if (S.on) {
      const uint64_t os = static_cast<uint64_t>(pg) * S.sp_b + of * S.sp_p;
      if (S.lane_on) lds_copy16(S.sp + os, S.ls, buf + S.lds);
    }
  };
  scale_copy(C.s0);
  if constexpr (L::NSA == 2) scale_copy(C.s1);
}

// s_waitcnt for "at most N vector-memory operations outstanding" (gfx9
// encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait until this wave's copies of the next tile have landed, leaving the
// copies of `later` (<= 2) further tiles in flight: each tile is NJ code
// copies and C.nsc scale copies of a copying wave.  A wave that copies
// nothing has nothing to wait for (the block barrier after this orders its
// reads behind the copying waves' waits).
template <int PER>
__device__ __forceinline__ void wait_later_tiles(int later) {
  if (later <= 0)
    wait_vmcnt<0>();
  else if (later == 1)
    wait_vmcnt<PER>();
  else
    wait_vmcnt<2 * PER>();
}

template <class L>
__device__ __forceinline__ void wait_tile_copies(int later, const CoopAddr& C) {
  if constexpr (L::NSA == 1) {
    if (C.s0.on) wait_later_tiles<L::NJ + 1>(later); else wait_later_tiles<L::NJ>(later);
  } else {
    if (!C.copier) return;
    if (C.nsc == 0)
      wait_later_tiles<L::NJ>(later);
    else if (C.nsc == 1)
      wait_later_tiles<L::NJ + 1>(later);
    else
      wait_later_tiles<L::NJ + 2>(later);
  }
}

template <int NG>
__device__ __forceinline__ void halves_from_lds(Halves<NG>& h, const uint8_t* p) {
  if constexpr (NG == 4)
    h.v = *reinterpret_cast<const uint2*>(p);
  else if constexpr (NG == 2)
    h.v = *reinterpret_cast<const uint32_t*>(p);
  else
    h.v = *reinterpret_cast<const uint16_t*>(p);
}

// This wave's head slice of the tile in `buf`, in the per-head lane layout:
// each lane holds a quarter of its token's K row (D/8 bytes of INT4 codes or
// D/4 bytes of INT8 codes) and the token's scale / zero halves.
template <class L, bool KASYM, bool VASYM, int NCH, int NG, int KCH, int NGK, int VCH>
__device__ __forceinline__ void coop_read(const uint8_t* buf, int wave, int col, int blk,
                                          SubTile<NCH, NG, KCH, NGK, VCH> (&st)[2]) {
  constexpr int KLB = L::HBK / 4;    // K code bytes per lane and token
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const uint8_t* kp = buf + L::K_OFF + x * 16 * L::CROWK;
    const int kb = wave * L::HBK + blk * KLB;
    if constexpr (KLB == 64) {          // fp16 K: a quarter row, 32 halves
#pragma unroll
      for (int j = 0; j < 4; ++j)
        st[x].k.v[j] = *reinterpret_cast<const uint4*>(kp + L::code_off(L::CROWK, col, kb + 16 * j));
    } else if constexpr (KLB == 32) {
      st[x].k.v = *reinterpret_cast<const uint4*>(kp + L::code_off(L::CROWK, col, kb));
      st[x].k.w = *reinterpret_cast<const uint4*>(kp + L::code_off(L::CROWK, col, kb + 16));
    } else if constexpr (KLB == 16) {
      st[x].k.v = *reinterpret_cast<const uint4*>(kp + L::code_off(L::CROWK, col, kb));
    } else {
      st[x].k.v = *reinterpret_cast<const uint2*>(kp + L::code_off(L::CROWK, col, kb));
    }
    if constexpr (L::SBK > 0)
      halves_from_lds<NGK>(st[x].ks, buf + L::KS_OFF + x * 16 * L::SROWK +
                                         L::scale_off(L::SROWK, col, wave * L::SBK));
    if constexpr (L::SBV > 0)
      halves_from_lds<NG>(st[x].vs, buf + L::VS_OFF + x * 16 * L::SROWV +
                                        L::scale_off(L::SROWV, col, wave * L::SBV));
    if constexpr (KASYM)
      halves_from_lds<NG>(st[x].kz, buf + L::KZ_OFF + x * 16 * L::SROWK +
                                        L::scale_off(L::SROWK, col, wave * L::SBK));
    if constexpr (VASYM)
      halves_from_lds<NG>(st[x].vz, buf + L::VZ_OFF + x * 16 * L::SROWV +
                                        L::scale_off(L::SROWV, col, wave * L::SBV));
  }
}

// V of this wave's head as PV B operands (pv_columns): vw[x][i] holds the
// D/32 bytes at columns (D/16)*col.. of token 16x + 4blk + i.  The four lane
// blocks read rows 4blk + i, whose chunk swizzles differ, so the 64 lanes
// hit 64 distinct banks.
//
// fp16 V (16 bytes per lane and token: the 8 halves of columns 8 col ..
// 8 col + 7): rows of a masked tile's tokens past t_end are read as 0, since
// the bytes there are stale and could hold Inf or NaN, which a zero
// probability would not cancel.
template <class L, int D, bool PAIRS = false, bool MASK = false, class VW>
__device__ __forceinline__ void coop_read_v(const uint8_t* buf, int wave, int col, int blk,
                                            VW (&vw)[2][4], int tb = 0, int t_end = 0) {
  constexpr int CB = L::HBV / 16;      // V code bytes per lane and token: 8 columns
  if constexpr (CB == 16) {
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = L::V_OFF + x * 16 * L::CROWV +
                      L::code_off(L::CROWV, 4 * blk + i, wave * L::HBV + 16 * col);
        const uint4 v = *reinterpret_cast<const uint4*>(buf + o);
        const bool ok = !MASK || tb + 16 * x + 4 * blk + i < t_end;
        vw[x][i] = ok ? v : uint4{0u, 0u, 0u, 0u};
      }
  } else if constexpr (PAIRS) {
    // token pairs (4 blk + 2p, 4 blk + 2p + 1): vw[x][2p] holds columns
    // 4 col .. 4 col + 3 (groups 0-1) of the two tokens, one per half,
    // vw[x][2p + 1] columns 64 + 4 col .. (groups 2-3): one v_perm per word
    // joins the two 16-bit reads (pv_columns<true> takes them as they are)
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int base = L::V_OFF + x * 16 * L::CROWV;
        const int b0 = wave * L::HBV + 2 * col;
        const int r = 4 * blk + 2 * p;
        const auto ld = [&](int row, int byte) {
          return *reinterpret_cast<const uint16_t*>(buf + base + L::code_off(L::CROWV, row, byte));
        };
        // (a two-element vector rather than shifts and ors, so that the
        // compiler joins the halves with one v_perm and no masking)
        const u16x2 lo = {ld(r, b0), ld(r + 1, b0)};
        const u16x2 hi = {ld(r, b0 + D / 4), ld(r + 1, b0 + D / 4)};
        vw[x][2 * p] = __builtin_bit_cast(uint32_t, lo);
        vw[x][2 * p + 1] = __builtin_bit_cast(uint32_t, hi);
      }
  } else {
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = L::V_OFF + x * 16 * L::CROWV +
                      L::code_off(L::CROWV, 4 * blk + i, wave * L::HBV + CB * col);
        if constexpr (CB == 8)
          vw[x][i] = *reinterpret_cast<const uint2*>(buf + o);
        else if constexpr (CB == 4)
          vw[x][i] = *reinterpret_cast<const uint32_t*>(buf + o);
        else
          vw[x][i] = *reinterpret_cast<const uint16_t*>(buf + o);
      }
  }
  (void)tb;
  (void)t_end;
}

// One tile, software-pipelined with the previous one: start the copy of tile
// i + NBUF - 1 into `nxt` (the buffer tile i - 1 used), read this wave's
// slice of tile i from `cur`, then QK and scores of tile i next to PV of tile
// i - 1 (independent work for the matrix cores while the VALU converts and
// scales), tile i's V into the registers that PV has just consumed, the
// running-max update, and P' of tile i, which PV consumes in the next call.
// Every head set runs the same steps on the same staged data.  Ends with a
// wait for this wave's copies of tile i + 1 and a block barrier, after which
// every wave's copies of tile i + 1 have landed.
template <class L, int D, int NSET, bool MASK, bool PV_PREV, class WS>
__device__ __forceinline__ void coop_tile(WS (&W)[NSET], const CoopAddr& C, int i, int ntiles,
                                          int t_begin, int t_end, int wave, int col, int blk,
                                          const uint8_t* cur, uint8_t* nxt,
                                          typename WS::VWord (&vw)[2][4],
                                          h8 (&ahi)[NSET], h8 (&alo)[NSET], PageWindow& PW,
                                          int lane) {
  constexpr int NBUF = L::NBUF;
  const int tb = t_begin + 32 * i;
  // `nxt` was last read by tile i - 1, before the previous barrier
  if (i + NBUF - 1 < ntiles) coop_issue<L>(C, PW, lane, wave, tb + 32 * (NBUF - 1), t_end, nxt);
  typename WS::ST st[2];
  coop_read<L, WS::KZ_USED, WS::VZ_USED>(cur, wave, col, blk, st);
  bool valid[2] = {true, true};
  if constexpr (MASK) {
    valid[0] = tb + col < t_end;
    valid[1] = tb + 16 + col < t_end;
  }
  float score[NSET][2][WS::GPL];
#pragma unroll
  for (int s = 0; s < NSET; ++s) W[s].template scores<MASK>(st, valid, score[s]);
  if constexpr (PV_PREV) {
#pragma unroll
    for (int s = 0; s < NSET; ++s) {
      if constexpr (WS::PAIRS_OK && NSET == 1)
        W[s].template pv_columns<true>(vw, ahi[s], alo[s]);
      else
        W[s].pv_columns(vw, ahi[s], alo[s]);
    }
  }
  // tile i's V replaces tile i - 1's in place once its PV has consumed it
  coop_read_v<L, D, WS::PAIRS_OK && NSET == 1, MASK>(cur, wave, col, blk, vw, tb, t_end);
  _Float16 sv[2][WS::NGV];
  const float svmax = W[0].template vscales<MASK>(st, valid, sv);
#pragma unroll
  for (int s = 0; s < NSET; ++s) {
    if (W[s].slow_tile(score[s], svmax)) W[s].slow_step(score[s], svmax);
    W[s].template probs<MASK, WS::PAIRS_OK && NSET == 1>(st, valid, score[s], sv, ahi[s],
                                                          alo[s]);
  }
  // copies issued after tile i + 1's: tiles i + 2 .. min(i + NBUF - 1, ntiles - 1)
  wait_tile_copies<L>(min(NBUF - 2, ntiles - 2 - i), C);
  __syncthreads();
}

// Tiles of 32 tokens in each row of sequence s: ceil(min(seq_len, max_context) / 32).
__device__ __forceinline__ uint32_t seq_tiles(int len, int max_context) {
  return static_cast<uint32_t>(max(0, min(len, max_context)) + 31) / 32;
}

// Inclusive prefix sum over the 64 lanes of a wave by DPP (row_shr within
// rows of 16 lanes, then row_bcast:15 / row_bcast:31 carry the row totals
// into the rows above), all in VALU: no LDS round trips.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  int v = static_cast<int>(x);
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);    // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);    // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);    // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);    // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);   // row_bcast:15, rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);   // row_bcast:31, rows 2, 3
  return static_cast<uint32_t>(v);
}

// floor(x T / Pe) for 0 <= x <= Pe <= 2^16: with T = q Pe + r, that is
// x q + floor(x r / Pe), x r < 2^32.  Two 32-bit divisions when T fits 32
// bits (a 64-bit division is a long dependent sequence, and the stream
// schedule's start runs several before its first copy).
__device__ __forceinline__ uint64_t share_bound(uint32_t x, uint64_t T, uint32_t Pe) {
  uint64_t q;
  uint32_t r;
  if ((T >> 32) == 0) {
    const uint32_t t = static_cast<uint32_t>(T);
    q = t / Pe;
    r = t - static_cast<uint32_t>(q) * Pe;
  } else {
    q = T / Pe;
    r = static_cast<uint32_t>(T - q * Pe);
  }
  return x * q + (x * r) / Pe;
}

// The block holding flattened position t < T of the stream schedule: the b
// with floor(b T / Pe) <= t < floor((b + 1) T / Pe), i.e.
// floor((t Pe + Pe - 1) / T).  For T < 2^32 and Pe <= 2^16 the numerator
// (< 2^48) and T are exact in fp64 and the quotient is below 2^16, so the
// correctly rounded fp64 quotient cannot cross an integer: the floor is
// exact.
__device__ __forceinline__ int block_of_position(uint64_t t, uint64_t T, uint32_t Pe) {
  const uint64_t num = t * Pe + Pe - 1;
  if ((T >> 32) == 0)
    return static_cast<int>(__builtin_floor(static_cast<double>(num) / static_cast<double>(T)));
  return static_cast<int>(num / T);
}

// Where a stream-schedule block starts: the sequence s holding flattened
// position f (rows of sequence s are cost + n_s positions long, nhg rows per
// sequence, laid end to end in sequence order), its first position sbase,
// n_s and its length; and T, all rows' positions.  The lengths of up to 64
// KMAX sequences are loaded at once and scanned 64 at a time; nothing here
// stays live in the segment loop.  Position counts fit 32 bits:
// num_seqs * (ceil(max_context / 32) + cost) < 2^31.
struct StreamStart {
  static constexpr int KMAX = 16;    // up to 1024 sequences
  uint64_t T, sbase;
  uint32_t n, cost;
  int s, len, Pe;

  // The length scan below in chunks of 64 sequences: KN = 1 (up to 64
  // sequences) or KMAX.  Its loops are unrolled over KN chunks, and each
  // chunk's loads and scans run whether or not the chunk holds a sequence:
  // at config 2 on the stream schedule one chunk takes the kernel from entry
  // to its first segment in 2.0 us where sixteen took 3.7 (the partial 57.8
  // -> 56.3 us, config 3's 109.3 -> 107.8 us).
  __device__ __forceinline__ void find(const DecodeArgs& a, int nhg, int b, int P, int lane,
                                       uint64_t* f0, uint64_t* f1) {
    if (a.num_seqs <= kWave)
      find_n<1>(a, nhg, b, P, lane, f0, f1);
    else
      find_n<KMAX>(a, nhg, b, P, lane, f0, f1);
  }

  template <int KN>
  __device__ __forceinline__ void find_n(const DecodeArgs& a, int nhg, int b, int P, int lane,
                                         uint64_t* f0, uint64_t* f1) {
    const int nk = (a.num_seqs + kWave - 1) / kWave;
    int len_k[KN];
#pragma unroll
    for (int k = 0; k < KN; ++k) {
      const int i = kWave * k + lane;
      len_k[k] = (k < nk && i < a.num_seqs) ? a.seq_lens[i] : 0;
    }
    // all rows' tiles (nhg rows per sequence), and whether every non-empty
    // sequence has the same tile count (that of lane 0's first non-empty one)
    uint32_t incl[KN];
    uint64_t tiles = 0;
    uint32_t nonempty = 0, tref = 0;
    bool ragged = false;
#pragma unroll
    for (int k = 0; k < KN; ++k) {
      incl[k] = 0;
      if (k < nk) {                                           // uniform
        const uint32_t t = seq_tiles(len_k[k], a.max_context);
        incl[k] = wave_incl_scan(t);
        tiles += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl[k]), 63));
        const uint64_t some = __ballot(t > 0);
        nonempty += static_cast<uint32_t>(__popcll(some));
        if (tref == 0 && some != 0)
          tref = static_cast<uint32_t>(
              __builtin_amdgcn_readlane(static_cast<int>(t), static_cast<int>(__builtin_ctzll(some))));
        ragged |= __any(t > 0 && t != tref);
      }
    }
    // Each row after a block's first costs the block its first loads and a
    // refill of its copy pipeline: a row is laid out as `cost` charged
    // positions then its n tiles, and blocks take equal shares of positions.
    // Charged only when every block's share exceeds `cost` positions (so every
    // block holds a tile, and holds no row's charged positions alone), and
    // only when some row would start inside a block's share: equal rows whose
    // count divides the blocks taking part start on share boundaries, each
    // block then holds tiles of one row (split-K's partition of a uniform
    // batch), and charges would only move the boundaries off the rows (config
    // 2 through the stream schedule: 59.7 us with charges, 58.6 without).
    const uint64_t T0 = static_cast<uint64_t>(nhg) * tiles;
    const uint32_t rows = static_cast<uint32_t>(nhg) * nonempty;
    const uint32_t Pe0 = static_cast<uint32_t>(min(static_cast<uint64_t>(P), T0));
    const bool aligned = !ragged && rows > 0 && Pe0 % rows == 0;
    cost = !aligned && T0 >= static_cast<uint64_t>(a.stream_row_cost + 1) * P
               ? static_cast<uint32_t>(a.stream_row_cost) : 0u;
    // inclusive prefix sums of the sequences' positions (tiles plus charges)
    uint64_t total = tiles;
    if (cost != 0) {
      total = 0;
#pragma unroll
      for (int k = 0; k < KN; ++k) {
        if (k < nk) {
          const uint32_t t = seq_tiles(len_k[k], a.max_context);
          incl[k] = wave_incl_scan(t > 0 ? t + cost : 0u);
          total += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl[k]), 63));
        }
      }
    }
    T = static_cast<uint64_t>(nhg) * total;
    // Pe = min(P, T) blocks take part, each at least one tile, so the blocks
    // holding one row's tiles are consecutive with no idle block among them
    // (the merge reads one entry per block from a row's first block on)
    Pe = static_cast<int>(min(static_cast<uint64_t>(P), T));
    *f0 = *f1 = 0;
    if (b >= Pe) return;
    const uint64_t f = share_bound(static_cast<uint32_t>(b), T, static_cast<uint32_t>(Pe));
    // the chunk holding f, then the lane within it
    uint64_t acc = 0;
    int kstar = 0;
#pragma unroll
    for (int k = 0; k < KN; ++k) {
      const uint64_t csum =
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl[k]), 63));
      if (k == kstar && k + 1 < nk && static_cast<uint64_t>(nhg) * (acc + csum) <= f) {
        acc += csum;
        kstar = k + 1;
      }
    }
    int lk = 0;
    uint32_t ik = 0;
#pragma unroll
    for (int k = 0; k < KN; ++k) {
      if (k == kstar) {
        lk = len_k[k];
        ik = incl[k];
      }
    }
    // lanes whose sequence's rows all end at or before f: a prefix of the chunk
    const int c = __popcll(__ballot(static_cast<uint64_t>(nhg) * (acc + ik) <= f));
    if (c >= kWave) return;                                   // (cannot happen: f < T)
    s = kWave * kstar + c;
    len = __builtin_amdgcn_readlane(lk, c);
    n = seq_tiles(len, a.max_context);
    if (s >= a.num_seqs || n == 0) return;                    // (cannot happen either)
    sbase = static_cast<uint64_t>(nhg) *
            (acc + static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ik), c)) -
             (n + cost));
    *f0 = f;
    *f1 = share_bound(static_cast<uint32_t>(b + 1), T, static_cast<uint32_t>(Pe));
  }
};

// One block per CU (8 waves), L::NBUF tile buffers of LDS: the copies run
// NBUF - 1 tiles ahead of the compute.  K8: INT8 K codes with NGK scale
// groups; NSET head sets per wave.
//
// Schedules.  Split (a.stream == 0): block (split, seq, head group) runs the
// tokens [split * split_tokens, ...) of one sequence.  Stream (a.stream = P):
// the grid is one block per CU, and block b < Pe = min(P, T) runs the
// positions [b T / Pe, (b + 1) T / Pe) of all (sequence, head group) rows laid
// end to end, each row a charge of `cost` positions (no work: what starting
// a row costs a block) then its tiles of 32 tokens (T positions in all):
// equal work per block whatever the sequence lengths, one partial per
// (block, row) segment, at entry (b + row) * HG + head, a number no two
// segments share (b + row is strictly increasing along the flattened rows).
// The block holding a row's first tile writes, for each q head of the row,
// its first entry and the count of blocks holding the row's tiles for the
// merge.

// ---------------------------------------------------------------------------
// Wide query groups: 5 <= G <= 8 query heads per kv head over INT8 K with one
// scale per row and packed INT4 V at D = 128 (config 5: G = 5, V g32).  With
// rows (head, V group) these shapes need two head sets of 16 rows (20 rows
// at G = 5, the second set using 4 of its 16) and 32 PV products per tile.
// Here one set serves every head:
//  QK  rows r = 2 g + dup, both rows of head g carrying all of q (one K scale
//      per token, so no row needs a part of q): the output lane (token col,
//      blk) holds heads 2 blk and 2 blk + 1 in its rows 0 and 2.
//  PV  products by 32-column blocks m and nibble h: lane col of product
//      (m, h) is column 32 m + 2 col + h (nibble h of byte 16 m + col), so
//      every product lies inside V group vg(m), and its A operand A_vg has
//      rows (g, hi / lo) of P' = p s_v[vg]: a lane's (head 2 blk, head
//      2 blk + 1) x (hi, lo) are the slots 0-3 of one identity transpose,
//      whose output row is 2 g + hl.  8 PV products and 8 transposes per
//      tile whatever G (two head sets: 32 products, or 16 with group pairs).
//  V   read from LDS as byte pairs: byte 16 m + col of two tokens in the two
//      halves of a dword, one mask per nibble (kNib1 / kNib16).
// ---------------------------------------------------------------------------
//
// K INT4 in two scale groups (D = 128, g64; V then has the same two groups)
// fits the same lane layout: QK rows (g, K group) are 2 g + kg, as in
// WaveState with NG = 2, so only the PV differs from WaveState there.
template <int NGV, bool VASYM, bool K8 = true, bool KASYM = false>
struct WaveStateW {
  static constexpr int NCH = 4;                 // D = 128
  static constexpr int GPL = 2;                 // heads per lane
  static constexpr int KCH = K8 ? 8 : 4;        // K code dwords per lane and token
  static constexpr int NGK = K8 ? 1 : 2;        // K scale groups
  static_assert(K8 ? !KASYM : NGV == 2, "INT8 K per row, or INT4 K in V's two groups");
  using ST = SubTile<4, NGV, KCH, NGK, 4>;
  h8 aq[NCH];          // q rows 2g + part (A operands of QK)
  f4 cinit;            // QK accumulator start: -bias * 2^-24 * sum(q over the row)
  float qsum24[4];     // 2^-24 * sum(q) of rows 4 blk + i (asymmetric INT4 K)
  h4 eye;              // identity, B operand of the P' transposes
  f4 acc[4][2];        // [column block m][nibble h]: rows (g, hi/lo)
  float m_run[GPL], lsum[GPL], sl2[GPL], thr[GPL];
  float zacc[GPL][NGV];
  float kexp, svlim;

  __device__ static constexpr int vg_of(int m) { return m * NGV / 4; }

  template <bool MASK>
  __device__ __forceinline__ void scores(const ST (&st)[2], const bool (&valid)[2],
                                         float (&score)[2][GPL]) const {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      f4 S = KASYM ? f4{0.f, 0.f, 0.f, 0.f} : cinit;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        S = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            aq[c],
            K8 ? bytes_to_h8_sub(st[x].k.dw(2 * c), st[x].k.dw(2 * c + 1))
               : nibbles_to_h8_sub(st[x].k.dw(c)),
            S, 0, 0, 0);
#pragma unroll
      for (int gi = 0; gi < GPL; ++gi) {
        float sc;
        if constexpr (K8) {
          sc = st[x].ks.get(0) * S[2 * gi];            // rows 2 gi, 2 gi + 1 are equal
        } else {
          sc = 0.0f;
#pragma unroll
          for (int kg = 0; kg < 2; ++kg) {
            if constexpr (KASYM) sc = fmaf(st[x].kz.get(kg), qsum24[2 * gi + kg], sc);
            sc = fmaf(st[x].ks.get(kg), S[2 * gi + kg], sc);
          }
        }
        score[x][gi] = (MASK && !valid[x]) ? -INFINITY : sc;
      }
    }
  }

  // V scales in fp16 (0 past the end) and their largest value.
  template <bool MASK>
  __device__ __forceinline__ float vscales(const ST (&st)[2], const bool (&valid)[2],
                                           _Float16 (&sv)[2][NGV]) const {
    float m = 0.0f;
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int g = 0; g < NGV; ++g) {
        sv[x][g] = st[x].vs.geth(g);
        if constexpr (MASK) sv[x][g] = valid[x] ? sv[x][g] : static_cast<_Float16>(0.0f);
        m = fmaxf(m, static_cast<float>(sv[x][g]));
      }
    return m;
  }

  __device__ __forceinline__ bool slow_tile(const float (&score)[2][GPL], float svmax) const {
    bool up = svmax > svlim;
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) up |= fmaxf(score[0][gi], score[1][gi]) > m_run[gi] + thr[gi];
    return __any(up);
  }

  // As WaveState::slow_step: raise the running maxima that moved, lower k
  // for a larger V scale, rescale by both (powers of two for k).
  __device__ __forceinline__ void slow_step(const float (&score)[2][GPL], float svmax) {
    float smax = row_max16(svmax);
    smax = fmaxf(smax, __shfl_xor(smax, 16, kWave));
    smax = fmaxf(smax, __shfl_xor(smax, 32, kWave));
    int e = 0;
    frexpf(smax, &e);
    const float knew = fminf(kexp, static_cast<float>(12 - e));
    const float kscale = ldexpf(1.0f, static_cast<int>(knew - kexp));
    kexp = knew;
    svlim = ldexpf(1.0f, 12 - static_cast<int>(knew));
    float alpha[GPL];
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) {
      const float tmax = row_max16(fmaxf(score[0][gi], score[1][gi]));
      const bool up = tmax > m_run[gi] + thr[gi];
      alpha[gi] = (up ? __builtin_amdgcn_exp2f((m_run[gi] - tmax) * sl2[gi]) : 1.0f) * kscale;
      m_run[gi] = up ? tmax : m_run[gi];
    }
#pragma unroll
    for (int gi = 0; gi < GPL; ++gi) {
      lsum[gi] *= alpha[gi];
#pragma unroll
      for (int g = 0; g < NGV; ++g) zacc[gi][g] *= alpha[gi];
    }
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[m][h][i] *= alpha[i / 2];
  }

  // p (times 2^k), P' = p s_v[vg] as fp16 hi + lo, the zero-point term, and
  // for each V group the PV A operand (rows 2g + hl, slots = tokens).
  template <bool MASK>
  __device__ __forceinline__ void probs(const ST (&st)[2], const bool (&valid)[2],
                                        const float (&score)[2][GPL],
                                        const _Float16 (&svt)[2][NGV], h8 (&aw)[NGV]) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      float p[GPL];
#pragma unroll
      for (int gi = 0; gi < GPL; ++gi) {
        p[gi] = __builtin_amdgcn_exp2f(fmaf(score[x][gi] - m_run[gi], sl2[gi], kexp));
        lsum[gi] += p[gi];
      }
#pragma unroll
      for (int g = 0; g < NGV; ++g) {
        const float sv = static_cast<float>(svt[x][g]);
        const float P0 = fmaf(p[0], sv, 0.0f), P1 = fmaf(p[1], sv, 0.0f);
        if constexpr (VASYM) {
          float zv = st[x].vz.get(g);
          if constexpr (MASK) zv = valid[x] ? zv : 0.0f;
          zacc[0][g] = fmaf(p[0], zv, zacc[0][g]);
          zacc[1][g] = fmaf(p[1], zv, zacc[1][g]);
        } else {
          zacc[0][g] = fmaf(-8.0f, P0, zacc[0][g]);
          zacc[1][g] = fmaf(-8.0f, P1, zacc[1][g]);
        }
        const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(P0, P1));
        const float r0 = fmaf(p[0], sv, -static_cast<float>(hi[0]));
        const float r1 = fmaf(p[1], sv, -static_cast<float>(hi[1]));
        const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(r0, r1));
        // slots 0-3: (head 2 blk, hi), (2 blk, lo), (2 blk + 1, hi), (2 blk + 1, lo)
        const h4 xin = {hi[0], lo[0], hi[1], lo[1]};
        const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
        const f4 t = __builtin_amdgcn_mfma_f32_16x16x16f16(xin, eye, zero4, 0, 0, 0);
        const h2 t01 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(t[0], t[1]));
        const h2 t23 = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(t[2], t[3]));
        aw[g][4 * x + 0] = t01[0]; aw[g][4 * x + 1] = t01[1];
        aw[g][4 * x + 2] = t23[0]; aw[g][4 * x + 3] = t23[1];
      }
    }
  }

  // PV: vb[m][q] holds byte 16 m + col of tokens (t0, t0 + 1) in its two
  // halves, t0 = 16 (q / 2) + 4 blk + 2 (q % 2): the tokens of A slots 2q,
  // 2q + 1.  Nibble h of those bytes is column 32 m + 2 col + h.
  __device__ __forceinline__ void pv(const uint32_t (&vb)[4][4], const h8 (&aw)[NGV]) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u4 bw;
#pragma unroll
        for (int q = 0; q < 4; ++q) bw[q] = vb[m][q] & (h ? kNib16 : kNib1);
        acc[m][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[vg_of(m)],
                                                           __builtin_bit_cast(h8, bw), acc[m][h],
                                                           0, 0, 0);
      }
  }
};

// q rows (two per head), constants and accumulators of the wave serving kv
// head `kvh` with all its G <= 8 query heads (qw from load_q<128, 2>: lane
// (col, blk) holds elements 32 blk .. 32 blk + 31 of head col / 2).  INT8 K:
// both rows of a head carry all of q; INT4 K: row 2 g + kg carries the
// elements of K group kg (the lane's elements, 32 blk .. 32 blk + 31, lie in
// group blk / 2), in the nibble slot order with q / 16 facing odd nibbles.
template <int NGV, bool VASYM, bool K8, bool KASYM>
__device__ __forceinline__ void init_wave_w(WaveStateW<NGV, VASYM, K8, KASYM>& W,
                                            const uint4 (&qw)[4], const DecodeArgs& a, int col,
                                            int blk) {
  const bool qneg = a.scale_log2 < 0.0f;
  const bool qzero = a.scale_log2 == 0.0f;
  const bool on = col < 2 * a.group && !qzero && (K8 || blk / 2 == col % 2);
  uint16_t qv[32];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t ws[4] = {qw[i].x, qw[i].y, qw[i].z, qw[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qv[8 * i + 2 * j] = static_cast<uint16_t>(ws[j]);
      qv[8 * i + 2 * j + 1] = static_cast<uint16_t>(ws[j] >> 16);
    }
  }
  float qscale = 1.0f;
  if (a.q_bf16) {
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(bf16_bits_to_float(qv[i])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    int ex = 0;
    frexpf(mx, &ex);
    qscale = mx > 0.0f ? ldexpf(1.0f, 14 - ex) : 1.0f;
  }
  float qpart = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int el = 8 * c + (K8 ? kByteK8[e] : kNibK[e]);
      _Float16 v = !on ? _Float16(0)
                   : a.q_bf16 ? static_cast<_Float16>(bf16_bits_to_float(qv[el]) * qscale)
                              : __builtin_bit_cast(_Float16, qv[el]);
      if (qneg) v = -v;
      W.aq[c][e] = (!K8 && (e & 2)) ? v * static_cast<_Float16>(0.0625f) : v;
      qpart += static_cast<float>(v);
    }
  qpart += __shfl_xor(qpart, 16, kWave);
  qpart += __shfl_xor(qpart, 32, kWave);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    W.qsum24[i] = __shfl(qpart, 4 * blk + i, kWave) * 0x1p-24f;
    W.cinit[i] = KASYM ? 0.0f : (K8 ? -128.0f : -8.0f) * W.qsum24[i];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) W.eye[e] = (blk == col / 4 && e == col % 4) ? 1.0f : 0.0f;
#pragma unroll
  for (int m = 0; m < 4; ++m) W.acc[m][0] = W.acc[m][1] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    W.m_run[gi] = -INFINITY;
    W.lsum[gi] = 0.0f;
#pragma unroll
    for (int g = 0; g < NGV; ++g) W.zacc[gi][g] = 0.0f;
    const float qs = __shfl(qscale, 4 * blk + 2 * gi, kWave);
    W.sl2[gi] = (qzero ? 1.0f : fabsf(a.scale_log2)) * 0x1p24f / qs;
    W.thr[gi] = kRescaleLog2 / W.sl2[gi];
  }
  W.kexp = 40.0f;
  W.svlim = 0x1p-28f;
}

// The wave's partial (acc, max, sum) for each of its kv head's G query heads
// at entry base + g * stride.
template <int NGV, bool VASYM, bool K8, bool KASYM>
__device__ __forceinline__ void write_partials_w(WaveStateW<NGV, VASYM, K8, KASYM>& W,
                                                 const DecodeArgs& a, int64_t base, int64_t stride,
                                                 int col, int blk) {
  const int G = a.group;
  const float kinv = ldexpf(1.0f, -static_cast<int>(W.kexp));
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    W.lsum[gi] = row_sum16(W.lsum[gi]) * kinv;
#pragma unroll
    for (int g = 0; g < NGV; ++g) W.zacc[gi][g] = row_sum16(W.zacc[gi][g]);
  }
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    const int g = 2 * blk + gi;
    if (g < G) {
      const int64_t row = base + g * stride;
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const f4 v = W.acc[m][h];
          const float hl = gi ? v[2] + v[3] : v[0] + v[1];
          // high nibbles arrive as 16 n: a factor 16 fewer
          a.part_o[row * 128 + 32 * m + 2 * col + h] =
              fmaf(hl, h ? 0x1p20f : 0x1p24f, W.zacc[gi][W.vg_of(m)]) * kinv;
        }
      if (col == 0) {
        a.part_ml[2 * row] = W.m_run[gi] * W.sl2[gi];
        a.part_ml[2 * row + 1] = W.lsum[gi];
      }
    }
  }
}

// V of this wave's head as byte pairs (WaveStateW::pv): vb[m][q] = byte
// 16 m + col of tokens t0 and t0 + 1, t0 = 16 (q / 2) + 4 blk + 2 (q % 2).
template <class L>
__device__ __forceinline__ void coop_read_v_w(const uint8_t* buf, int wave, int col, int blk,
                                              uint32_t (&vb)[4][4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint8_t* sub = buf + L::V_OFF + (q / 2) * 16 * L::CROWV;
    const int r0 = 4 * blk + 2 * (q % 2);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int byte = wave * L::HBV + 16 * m + col;
      const uint32_t b0 = sub[L::code_off(L::CROWV, r0, byte)];
      const uint32_t b1 = sub[L::code_off(L::CROWV, r0 + 1, byte)];
      vb[m][q] = b0 | (b1 << 16);
    }
  }
}

// One tile of the wide-group kernel, pipelined as coop_tile: copies of tile
// i + NBUF - 1, this wave's slice of tile i, QK of tile i next to PV of tile
// i - 1, tile i's V into the registers PV has consumed, then P' of tile i.
template <class L, int NGV, bool VASYM, bool K8, bool KASYM, bool MASK, bool PV_PREV>
__device__ __forceinline__ void coop_tile_w(WaveStateW<NGV, VASYM, K8, KASYM>& W, const CoopAddr& C,
                                            int i,
                                            int ntiles, int t_begin, int t_end, int wave, int col,
                                            int blk, const uint8_t* cur, uint8_t* nxt,
                                            uint32_t (&vb)[4][4], h8 (&aw)[NGV], PageWindow& PW,
                                            int lane) {
  using WS = WaveStateW<NGV, VASYM, K8, KASYM>;
  constexpr int NBUF = L::NBUF;
  const int tb = t_begin + 32 * i;
  if (i + NBUF - 1 < ntiles) coop_issue<L>(C, PW, lane, wave, tb + 32 * (NBUF - 1), t_end, nxt);
  typename WS::ST st[2];
  coop_read<L, KASYM, VASYM>(cur, wave, col, blk, st);
  bool valid[2] = {true, true};
  if constexpr (MASK) {
    valid[0] = tb + col < t_end;
    valid[1] = tb + 16 + col < t_end;
  }
  float score[2][WS::GPL];
  W.template scores<MASK>(st, valid, score);
  if constexpr (PV_PREV) W.pv(vb, aw);
  coop_read_v_w<L>(cur, wave, col, blk, vb);
  _Float16 sv[2][NGV];
  const float svmax = W.template vscales<MASK>(st, valid, sv);
  if (W.slow_tile(score, svmax)) W.slow_step(score, svmax);
  W.template probs<MASK>(st, valid, score, sv, aw);
  wait_tile_copies<L>(min(NBUF - 2, ntiles - 2 - i), C);
  __syncthreads();
}

// One segment: tokens [t_begin, t_begin + seg_tokens) (cut at the sequence's
// length) of sequence `seq`, kv heads 8 hg .. 8 hg + 7.  seq_len < 0: load it
// here (together with q and the block table).  Partial of head set s, query
// head g of this wave at entry base(s) + g * stride, base(s) = base0 +
// s * heads_per_set.  Returns without work (uniformly) when the segment is
// empty.
// WIDE: the wide-group wave state (WaveStateW: one set for 5 <= G <= 8,
// INT8 K with one scale per row, INT4 V with NG groups, D = 128).  K16 / V16:
// fp16 K (4 kv heads per block) / fp16 V.  FEW: waves 0-3 issue every tile
// copy (CoopLayout).
template <int D, int NG, bool KASYM, bool VASYM, bool K8, int NGK, int NSET, bool V8,
          bool WIDE = false, bool K16 = false, bool V16 = false, bool FEW = false>
__device__ __forceinline__ void coop_segment(
    const DecodeArgs& a,
    uint8_t (&lds)[CoopLayout<D, NG, K8, NGK, V8, K16, V16>::NBUF]
                  [CoopLayout<D, NG, K8, NGK, V8, K16, V16>::BYTES],
    int seq, int hg, int t_begin, int seg_tokens, int seq_len_known, int64_t base0,
    int64_t stride) {
  using L = CoopLayout<D, NG, K8, NGK, V8, K16, V16, FEW>;
  constexpr int NCH = D / 32;
  constexpr int KCH = K16 ? 4 * NCH : K8 ? 2 * NCH : NCH;
  constexpr int NBUF = L::NBUF;
  constexpr int KEB = K16 ? 2 : 1;    // bytes per element of the K / V arrays
  constexpr int VEB = V16 ? 2 : 1;    // (their strides are in elements)
  using WS = WaveState<NCH, NG, KASYM, VASYM, KCH, NGK, V8, V16>;
  // An opaque thread index: the stream schedule runs this once per segment
  // in a loop, and lane-derived set-up hoisted out of that loop would stay
  // live in VGPRs through every segment's tile loop (+50 VGPRs, and spills
  // with two head sets); recomputing it per segment costs a few VALU.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & (kWave - 1);
  const int col = lane & 15;
  const int blk = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int h0 = hg * L::kHeads;
  const int kvh = h0 + wave;
  CoopAddr C;
  {
    const knlp_kv_plane& K = a.kp;
    const knlp_kv_plane& V = a.vp;
    C.kc = static_cast<const uint8_t*>(K.data) + KEB * h0 * K.stride_head;
    C.vc = static_cast<const uint8_t*>(V.data) + VEB * h0 * V.stride_head;
    C.kc_b = static_cast<uint32_t>(KEB * K.stride_block);
    C.kc_p = static_cast<uint32_t>(KEB * K.stride_page);
    C.vc_b = static_cast<uint32_t>(VEB * V.stride_block);
    C.vc_p = static_cast<uint32_t>(VEB * V.stride_page);
    C.same_kv = C.kc_b == C.vc_b && C.kc_p == C.vc_p;
    // code copy: lane -> LDS byte part*1024 + 16*lane of a sub-tile, which
    // holds logical chunk (physical chunk) ^ row of that row; a copying
    // wave's parts are (wave >> 1) + WPS k
#pragma unroll
    for (int k = 0; k < L::NPWK; ++k) {
      const int byte = ((wave >> 1) + L::WPS * k) % L::CPSK * 1024 + 16 * lane;
      const int r = byte / L::CROWK;
      const int c = ((byte % L::CROWK) >> 4) ^ r;
      C.lk[k] = static_cast<uint32_t>(r * C.kc_p + 16 * c);
    }
#pragma unroll
    for (int k = 0; k < L::NPWV; ++k) {
      const int byte = ((wave >> 1) + L::WPS * k) % L::CPSV * 1024 + 16 * lane;
      const int r = byte / L::CROWV;
      const int c = ((byte % L::CROWV) >> 4) ^ r;
      C.lv[k] = static_cast<uint32_t>(r * C.vc_p + 16 * c);
    }
    // copying wave w copies scale arrays L::s_array(w, j) (ks, vs, kz, vz)
    // of sub-tile w % 2
    C.copier = L::ALL || wave < L::NCW;
    C.x = wave & 1;
    const auto scale_addr = [&](CoopScale& S, int arr) {
      const uint16_t* base = arr == 0 ? static_cast<const uint16_t*>(K.scales)
                           : arr == 1 ? static_cast<const uint16_t*>(V.scales)
                           : arr == 2 ? static_cast<const uint16_t*>(K.zeros)
                                      : static_cast<const uint16_t*>(V.zeros);
      const int64_t sh = arr == 0 ? K.s_stride_head : arr == 1 ? V.s_stride_head
                       : arr == 2 ? K.z_stride_head : V.z_stride_head;
      const int64_t sbk = arr == 0 ? K.s_stride_block : arr == 1 ? V.s_stride_block
                        : arr == 2 ? K.z_stride_block : V.z_stride_block;
      const int64_t spg = arr == 0 ? K.s_stride_page : arr == 1 ? V.s_stride_page
                        : arr == 2 ? K.z_stride_page : V.z_stride_page;
      // (fp16 planes have no scales or zero-points)
      const bool arr_on = C.copier && ((arr == 0 && !K16) || (arr == 1 && !V16) ||
                                       (arr == 2 && KASYM) || (arr == 3 && VASYM));
      const int srow = L::s_row(arr);
      S.on = arr_on;
      S.lane_on = arr_on && lane < srow;
      S.sp = arr_on ? reinterpret_cast<const uint8_t*>(base + h0 * sh) : nullptr;
      S.sp_b = static_cast<uint32_t>(2 * sbk);
      S.sp_p = static_cast<uint32_t>(2 * spg);
      S.ls = 0;
      if (arr_on) {
        const int byte = 16 * lane;
        const int r = byte / srow;
        const int c = ((byte % srow) >> 4) ^ L::scale_swz(srow, r);
        S.ls = static_cast<uint32_t>(r * S.sp_p + 16 * c);
      }
      S.lds = L::s_off(arr) + C.x * 16 * srow;
    };
    scale_addr(C.s0, L::s_array(wave, 0));
    C.nsc = C.s0.on ? 1 : 0;
    if constexpr (L::NSA == 2) {
      scale_addr(C.s1, L::s_array(wave, 1));
      C.nsc += C.s1.on ? 1 : 0;
    }
    C.bt = a.block_table + seq * a.bt_stride;
    C.bs_shift = a.block_shift;
  }

  // First loads, issued together and waited for once: seq_lens (split
  // schedule), this lane's q and the block-table window (bounded by the
  // row's width, max_context, before seq_len is known: entries past the
  // sequence are read, never used).  Only then the tile copies, so no later
  // wait for these loads (whose counter the copies share) holds up the
  // copies in flight.
  const int seq_len_raw = seq_len_known >= 0 ? seq_len_known : a.seq_lens[seq];
  static_assert(!WIDE || (D == 128 && !V8 && NSET == 1 &&
                          (K8 ? NGK == 1 && !KASYM : NGK == 2 && NG == 2)),
                "the wide-group wave state's shapes");
  uint4 qw[NSET][D / 32];
  if constexpr (WIDE) {
    load_q<D, 2>(qw[0], a, seq, kvh, col, blk, 0);     // two rows per head, all of q
  } else {
#pragma unroll
    for (int s = 0; s < NSET; ++s)
      load_q<D, NG>(qw[s], a, seq, kvh, col, blk, s * heads_per_set<NG>());
  }
  PageWindow PW;
  PW.last = (a.max_context - 1) >> C.bs_shift;
  PW.fill(C.bt, lane, t_begin >> C.bs_shift);              // waits for all three
  // every exit below is uniform over the block: all waves reach every barrier
  const int seq_len = min(seq_len_raw, a.max_context);
  if (t_begin >= seq_len) return;
  const int t_end = min(seq_len, t_begin + seg_tokens);
  PW.last = (t_end - 1) >> C.bs_shift;
  // the token being decoded, when the caller fused its append into this launch;
  // the barrier orders every wave's rows before any wave copies the page
  decode_append_if<D>(a, seq, kvh, t_end == seq_len, lane);
  if (a.app.key != nullptr || a.app.value != nullptr) __syncthreads();

  const int ntiles = (t_end - t_begin + 31) / 32;
#pragma unroll
  for (int t = 0; t < NBUF - 1; ++t)
    if (t < ntiles) coop_issue<L>(C, PW, lane, wave, t_begin + 32 * t, t_end, lds[t]);
  const int nfull = (t_end - t_begin) / 32;
  if constexpr (WIDE) {
    WaveStateW<NG, VASYM, K8, KASYM> W;
    init_wave_w(W, qw[0], a, col, blk);
    wait_tile_copies<L>(min(NBUF - 2, ntiles - 1), C);
    __syncthreads();
    uint32_t vb[4][4];
    h8 aw[NG];
#define KNLP_COOP_TILE_W(MASK, PV_PREV)                                                     \
  coop_tile_w<L, NG, VASYM, K8, KASYM, MASK, PV_PREV>(W, C, i, ntiles, t_begin, t_end,      \
                                                      wave, col, blk,                      \
                                           lds[i % NBUF], lds[(i + NBUF - 1) % NBUF], vb,   \
                                           aw, PW, lane)
    int i = 0;
    if (nfull > 0) {
      KNLP_COOP_TILE_W(false, false);
      for (i = 1; i < nfull; ++i) KNLP_COOP_TILE_W(false, true);
      if (i < ntiles) KNLP_COOP_TILE_W(true, true);
    } else {
      KNLP_COOP_TILE_W(true, false);
    }
#undef KNLP_COOP_TILE_W
    W.pv(vb, aw);
    write_partials_w(W, a, base0, stride, col, blk);
    return;
  }
  // q -> matrix-core operands while the first tiles are in flight
  WS W[NSET];
#pragma unroll
  for (int s = 0; s < NSET; ++s)
    init_wave<D, NG, KASYM, VASYM, KCH, NGK, V8, V16>(W[s], qw[s], a, col, blk,
                                                      s * heads_per_set<NG>());
  wait_tile_copies<L>(min(NBUF - 2, ntiles - 1), C);
  __syncthreads();
  // tile 0 (no PV pending), full tiles, an optional partial last tile, and
  // the PV of the last tile
  typename WS::VWord vw[2][4];
  h8 ahi[NSET], alo[NSET];
#define KNLP_COOP_TILE(MASK, PV_PREV)                                                       \
  coop_tile<L, D, NSET, MASK, PV_PREV>(W, C, i, ntiles, t_begin, t_end, wave, col, blk,     \
                                       lds[i % NBUF], lds[(i + NBUF - 1) % NBUF], vw, ahi,  \
                                       alo, PW, lane)
  int i = 0;
  if (nfull > 0) {
    KNLP_COOP_TILE(false, false);
    for (i = 1; i < nfull; ++i) KNLP_COOP_TILE(false, true);
    if (i < ntiles) KNLP_COOP_TILE(true, true);
  } else {
    KNLP_COOP_TILE(true, false);
  }
#undef KNLP_COOP_TILE
#pragma unroll
  for (int s = 0; s < NSET; ++s) {
    constexpr bool PAIRS = std::remove_reference_t<decltype(W[s])>::PAIRS_OK && NSET == 1;
    if constexpr (PAIRS)
      W[s].template pv_columns<true>(vw, ahi[s], alo[s]);
    else
      W[s].pv_columns(vw, ahi[s], alo[s]);
    write_partials_at<D, NG, KASYM, VASYM, true, KCH, NGK, V8, V16, PAIRS>(
        W[s], a, base0 + s * heads_per_set<NG>() * stride, stride, col, blk,
        s * heads_per_set<NG>());
  }
}

// The stream schedule's walk over the flattened positions: the next position
// f, the block's end fe, all positions T, the current sequence s (its rows
// start at position sbase and are cost + n positions long, the charge then n
// tiles; len tokens) and the blocks taking part Pe.  Through each segment's tile loop it lives in the lanes of one VGPR
// (hold() returns it, field i in lane i): as uniform values the compiler would keep
// its 12 words in SGPRs, which the tile loop needs all of, or in 12 VGPRs,
// which a two-head-set tile loop does not have to spare; uniform() reads it
// back at segment boundaries.
struct StreamWalk {
  uint64_t f, fe, T, sbase;
  uint32_t n, cost;
  int s, len, Pe;

  // the walk in one VGPR, field i in lane i
  __device__ __forceinline__ uint32_t hold() const {
    const uint32_t w[13] = {static_cast<uint32_t>(f),     static_cast<uint32_t>(f >> 32),
                            static_cast<uint32_t>(fe),    static_cast<uint32_t>(fe >> 32),
                            static_cast<uint32_t>(T),     static_cast<uint32_t>(T >> 32),
                            static_cast<uint32_t>(sbase), static_cast<uint32_t>(sbase >> 32),
                            n, static_cast<uint32_t>(s), static_cast<uint32_t>(len),
                            static_cast<uint32_t>(Pe), cost};
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 13; ++i) v = lane == i ? w[i] : v;
    asm volatile("" : "+v"(v));     // opaque: reads below come from the VGPR
    return v;
  }
  __device__ __forceinline__ static StreamWalk uniform(uint32_t packed) {
    const auto lane = [&](int i) {
      return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(packed), i));
    };
    const auto u64 = [&](int i) { return (static_cast<uint64_t>(lane(i + 1)) << 32) | lane(i); };
    StreamWalk u;
    u.f = u64(0);
    u.fe = u64(2);
    u.T = u64(4);
    u.sbase = u64(6);
    u.n = lane(8);
    u.s = static_cast<int>(lane(9));
    u.len = static_cast<int>(lane(10));
    u.Pe = static_cast<int>(lane(11));
    u.cost = lane(12);
    return u;
  }
};

// The two schedules are separate kernels (each with its own register
// allocation: the stream loop's state would otherwise cost the split kernel
// registers through its whole tile loop).
template <bool STREAM, int D, int NG, bool KASYM, bool VASYM, bool K8, int NGK, int NSET, bool V8,
          bool WIDE, bool K16 = false, bool V16 = false>
__device__ __forceinline__ void coop_kernel_body(
    const DecodeArgs& a,
    uint8_t (&lds)[CoopLayout<D, NG, K8, NGK, V8, K16, V16>::NBUF]
                  [CoopLayout<D, NG, K8, NGK, V8, K16, V16>::BYTES]) {
  using L = CoopLayout<D, NG, K8, NGK, V8, K16, V16>;
  static_assert(!(K8 && KASYM) && !(V8 && VASYM), "INT8 codes are symmetric");
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  if constexpr (!STREAM) {
    const int split = blockIdx.x;
    const int seq = blockIdx.y;
    const int hg = blockIdx.z;
    const int64_t row0 = static_cast<int64_t>(seq) * a.num_q_heads + (hg * L::kHeads + wave) * a.group;
    // (four copying waves: shorter tile loops in every layout)
    coop_segment<D, NG, KASYM, VASYM, K8, NGK, NSET, V8, WIDE, K16, V16, true>(
        a, lds, seq, hg, split * a.split_tokens, a.split_tokens, -1,
        row0 * a.num_splits + split, a.num_splits);
  } else {
    // stream schedule
    uint32_t walk;                  // StreamWalk::hold(): the walk's state in one VGPR
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int b = blockIdx.x;
    {
      const int nhg = a.num_kv_heads / L::kHeads;
      if (b == 0 && threadIdx.x == 0) a.stream_hdr[0] = L::kHeads * a.group;
      StreamStart st;
      uint64_t f0, f1;
      st.find(a, nhg, b, gridDim.x, lane, &f0, &f1);
      if (f0 >= f1) return;                                   // uniform: no tiles here
      StreamWalk W;
      W.f = f0;
      W.fe = f1;
      W.T = st.T;
      W.sbase = st.sbase;
      W.n = st.n;
      W.s = st.s;
      W.len = st.len;
      W.Pe = st.Pe;
      W.cost = st.cost;
      walk = W.hold();
    }
    while (true) {                                            // uniform
      // this segment's uniform view of the walk
      const StreamWalk U = StreamWalk::uniform(walk);
      const int nhg = a.num_kv_heads / L::kHeads;
      const int HG = L::kHeads * a.group;
      const uint32_t nv = U.n + U.cost;                     // a row's positions
      // (a sequence's rows span nhg * nv < 2^32 positions)
      const int hg = static_cast<int>(static_cast<uint32_t>(U.f - U.sbase) / nv);
      if (hg >= nhg) break;                                   // (cannot happen)
      const uint64_t srow = U.sbase + static_cast<uint64_t>(hg) * nv;
      const uint64_t r0 = srow + U.cost;                      // the row's first tile
      const uint64_t send = min(U.fe, srow + nv);
      // the block's share ends among the row's charged positions: no tile of
      // it here (the next block starts the row)
      if (send <= r0) break;
      const int t0 = static_cast<int>(max(U.f, r0) - r0);
      const int t1 = static_cast<int>(send - r0);
      const int row = U.s * nhg + hg;
      if (t0 == 0 && static_cast<int>(threadIdx.x) < HG) {
        // the row's record, one per q head j: its first entry and the count
        // of blocks holding the row's tiles (the block holding flattened
        // position t: the b with floor(b T / Pe) <= t < floor((b + 1) T / Pe))
        const uint64_t tl = srow + nv - 1;
        const int j = threadIdx.x;
        int32_t* rec = a.row_meta + 2 * (static_cast<int64_t>(U.s) * a.num_q_heads + hg * HG + j);
        rec[0] = (b + row) * HG + j;
        rec[1] = block_of_position(tl, U.T, static_cast<uint32_t>(U.Pe)) - b + 1;
      }
      {
        StreamWalk N = U;
        N.f = send;
        walk = N.hold();
      }
      // the kernel arguments (the kernel's only argument, at offset 0 of the
      // kernarg segment) through a pointer the compiler cannot see through:
      // their loads stay in this iteration instead of being hoisted out of
      // the loop and held in SGPRs through every segment
      using KArgs = const __attribute__((address_space(4))) DecodeArgs;
      KArgs* kp = (KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
      asm volatile("" : "+s"(kp));
      const DecodeArgs& A = *(const DecodeArgs*)kp;
      // (four copying waves, as split-K)
      coop_segment<D, NG, KASYM, VASYM, K8, NGK, NSET, V8, WIDE, K16, V16, true>(
          A, lds, U.s, hg, 32 * t0, 32 * (t1 - t0), U.len,
          static_cast<int64_t>(b + row) * HG + wave * A.group, 1);
      StreamWalk V = StreamWalk::uniform(walk);
      if (V.f >= V.fe) break;
      __syncthreads();    // the next segment's copies reuse the tile buffers
      // past this sequence's rows: the next sequence with tiles (one exists,
      // since tiles remain before fe <= T)
      if (V.f == V.sbase + static_cast<uint64_t>(nhg) * (V.n + V.cost)) {
        V.sbase = V.f;
        V.n = 0;
        while (V.n == 0 && V.s + 1 < a.num_seqs) {
          ++V.s;
          V.len = a.seq_lens[V.s];
          V.n = seq_tiles(V.len, a.max_context);
        }
        if (V.n == 0) break;
      }
      walk = V.hold();
    }
  }
}

template <int D, int NG, bool KASYM, bool VASYM, bool K8, int NGK, int NSET, bool V8 = false,
          bool WIDE = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void decode_mfma_coop_kernel(DecodeArgs a) {
  using L = CoopLayout<D, NG, K8, NGK, V8>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[L::NBUF][L::BYTES];
  coop_kernel_body<false, D, NG, KASYM, VASYM, K8, NGK, NSET, V8, WIDE>(a, lds);
}

template <int D, int NG, bool KASYM, bool VASYM, bool K8, int NGK, int NSET, bool V8 = false,
          bool WIDE = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void decode_mfma_coop_stream_kernel(DecodeArgs a) {
  using L = CoopLayout<D, NG, K8, NGK, V8>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[L::NBUF][L::BYTES];
  coop_kernel_body<true, D, NG, KASYM, VASYM, K8, NGK, NSET, V8, WIDE>(a, lds);
}

// fp16 K (and fp16, INT4 or INT8 V) on the cooperative loader: 4 kv heads
// per block (one wave each), one block per CU, so a wave may use the whole
// register file of its SIMD lane.
template <int D, int NG, bool VASYM, bool V8, bool V16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
void decode_mfma_coop16_kernel(DecodeArgs a) {
  using L = CoopLayout<D, NG, false, NG, V8, true, V16>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[L::NBUF][L::BYTES];
  coop_kernel_body<false, D, NG, false, VASYM, false, NG, 1, V8, false, true, V16>(a, lds);
}

template <int D, int NG, bool VASYM, bool V8, bool V16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
void decode_mfma_coop16_stream_kernel(DecodeArgs a) {
  using L = CoopLayout<D, NG, false, NG, V8, true, V16>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[L::NBUF][L::BYTES];
  coop_kernel_body<true, D, NG, false, VASYM, false, NG, 1, V8, false, true, V16>(a, lds);
}

inline int heads_per_block_mfma(int num_kv_heads) {
  for (int h = 8; h >= 1; h >>= 1)
    if (num_kv_heads % h == 0) return h;
  return 1;
}

}  // namespace
}  // namespace knlp

namespace knlp {

// Launchers of the three kernel families (one translation unit each).
int launch_mfma_perhead(const DecodeArgs& a, int head_size, hipStream_t stream);
int launch_mfma_coop_split(const DecodeArgs& a, int head_size, hipStream_t stream);
int launch_mfma_coop_stream(const DecodeArgs& a, int head_size, hipStream_t stream);

}  // namespace knlp
