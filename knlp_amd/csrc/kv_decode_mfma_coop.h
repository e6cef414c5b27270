// Launches of the cooperative kernel (8 waves stage pages of 8 kv heads
// through LDS) for every format it takes, on either schedule: STREAM picks
// decode_mfma_coop_stream_kernel (one block per CU, equal tile shares) over
// decode_mfma_coop_kernel (split-K).  Included by kv_decode_mfma_coop.hip and
// kv_decode_mfma_stream.hip, one schedule each, so they compile in parallel.
#pragma once

#include "kv_decode_mfma.h"

namespace knlp {
namespace {

// fp16 K on the cooperative loader (4 kv heads per block): fp16 V, or INT4 /
// INT8 V in 2 or 4 scale groups with one head set, D = 128 (with one V scale
// per row the block's heads' scales of a token are 8 bytes, less than the
// 16-byte chunk a lane copies: the per-head kernel takes that shape).
template <bool STREAM>
int launch_coop16(const DecodeArgs& a, int head_size, hipStream_t stream) {
  if (head_size != 128) return KNLP_ERR_SHAPE;
  const int ng = a.vp.format == KNLP_KV_FP16 ? 1 : head_size / a.vp.group_size;
  const bool va = a.vp.format == KNLP_KV_INT4_ASYM;
  const bool v8 = a.vp.format == KNLP_KV_INT8_SYM;
  const bool v16 = a.vp.format == KNLP_KV_FP16;
  if (a.group * ng > 16) return KNLP_ERR_SHAPE;
  const dim3 grid = STREAM ? dim3(a.stream) : dim3(a.num_splits, a.num_seqs, a.num_kv_heads / 4);
  const dim3 block(kWave * 4);
#define KNLP_LAUNCH_COOP16(...)                                                            \
  do {                                                                                     \
    if constexpr (STREAM)                                                                  \
      hipLaunchKernelGGL((decode_mfma_coop16_stream_kernel<__VA_ARGS__>), grid, block, 0,  \
                         stream, a);                                                       \
    else                                                                                   \
      hipLaunchKernelGGL((decode_mfma_coop16_kernel<__VA_ARGS__>), grid, block, 0, stream, \
                         a);                                                               \
  } while (0)
  if (v16) KNLP_LAUNCH_COOP16(128, 1, false, false, true);
  else if (v8 && ng == 4) KNLP_LAUNCH_COOP16(128, 4, false, true, false);
  else if (v8) return KNLP_ERR_SHAPE;
  else if (ng == 4) { if (va) KNLP_LAUNCH_COOP16(128, 4, true, false, false);
                      else KNLP_LAUNCH_COOP16(128, 4, false, false, false); }
  else if (ng == 2) { if (va) KNLP_LAUNCH_COOP16(128, 2, true, false, false);
                      else KNLP_LAUNCH_COOP16(128, 2, false, false, false); }
  else return KNLP_ERR_SHAPE;
#undef KNLP_LAUNCH_COOP16
  return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
}

template <bool STREAM>
int launch_coop(const DecodeArgs& a, int head_size, hipStream_t stream) {
  if (a.kp.format == KNLP_KV_FP16) return launch_coop16<STREAM>(a, head_size, stream);
  const int ng = head_size / a.vp.group_size;
  const bool k8 = a.kp.format == KNLP_KV_INT8_SYM;
  const int ngk = head_size / a.kp.group_size;
  const bool ka = a.kp.format == KNLP_KV_INT4_ASYM;
  const bool va = a.vp.format == KNLP_KV_INT4_ASYM;
  const bool v8 = a.vp.format == KNLP_KV_INT8_SYM;
  const int nset = (a.group * ng + 15) / 16;
  const dim3 grid = STREAM ? dim3(a.stream) : dim3(a.num_splits, a.num_seqs, a.num_kv_heads / 8);
  const dim3 block(kWave * 8);
#define KNLP_LAUNCH_COOP(...)                                                            \
  do {                                                                                   \
    if constexpr (STREAM)                                                                \
      hipLaunchKernelGGL((decode_mfma_coop_stream_kernel<__VA_ARGS__>), grid, block, 0,  \
                         stream, a);                                                     \
    else                                                                                 \
      hipLaunchKernelGGL((decode_mfma_coop_kernel<__VA_ARGS__>), grid, block, 0, stream, \
                         a);                                                             \
  } while (0)
#define KNLP_ASYM_COOP(D, NG, NSETS)                                                     \
  if (ka && va) KNLP_LAUNCH_COOP(D, NG, true, true, false, NG, NSETS);                   \
  else if (ka) KNLP_LAUNCH_COOP(D, NG, true, false, false, NG, NSETS);                   \
  else if (va) KNLP_LAUNCH_COOP(D, NG, false, true, false, NG, NSETS);                   \
  else KNLP_LAUNCH_COOP(D, NG, false, false, false, NG, NSETS);
#define KNLP_INT4(D, NG)                                                                  \
  if (!k8 && !v8 && head_size == D && ng == NG) {                                         \
    if (nset == 1) {                                                                      \
      KNLP_ASYM_COOP(D, NG, 1)                                                            \
    } else {                                                                              \
      KNLP_ASYM_COOP(D, NG, 2)                                                            \
    }                                                                                     \
    return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;                   \
  }
#define KNLP_INT8K_SETS(NG, NGK)                                                          \
  if (nset == 1) {                                                                        \
    if (va) KNLP_LAUNCH_COOP(128, NG, false, true, true, NGK, 1);                         \
    else KNLP_LAUNCH_COOP(128, NG, false, false, true, NGK, 1);                           \
  } else {                                                                                \
    if (va) KNLP_LAUNCH_COOP(128, NG, false, true, true, NGK, 2);                         \
    else KNLP_LAUNCH_COOP(128, NG, false, false, true, NGK, 2);                           \
  }
  // The wide-group wave state (kv_decode_mfma.h, WaveStateW: two QK rows
  // per head, PV per V group): INT8 K with one scale per row and INT4 V in
  // four groups at 5 <= G <= 8 (one head set instead of two), and INT4 K
  // and V in two groups at G <= 8 (PV products within one group)
  if (k8 && !v8 && head_size == 128 && ng == 4 && ngk == 1 && a.group >= 5 && a.group <= 8) {
    if (va) KNLP_LAUNCH_COOP(128, 4, false, true, true, 1, 1, false, true);
    else KNLP_LAUNCH_COOP(128, 4, false, false, true, 1, 1, false, true);
    return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
  }
  if (!k8 && !v8 && head_size == 128 && ng == 2 && a.group <= 8) {
    if (ka && va) KNLP_LAUNCH_COOP(128, 2, true, true, false, 2, 1, false, true);
    else if (ka) KNLP_LAUNCH_COOP(128, 2, true, false, false, 2, 1, false, true);
    else if (va) KNLP_LAUNCH_COOP(128, 2, false, true, false, 2, 1, false, true);
    else KNLP_LAUNCH_COOP(128, 2, false, false, false, 2, 1, false, true);
    return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
  }
#define KNLP_INT8K(NG)                                                                    \
  if (k8 && !v8 && head_size == 128 && ng == NG) {                                        \
    if (ngk == 1) {                                                                       \
      KNLP_INT8K_SETS(NG, 1)                                                              \
    } else {                                                                              \
      KNLP_INT8K_SETS(NG, NG)                                                             \
    }                                                                                     \
    return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;                   \
  }
  KNLP_INT4(128, 4)
  KNLP_INT4(128, 2)
  KNLP_INT4(128, 1)
  KNLP_INT4(64, 4)
  KNLP_INT4(64, 2)
  KNLP_INT4(64, 1)
  KNLP_INT8K(4)
  KNLP_INT8K(2)
  KNLP_INT8K(1)
  // INT8 V (symmetric, biased codes): K INT4 (V's groups) or INT8 (one scale
  // per row or V's groups)
#define KNLP_V8_SETS(KA, K8, NG, NGK)                                                    \
  if (nset == 1) KNLP_LAUNCH_COOP(128, NG, KA, false, K8, NGK, 1, true);                 \
  else KNLP_LAUNCH_COOP(128, NG, KA, false, K8, NGK, 2, true);
#define KNLP_V8(NG)                                                                       \
  if (v8 && head_size == 128 && ng == NG) {                                               \
    if (k8 && ngk == 1) {                                                                 \
      KNLP_V8_SETS(false, true, NG, 1)                                                    \
    } else if (k8) {                                                                      \
      KNLP_V8_SETS(false, true, NG, NG)                                                   \
    } else if (ka) {                                                                      \
      KNLP_V8_SETS(true, false, NG, NG)                                                   \
    } else {                                                                              \
      KNLP_V8_SETS(false, false, NG, NG)                                                  \
    }                                                                                     \
    return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;                   \
  }
  KNLP_V8(4)
  KNLP_V8(1)
#undef KNLP_V8
#undef KNLP_V8_SETS
#undef KNLP_INT8K
#undef KNLP_INT8K_SETS
#undef KNLP_INT4
#undef KNLP_ASYM_COOP
#undef KNLP_LAUNCH_COOP
  return KNLP_ERR_SHAPE;
}

}  // namespace
}  // namespace knlp
