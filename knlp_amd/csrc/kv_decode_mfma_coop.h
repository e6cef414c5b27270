// Launches of the cooperative kernel (8 waves stage pages of 8 kv heads
// through LDS) for every format it takes, on either schedule: STREAM picks
// decode_mfma_coop_stream_kernel (one block per CU, equal tile shares) over
// decode_mfma_coop_kernel (split-K).  Included by kv_decode_mfma_coop.hip and
// kv_decode_mfma_stream.hip, one schedule each, so they compile in parallel.
#pragma once

#include "kv_decode_mfma.h"

namespace knlp {
namespace {

template <bool STREAM>
int launch_coop(const DecodeArgs& a, int head_size, hipStream_t stream) {
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
  // INT8 K with one scale per row, INT4 V in four groups, 5 <= G <= 8: the
  // wide-group wave state (one head set; kv_decode_mfma.h, WaveStateW)
  if (k8 && !v8 && head_size == 128 && ng == 4 && ngk == 1 && a.group >= 5 && a.group <= 8) {
    if (va) KNLP_LAUNCH_COOP(128, 4, false, true, true, 1, 1, false, true);
    else KNLP_LAUNCH_COOP(128, 4, false, false, true, 1, 1, false, true);
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
