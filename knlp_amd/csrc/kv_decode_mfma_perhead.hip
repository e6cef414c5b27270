// Stage 2 (matrix-core path): the per-head kernel's launches (one wave per
// (sequence, kv head, split), loads straight into VGPRs): fp16 K with INT4,
// INT8 or fp16 V, and INT4 K and V on layouts the cooperative kernel does not
// take.  Kernels in kv_decode_mfma.h.
#include "kv_decode_mfma.h"

namespace knlp {

int launch_mfma_perhead(const DecodeArgs& a, int head_size, hipStream_t stream) {
  const int ng = head_size / a.vp.group_size;
  const bool ka = a.kp.format == KNLP_KV_INT4_ASYM;
  const bool va = a.vp.format == KNLP_KV_INT4_ASYM;
  const bool v8 = a.vp.format == KNLP_KV_INT8_SYM;
  const bool k16 = a.kp.format == KNLP_KV_FP16;
  const int hpb = heads_per_block_mfma(a.num_kv_heads);
  const dim3 grid(a.num_splits, a.num_seqs, a.num_kv_heads / hpb);
  const dim3 block(kWave * hpb);
  const auto done = [] { return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH; };
#define KNLP_LAUNCH(...) hipLaunchKernelGGL((__VA_ARGS__), grid, block, 0, stream, a)
  if (k16) {
    if (a.vp.format == KNLP_KV_FP16) {   // fp16 K and V: at most 4 waves per block
      const int h4 = min(4, hpb);
      const dim3 grid4(a.num_splits, a.num_seqs, a.num_kv_heads / h4);
      const dim3 block4(kWave * h4);
      if (head_size == 128)
        hipLaunchKernelGGL((decode_mfma_kernel<128, 1, false, false, true, false, true>), grid4,
                           block4, 0, stream, a);
      else if (head_size == 64)
        hipLaunchKernelGGL((decode_mfma_kernel<64, 1, false, false, true, false, true>), grid4,
                           block4, 0, stream, a);
      else
        return KNLP_ERR_SHAPE;
      return done();
    }
    if (v8 && head_size == 128 && ng == 4) {
      KNLP_LAUNCH(decode_mfma_kernel<128, 4, false, false, true, true>);
      return done();
    }
    if (v8 && head_size == 128 && ng == 1) {
      KNLP_LAUNCH(decode_mfma_kernel<128, 1, false, false, true, true>);
      return done();
    }
#define KNLP_K16(D, NG)                                                                   \
    if (head_size == D && ng == NG && !v8) {                                              \
      if (va) KNLP_LAUNCH(decode_mfma_kernel<D, NG, false, true, true>);                  \
      else KNLP_LAUNCH(decode_mfma_kernel<D, NG, false, false, true>);                    \
      return done();                                                                      \
    }
    KNLP_K16(128, 4)
    KNLP_K16(128, 2)
    KNLP_K16(128, 1)
    KNLP_K16(64, 4)
    KNLP_K16(64, 2)
    KNLP_K16(64, 1)
#undef KNLP_K16
    return KNLP_ERR_SHAPE;
  }
  // INT4 K and V
  if (a.kp.format == KNLP_KV_INT8_SYM || v8) return KNLP_ERR_SHAPE;
#define KNLP_INT4(D, NG)                                                                  \
  if (head_size == D && ng == NG) {                                                       \
    if (ka && va) KNLP_LAUNCH(decode_mfma_kernel<D, NG, true, true>);                     \
    else if (ka) KNLP_LAUNCH(decode_mfma_kernel<D, NG, true, false>);                     \
    else if (va) KNLP_LAUNCH(decode_mfma_kernel<D, NG, false, true>);                     \
    else KNLP_LAUNCH(decode_mfma_kernel<D, NG, false, false>);                            \
    return done();                                                                        \
  }
  KNLP_INT4(128, 4)
  KNLP_INT4(128, 2)
  KNLP_INT4(128, 1)
  KNLP_INT4(64, 4)
  KNLP_INT4(64, 2)
  KNLP_INT4(64, 1)
#undef KNLP_INT4
#undef KNLP_LAUNCH
  return KNLP_ERR_SHAPE;
}

}  // namespace knlp
