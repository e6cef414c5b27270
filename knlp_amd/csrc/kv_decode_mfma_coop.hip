// Stage 2 (matrix-core path): the cooperative kernel on the split-K schedule.
#include "kv_decode_mfma_coop.h"

namespace knlp {

int launch_mfma_coop_split(const DecodeArgs& a, int head_size, hipStream_t stream) {
  return launch_coop<false>(a, head_size, stream);
}

}  // namespace knlp
