// Stage 2 (matrix-core path): the cooperative kernel on the stream schedule.
#include "kv_decode_mfma_coop.h"

namespace knlp {

int launch_mfma_coop_stream(const DecodeArgs& a, int head_size, hipStream_t stream) {
  return launch_coop<true>(a, head_size, stream);
}

}  // namespace knlp
