// Stage 2 (MFMA path): placeholder until the matrix-core kernel lands.
#include "kv_decode.h"

namespace knlp {

bool mfma_supported(int, int, int, int, int, int, int) { return false; }

int launch_decode_mfma(const DecodeArgs&, int, hipStream_t) { return KNLP_ERR_SHAPE; }

}  // namespace knlp
