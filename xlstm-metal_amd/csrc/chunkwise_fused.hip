// Fused single-pass chunkwise mLSTM forward (bf16 MFMA) — not built yet.
#include "chunkwise.h"

namespace xl {

bool chunkwise_fused_supported(const ChunkwiseArgs& a, const char** why) {
  (void)a;
  if (why) *why = "fused kernel not available in this build";
  return false;
}

int chunkwise_fused(const ChunkwiseArgs& a) {
  (void)a;
  return set_error(XL_ERR_UNSUPPORTED, "xl_mlstm_chunkwise_fwd: fused kernel not available in this build");
}

}  // namespace xl
