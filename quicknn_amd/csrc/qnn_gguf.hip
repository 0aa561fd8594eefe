// qnn_gguf.hip -- GGUF K-quant / Q8_0 kernels (placeholder until the GGUF path lands).
#include "qnn_internal.h"

namespace qnn {
GGLayout gguf_layout(int enc, int rows, int cols) {
  (void)enc; (void)rows; (void)cols;
  fail(QNN_E_NOT_SUPPORTED, "GGUF weights not built yet");
}
void gguf_repack_launch(const uint8_t *, const GGLayout &, void *, hipStream_t) {
  fail(QNN_E_NOT_SUPPORTED, "GGUF weights not built yet");
}
void gguf_dequant_launch(const GGLayout &, const void *, float *, hipStream_t) {
  fail(QNN_E_NOT_SUPPORTED, "GGUF weights not built yet");
}
}  // namespace qnn
