// End-to-end two-stage top-k (YOLO26 / v10 heads).
#include "sy_internal.h"

namespace sy {

int op_e2e_topk(sy_ctx* ctx, const float* head, int batch, int channels, int anchors, int nc, int maximum, int onnx,
                float* out) {
  (void)ctx; (void)head; (void)batch; (void)channels; (void)anchors; (void)nc; (void)maximum; (void)onnx; (void)out;
  set_error("end-to-end top-k is not implemented yet");
  return SY_EUNSUPPORTED;
}

}  // namespace sy
