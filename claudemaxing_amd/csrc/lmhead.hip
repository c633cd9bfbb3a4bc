// Fused LM head + cross-entropy (gfx950). Entry points are declared in claudemaxing_amd.h.
// Not built yet: the entry point reports hipErrorNotSupported and the caller raises.
#include "common.h"

extern "C" int64_t cm_lmhead_ce_workspace_bytes(int64_t n_rows, int64_t vocab, int hidden_size,
                                                int64_t chunk_cols) {
  (void)n_rows; (void)vocab; (void)hidden_size; (void)chunk_cols;
  return 0;
}

extern "C" int cm_lmhead_ce(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
                            const int64_t* target, int64_t n_rows, int64_t vocab, int hidden_size,
                            int64_t chunk_cols, float* loss, float* entropy, int32_t* correct, float* grad,
                            float grad_scale, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  (void)hidden; (void)ld_h; (void)weight; (void)ld_w; (void)target; (void)n_rows; (void)vocab;
  (void)hidden_size; (void)chunk_cols; (void)loss; (void)entropy; (void)correct; (void)grad; (void)grad_scale;
  (void)workspace; (void)workspace_bytes; (void)stream;
  return static_cast<int>(hipErrorNotSupported);
}
