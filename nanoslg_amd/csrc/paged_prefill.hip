// Paged causal prefill attention (placeholder until the MFMA kernel lands).
#include "nslg_common.h"

using namespace nslg;

extern "C" size_t nslg_paged_prefill_workspace_size(int32_t batch, int32_t num_qo_heads,
                                                    int32_t head_dim, int64_t total_q,
                                                    int32_t max_q) {
  (void)batch; (void)num_qo_heads; (void)head_dim; (void)total_q; (void)max_q;
  return 256;
}

extern "C" int nslg_paged_prefill(const void*, int64_t, const int32_t*, int64_t, int32_t,
                                  const void*, const void*, int64_t, int32_t, const int32_t*,
                                  const int32_t*, const int32_t*, int32_t, int32_t, int32_t,
                                  int32_t, float, int32_t, void*, int64_t, void*, size_t,
                                  nslg_stream_t) {
  return fail(NSLG_EUNSUPPORTED, "paged_prefill: not built yet");
}
