// Chunked-prefill attention over the paged int4 / k8v4 cache (bf16 MFMA, K/V dequantised in LDS).
#include "qp_common.h"

extern "C" int qp_prefill(const qp_paged_cache *cache, const qp_prefill_args *a, qp_stream_t stream) {
  (void)cache;
  (void)a;
  (void)stream;
  return ::qp::fail(QP_ERR_UNSUPPORTED, "qp_prefill: not available in this build");
}
