// NF4 prefill / training GEMM (M > 16) for gfx950.
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"

namespace rq {

int gemm_workspace(const LinearArgs& L, size_t* bytes) {
  (void)L;
  *bytes = 0;
  return RQ_ERR_UNSUPPORTED;
}

int run_nf4_gemm(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  (void)L; (void)workspace; (void)ws_bytes; (void)stream;
  return RQ_ERR_UNSUPPORTED;
}

}  // namespace rq
