// Library-level C-ABI entry points: status text, version, build target.
#include "rq_launch.h"

extern "C" const char* rq_status_string(int status) {
  switch (status) {
    case RQ_OK: return "ok";
    case RQ_ERR_NULL_POINTER: return "null device pointer";
    case RQ_ERR_BAD_DTYPE: return "unsupported dtype code";
    case RQ_ERR_BAD_SHAPE: return "invalid shape or size";
    case RQ_ERR_BAD_ALIGNMENT: return "pointer or leading dimension misaligned";
    case RQ_ERR_UNSUPPORTED: return "unsupported configuration";
    case RQ_ERR_WORKSPACE: return "workspace missing or too small";
    case RQ_ERR_HIP: return "HIP launch error";
    case RQ_ERR_SCRATCH_LIMIT: return "call needs more workspace than the allocation-free entry point's scratch";
    default: return "unknown status";
  }
}

extern "C" int rq_version(void) { return 100; }

extern "C" const char* rq_build_arch(void) { return "gfx950"; }

extern "C" int rq_stream_capture_id(hipStream_t stream, uint64_t* id) {
  if (!id) return RQ_ERR_NULL_POINTER;
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long cid = 0;
  if (hipStreamGetCaptureInfo(stream, &status, &cid) != hipSuccess) return RQ_ERR_HIP;
  *id = status == hipStreamCaptureStatusActive ? uint64_t(cid) : 0;
  return RQ_OK;
}
