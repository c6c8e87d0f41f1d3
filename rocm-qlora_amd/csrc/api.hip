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
    default: return "unknown status";
  }
}

extern "C" int rq_version(void) { return 100; }

extern "C" const char* rq_build_arch(void) { return "gfx950"; }
