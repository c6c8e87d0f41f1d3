// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "rocm_qlora_amd.h"

namespace rq {

inline bool valid_float_dtype(int dt) {
  return dt == RQ_DTYPE_F32 || dt == RQ_DTYPE_BF16 || dt == RQ_DTYPE_F16;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline size_t dtype_size(int dt) { return dt == RQ_DTYPE_F32 ? 4 : 2; }

// Largest grid.x * block.x the AMD dispatcher accepts in one dimension.
constexpr int64_t kMaxThreads1D = (int64_t(1) << 32) - 1024;

inline int rq_check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RQ_OK : RQ_ERR_HIP;
}

// Raises `kernel`'s dynamic LDS limit to `bytes` on the current device once
// (bit d of `done` marks device d; setting it twice from racing threads is
// harmless, the attribute value being the same).
inline int allow_dynamic_lds(const void* kernel, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return RQ_ERR_HIP;
  const uint64_t bit = dev < 64 ? (uint64_t(1) << dev) : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return RQ_OK;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) return RQ_ERR_HIP;
  done.fetch_or(bit, std::memory_order_release);
  return RQ_OK;
}

}  // namespace rq

// Instantiate `stmt` with the compile-time dtype constant NAME for a runtime
// float dtype code.
#define RQ_DISPATCH_DT(dt, NAME, ...)                                     \
  do {                                                                    \
    switch (dt) {                                                         \
      case RQ_DTYPE_F32: { constexpr int NAME = RQ_DTYPE_F32; __VA_ARGS__; break; }   \
      case RQ_DTYPE_BF16: { constexpr int NAME = RQ_DTYPE_BF16; __VA_ARGS__; break; } \
      default: { constexpr int NAME = RQ_DTYPE_F16; __VA_ARGS__; break; }             \
    }                                                                     \
  } while (0)
