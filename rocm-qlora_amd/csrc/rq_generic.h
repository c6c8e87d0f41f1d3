// Host interface of the generic dequantize-and-multiply kernels
// (generic_linear.hip): every shape, block size, alignment and activation
// dtype the reference's QuantLinear and _FP8LinearFunc accept, for the calls
// the specialized kernels do not take.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "rq_common.h"
#include "rq_linear.h"

namespace rq {

// Workspace bytes the generic NF4 forward or dX needs after the
// synchronization area: the LoRA operand, [M, rank] in the activation dtype.
size_t generic_lora_bytes(int x_dtype, int64_t M, int64_t rank);

// NF4 forward (rq_nf4_linear's contract); its LoRA operand lies at
// workspace + kLinearSyncBytes.
int run_generic_nf4_linear(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream);

// NF4 dX (rq_nf4_linear_dx's contract, dy fp32 too); its LoRA operand lies
// at the start of the workspace.
int run_generic_nf4_dx(const DxArgs& D, void* workspace, size_t ws_bytes, hipStream_t stream);

// INT8 weights q [N, K] (flat), per-row scales (block_size 0) or blockwise
// scales over the flat weight: y = x W^T + bias, or (dx) dX = dY W.
struct GenericInt8 {
  const void* x;  // x [M, K] (forward) or dY [M, N] (dX), row stride ldx
  int x_dtype;
  int64_t M, K, N, ldx;
  const int8_t* q;
  int64_t block_size;
  const void* scales;
  int scales_dtype;
  const void* bias;
  int bias_dtype;
  void* y;  // [M, N] (forward) or [M, K] (dX), row stride ldy
  int64_t ldy;
};
int run_generic_int8_linear(const GenericInt8& A, hipStream_t stream);
int run_generic_int8_dx(const GenericInt8& A, hipStream_t stream);

// FP8 (_FP8LinearFunc.forward restated as decode-then-multiply): x codes
// (e4m3fnuz, [M, K] dense) and their device scale, the weight's e4m3fn codes
// [N, K] and device scale; y = RND(RND((x8 sx)(w8 sw)^T) + RND(bias)) with
// the products summed in fp32 and RND the rounding to x_dtype (fp32: none).
int run_generic_fp8(int x_dtype, const uint8_t* x_codes, const float* x_scale, int64_t M, int64_t K,
                    const uint8_t* w_codes, const float* w_scale, int64_t N, const void* bias, int bias_dtype,
                    void* y, int64_t ldy, hipStream_t stream);

}  // namespace rq
