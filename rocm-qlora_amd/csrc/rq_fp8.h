// FP8 (e4m3) linears on gfx950's fp8 matrix cores: shared declarations.
#pragma once

#include "rq_common.h"
#include "rq_launch.h"

namespace rq {

// Four e4m3fnuz codes (one per byte) -> the e4m3fn codes of the same values
// (gfx950's MFMA format), lane-parallel over the bytes of a dword:
//   magnitude m >= 16 (fnuz exponent >= 2): m - 8 (exponent bias 8 -> 7);
//   m < 16: round-half-even(m / 2) (fn's subnormal step is twice fnuz's);
//   0x80 (fnuz NaN) -> 0x7F (fn NaN, as torch's conversion gives); other
//   codes keep their sign bit.
// No step carries or borrows across bytes (every byte operand stays within
// 0..0xFF).
__host__ __device__ inline uint32_t fnuz_to_fn4(uint32_t w) {
  const uint32_t sgn = w & 0x80808080u;
  const uint32_t mag = w & 0x7F7F7F7Fu;
  const uint32_t big = (mag + 0x70707070u) & 0x80808080u;                   // 0x80 where m >= 16
  const uint32_t bigm = (big >> 7) * 0xFFu;                                  // 0xFF where m >= 16
  const uint32_t hi = ((mag | 0x80808080u) - 0x08080808u) & 0x7F7F7F7Fu;    // m - 8
  const uint32_t lo = ((mag + ((mag >> 1) & 0x01010101u)) >> 1) & 0x7F7F7F7Fu;  // rne(m / 2)
  const uint32_t nz = (mag + 0x7F7F7F7Fu) & 0x80808080u;                    // 0x80 where m != 0
  const uint32_t nan = sgn & ~nz;                                            // 0x80 where the byte is 0x80
  return (sgn ^ nan) | (hi & bigm) | (lo & ~bigm) | (nan - (nan >> 7));
}

// Kernel arguments of the FP8 GEMV / GEMM.
struct Fp8Args {
  const uint8_t* x;  // [M][K] e4m3fn activation codes, dense
  const uint8_t* w;  // [N][K] e4m3fn weight codes, dense
  int64_t M, N, K;
  int tiles_m, tiles_n;
  bool xcd_map;
  int gv_steps;          // GEMV: 128-k steps per wave chunk
  const float* sx;       // device scale(s) of the activations: per tensor (FP8) or per row (W8A8)
  const float* sw;       // FP8: device per-tensor weight scale
  const void* w_row_scale;  // W8A8: per-row weight scales of w_row_scale_dt
  int w_row_scale_dt;
  const void* bias;
  int bias_dt;
  uint16_t* y;
  int64_t ldy;
};

// A validated rq_fp8_linear call.
struct Fp8LinearCall {
  const void* x;
  int x_dtype;
  int64_t M, K, ldx;
  const uint8_t* w;  // e4m3fn codes
  int64_t N;
  const float* w_scale;
  const void* bias;
  int bias_dtype;
  void* y;
  int64_t ldy;
};

struct W8A8LinearCall {
  const void* x;
  int x_dtype;
  int64_t M, K, ldx;
  const int8_t* w;  // [N, K] int8, one scale per row
  int64_t N;
  const void* w_scales;
  int w_scales_dtype;
  const void* bias;
  int bias_dtype;
  void* y;
  int64_t ldy;
};

size_t fp8_act_ws_bytes(int64_t M, int64_t K);
size_t w8a8_ws_bytes(int64_t M, int64_t K);
int w8a8_linear_run(const W8A8LinearCall& c, void* workspace, hipStream_t stream);
int i8_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, float* scales, int8_t* codes,
                     hipStream_t stream);
int fp8_linear_run(const Fp8LinearCall& c, void* workspace, hipStream_t stream);
int fp8_fnuz_to_fn(const uint8_t* in, int64_t n, uint8_t* out, hipStream_t stream);
// Per-tensor FP8 quantization of a [rows, cols] tensor of dtype dt (row
// stride ld): part holds 1024 fp32 partial maxima, scale one fp32, codes the
// e4m3fnuz codes, dense.
int fp8_quantize(int dt, const void* t, int64_t rows, int64_t cols, int64_t ld, float* part, float* scale,
                 uint8_t* codes, hipStream_t stream);

}  // namespace rq
