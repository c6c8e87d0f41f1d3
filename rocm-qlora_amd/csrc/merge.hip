// Merged LoRA weights straight from the quantized buffers, for gfx950.
//
// LoRALinear.merge_lora (lora_layer.py:72-113) and the export path's
// _export_dequant_layer (export/gguf_export.py:30-79) both build
//   W[n][k] = dequantized base weight (fp32: T[code] * scale for NF4, with
//             the scale c2 * c2_scale under double quantization; float(q) *
//             scale for INT8), and
//   d[n][k] = RND_L(RND_L(sum_j B[n][j] A[j][k]) * s), the LoRA delta (B @ A)
//             * scaling in the adapters' dtype L,
// and round them to a 16-bit weight, in one of two ways:
//   RQ_MERGE_SUM_THEN_ROUND  out = RND_o(W + d)            merge_lora
//   RQ_MERGE_ROUND_THEN_SUM  out = RND_o(RND_o(W) + RND_o(d))  export
// (RND_o: round to the output dtype; the second form is an add of two
// 16-bit tensors, which torch computes in fp32 and rounds once).  The delta's
// sum over the rank is an fp32 fma chain in ascending j.
//
// Workgroup: 256 columns k0 .. k0 + 255 (one per thread) x 64 rows n0 ..
// n0 + 63.  The rank runs in chunks of 32: the chunk's A rows for the 256
// columns and B columns for the 64 rows are staged in LDS (A read by column,
// B by broadcast, four ranks per read), each thread keeping its 64 sums in
// registers; the epilogue dequantizes the thread's 64 weights and stores.
#include "rq_common.h"
#include "rq_launch.h"
#include "rq_linear_dev.h"
#include "rq_mfma.h"

namespace rq {

constexpr int kMergeCols = 256;
constexpr int kMergeRows = 64;
constexpr int kMergeChunk = 32;

struct MergeArgs {
  const uint8_t* w;
  int w_format;
  int64_t N, K;
  int bs_log2;       // log2(block_size); -1: one scale per row (INT8)
  const void* scales;
  int scales_dt;
  const uint8_t* c2;  // NF4 double quantization: c2 codes, scales = c2_scales
  int c2_format;
  int64_t block2;
  const void* a;      // [rank, K]
  const void* b;      // [N, rank], row stride ldb
  int64_t ldb;
  int lora_dt;
  int64_t rank;
  float scaling;
  int mode;
  void* out;
  int out_dt;
  int64_t ldo;
};

__device__ __forceinline__ float load_any(const void* p, int64_t i, int dt) { return load_as_f32(p, i, dt); }

// The fp32 dequantized weight of flat element e (row-major [N, K]).
__device__ __forceinline__ float dequant_elem(const MergeArgs& a, int64_t n, int64_t e) {
  if (a.w_format == RQ_WEIGHT_INT8) {
    const int64_t blk = a.bs_log2 < 0 ? n : (e >> a.bs_log2);
    return __fmul_rn(float(int8_t(a.w[e])), load_any(a.scales, blk, a.scales_dt));  // quant_ops.py:65, :73
  }
  const uint8_t byte = a.w[e >> 1];
  const int code = (e & 1) ? (byte >> 4) : (byte & 15);  // quant_ops.py:137-141
  const int64_t blk = e >> a.bs_log2;
  float s;
  if (a.c2) {  // double_quant.py:108-111
    const int64_t g = blk / a.block2;
    const float hi = load_any(a.scales, g, a.scales_dt);
    const uint8_t c = a.c2[blk];
    const float lo = a.c2_format == RQ_C2_FP8_E4M3FNUZ ? fnuz_to_f32(c) : __fdiv_rn(float(int8_t(c)), 127.0f);
    s = __fmul_rn(lo, hi);
  } else {
    s = load_any(a.scales, blk, a.scales_dt);
  }
  return __fmul_rn(__uint_as_float(nf4_bits(code)), s);  // quant_ops.py:144-148
}

__global__ __launch_bounds__(kMergeCols) void merge_lora_kernel(MergeArgs a) {
  __shared__ float As[kMergeChunk][kMergeCols];      // 32 KiB
  __shared__ f32x4 Bs[kMergeRows][kMergeChunk / 4];  // 8 KiB
  const int t = threadIdx.x;
  const int64_t k = int64_t(blockIdx.x) * kMergeCols + t;
  const int64_t n0 = int64_t(blockIdx.y) * kMergeRows;
  float acc[kMergeRows];
#pragma unroll
  for (int r = 0; r < kMergeRows; ++r) acc[r] = 0.0f;
  for (int64_t j0 = 0; j0 < a.rank; j0 += kMergeChunk) {
    __syncthreads();  // the previous chunk has been read
#pragma unroll 4
    for (int jj = 0; jj < kMergeChunk; ++jj) {
      const int64_t j = j0 + jj;
      As[jj][t] = (j < a.rank && k < a.K) ? load_any(a.a, j * a.K + k, a.lora_dt) : 0.0f;
    }
    float* bflat = reinterpret_cast<float*>(Bs);
    for (int idx = t; idx < kMergeRows * kMergeChunk; idx += kMergeCols) {
      const int r = idx / kMergeChunk, c = idx % kMergeChunk;
      const int64_t n = n0 + r, j = j0 + c;
      bflat[idx] = (n < a.N && j < a.rank) ? load_any(a.b, n * a.ldb + j, a.lora_dt) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kMergeChunk / 4; ++q) {
      const float a0 = As[4 * q][t], a1 = As[4 * q + 1][t], a2 = As[4 * q + 2][t], a3 = As[4 * q + 3][t];
#pragma unroll
      for (int r = 0; r < kMergeRows; ++r) {
        const f32x4 bv = Bs[r][q];
        float v = acc[r];
        v = __builtin_fmaf(bv.x, a0, v);
        v = __builtin_fmaf(bv.y, a1, v);
        v = __builtin_fmaf(bv.z, a2, v);
        v = __builtin_fmaf(bv.w, a3, v);
        acc[r] = v;
      }
    }
  }
  if (k >= a.K) return;
#pragma unroll 4
  for (int r = 0; r < kMergeRows; ++r) {
    const int64_t n = n0 + r;
    if (n >= a.N) break;
    const float w = dequant_elem(a, n, n * a.K + k);
    const float d = round_to(__fmul_rn(round_to(acc[r], a.lora_dt), a.scaling), a.lora_dt);
    const float v = a.mode == RQ_MERGE_SUM_THEN_ROUND ? __fadd_rn(w, d)
                                                      : __fadd_rn(round_to(w, a.out_dt), round_to(d, a.out_dt));
    store_from_f32(a.out, n * a.ldo + k, a.out_dt, v);
  }
}

}  // namespace rq

extern "C" int rq_merge_lora(const void* w, int w_format, int64_t N, int64_t K, int64_t block_size,
                             const void* scales, int scales_dtype, const uint8_t* c2, int c2_format, int64_t block2,
                             const void* lora_a, const void* lora_b, int64_t ld_lora_b, int lora_dtype, int64_t rank,
                             float scaling, int mode, void* out, int out_dtype, int64_t ld_out, hipStream_t stream) {
  using namespace rq;
  if (!w || !scales || !out) return RQ_ERR_NULL_POINTER;
  if (w_format != RQ_WEIGHT_NF4 && w_format != RQ_WEIGHT_INT8) return RQ_ERR_BAD_DTYPE;
  if (!valid_float_dtype(scales_dtype)) return RQ_ERR_BAD_DTYPE;
  if (out_dtype != RQ_DTYPE_BF16 && out_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (mode != RQ_MERGE_SUM_THEN_ROUND && mode != RQ_MERGE_ROUND_THEN_SUM) return RQ_ERR_BAD_SHAPE;
  if (N <= 0 || K <= 0 || ld_out < K || rank < 0) return RQ_ERR_BAD_SHAPE;
  if (rank > 0) {
    if (!lora_a || !lora_b) return RQ_ERR_NULL_POINTER;
    if (!valid_float_dtype(lora_dtype)) return RQ_ERR_BAD_DTYPE;
    if (ld_lora_b < rank) return RQ_ERR_BAD_SHAPE;
  }
  const bool per_row = w_format == RQ_WEIGHT_INT8 && block_size == 0;
  if (!per_row && (block_size <= 0 || (block_size & (block_size - 1)))) return RQ_ERR_BAD_SHAPE;
  if (c2) {
    if (w_format != RQ_WEIGHT_NF4) return RQ_ERR_BAD_SHAPE;
    if (c2_format != RQ_C2_FP8_E4M3FNUZ && c2_format != RQ_C2_INT8) return RQ_ERR_BAD_DTYPE;
    if (block2 <= 0) return RQ_ERR_BAD_SHAPE;
  }
  MergeArgs a{};
  a.w = static_cast<const uint8_t*>(w); a.w_format = w_format; a.N = N; a.K = K;
  a.bs_log2 = per_row ? -1 : pow2_shift(block_size);
  a.scales = scales; a.scales_dt = scales_dtype; a.c2 = c2; a.c2_format = c2_format; a.block2 = block2;
  a.a = lora_a; a.b = lora_b; a.ldb = ld_lora_b; a.lora_dt = lora_dtype; a.rank = rank; a.scaling = scaling;
  a.mode = mode; a.out = out; a.out_dt = out_dtype; a.ldo = ld_out;
  const int64_t gx = (K + kMergeCols - 1) / kMergeCols, gy = (N + kMergeRows - 1) / kMergeRows;
  if (gx > 0x7FFFFFFF || gy > 65535) return RQ_ERR_UNSUPPORTED;
  merge_lora_kernel<<<dim3(unsigned(gx), unsigned(gy)), kMergeCols, 0, stream>>>(a);
  return rq_check_launch();
}
