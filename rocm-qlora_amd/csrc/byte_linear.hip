// INT8 weight linears for gfx950, and the reference's FP8 quantizer.
//
// INT8 (QuantLinear bits=8 and the row-absmax recipe): W = RND(float(q) *
// scale) with one scale per output row (quant_ops.py:28-35, :63-65) or per
// 64-element block of the flat weight (quant_ops.py:36-53, :69-78), then
// y = RND(x W^T + RND(bias)) as F.linear does (quant_linear.py:193-197).
// The weights are decoded exactly (one fp32 multiply, one rounding to the
// activation dtype) and multiplied by bf16/fp16 MFMA in fp32.
//
// M > 16 runs the shared MFMA core (rq_gemm_core.h) with a byte-weight
// producer; M <= 16 runs byte_gemv_kernel, a weight-streaming MFMA GEMV.
//
// FP8 per-tensor quantization (fp8_linear.py:33-42) to the reference's
// e4m3fnuz codes is here too; the FP8 linear itself runs on the fp8 matrix
// cores (fp8_mfma.hip).
#include "rq_gemm_core.h"
#include "rq_gemm8.h"

namespace rq {

// 4 weight bytes -> 4 fp32 operand values: float(int8) * s (one fp32
// rounding, as q.float() * scale).
__device__ __forceinline__ void decode4(uint32_t w, float s, float (&v)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = __fmul_rn(float(int8_t(uint8_t(w >> (8 * i)))), s);
}

template <int XT>
__device__ __forceinline__ uint2 decode4_pk(uint32_t w, float s) {
  float v[4];
  decode4(w, s, v);
  return uint2{cvt_pk<XT>(v[0], v[1]), cvt_pk<XT>(v[2], v[3])};
}

// Forward producer for byte weights (512 threads): tile row = output feature
// n, 64 reduction k per step = 64 weight bytes per row.  Thread t decodes
// row t / 4, bytes 16 (t % 4) .. +16 of the step (piece p = bytes 8p .. 8p + 7).
template <int XT, class Scale>
struct Byte8Producer {
  static constexpr int kLoads = 1 + Scale::kLoads;
  struct Regs {
    u32x4 w;
    typename Scale::Raw s;
  };
  struct Step {
    float sc;
    u32x4 w;
    uint32_t r[4];
  };
  ProducerParams P;
  Scale scale;
  uint32_t tile_row, quarter, wrow;
  int64_t wn;

  __device__ __forceinline__ void init(const ProducerParams& p, const Scale& sc, const u32x2*, int tid,
                                       int64_t col0) {
    P = p;
    scale = sc;
    tile_row = uint32_t(tid >> 2);
    quarter = uint32_t(tid & 3);
    wn = col0 + tile_row;
    wn = wn < P.rows ? wn : P.rows - 1;  // rows past N re-read a live row; never stored
    wrow = uint32_t(wn * P.row_bytes + 16 * quarter);  // the host keeps the weights under 4 GiB
  }
  __device__ __forceinline__ void issue(Regs& R, int64_t kstep) const {
    R.w = *reinterpret_cast<const u32x4*>(P.packed + (wrow + uint32_t(kstep) * 64u));
    R.s = scale.load(wn * P.blocks_per_row + ((kstep * kGemmBK) >> P.bs_log2));
  }
  __device__ __forceinline__ void prep(Step& S, const Regs& R) const {
    S.sc = scale.value(R.s);
    S.w = R.w;
  }
  __device__ __forceinline__ void lookup(Step&, int) const {}
  __device__ __forceinline__ void finish(Step& S, int p, int hh, uint8_t* tile) const {
    const int d = 2 * p + hh;  // dword of this thread's 16 bytes
    const uint32_t word = d == 0 ? S.w.x : d == 1 ? S.w.y : d == 2 ? S.w.z : S.w.w;
    const uint2 pk = decode4_pk<XT>(word, S.sc);
    S.r[2 * hh] = pk.x;
    S.r[2 * hh + 1] = pk.y;
    if (hh == 1)
      *reinterpret_cast<u32x4*>(tile + swz(tile_row, 2u * quarter + uint32_t(p))) =
          u32x4{S.r[0], S.r[1], S.r[2], S.r[3]};
  }
};

// ---------------------------------------------------------------------------
// Decode GEMV for M <= 16 rows of activations.  Wave w of a workgroup owns
// 16 weight rows; lane (i, q) (i = lane % 16, q = lane / 16) streams 16
// bytes of row i per 64-k step (k = 16 q .. 16 q + 15 of the step, so a
// wave instruction reads 16 rows x 64 contiguous bytes) and feeds them as
// two v_mfma_f32_16x16x32 A operands (k order 16 q + e and 16 q + 8 + e,
// the activation operand uses the same order).  D[n][m] = sum_k W[n][k]
// x[m][k]: lane (i, q), register r holds row n = 4 q + r, activation row
// m = i.
// ---------------------------------------------------------------------------
constexpr int kByteGemvDepth = 8;  // 64-k steps of weights in flight per lane

struct ByteGemvArgs {
  const uint16_t* x;   // [M][K] activation rows
  int64_t ldx;
  const uint8_t* w;    // [N][K] weight bytes
  int64_t M, N, K;
  int64_t blocks_per_row;
  int bs_log2;
  const void* bias;
  int bias_dt;
  uint16_t* y;
  int64_t ldy;
};

template <int XT, class Scale>
__global__ __launch_bounds__(256) void byte_gemv_kernel(ByteGemvArgs a, Scale scale) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i16 = lane & 15, q4 = lane >> 4;
  const int64_t n0 = (int64_t(blockIdx.x) * 4 + wave) * 16;
  int64_t n = n0 + i16;
  n = n < a.N ? n : a.N - 1;  // rows past N re-read a live row; never stored
  const uint8_t* wr = a.w + n * a.K + 16 * q4;
  const bool mlive = i16 < a.M;
  const uint16_t* xr = a.x + (mlive ? int64_t(i16) : 0) * a.ldx + 16 * q4;
  const int64_t nk = a.K / 64;
  const int64_t sb = n * a.blocks_per_row;

  u32x4 wq[kByteGemvDepth];
  typename Scale::Raw sq[kByteGemvDepth];
#pragma unroll
  for (int d = 0; d < kByteGemvDepth; ++d) {
    const int64_t kt = d < nk ? d : nk - 1;
    wq[d] = *reinterpret_cast<const u32x4*>(wr + kt * 64);
    sq[d] = scale.load(sb + ((kt * 64) >> a.bs_log2));
  }
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t kt = 0; kt < nk; kt += kByteGemvDepth) {
#pragma unroll
    for (int d = 0; d < kByteGemvDepth; ++d) {
      const int64_t k = kt + d;
      if (k >= nk) break;
      const u32x4 w = wq[d];
      const float s = scale.value(sq[d]);
      // activation operands of this step (rows >= M are zero)
      u32x4 xb0 = *reinterpret_cast<const u32x4*>(xr + k * 64);
      u32x4 xb1 = *reinterpret_cast<const u32x4*>(xr + k * 64 + 8);
      if (!mlive) xb0 = xb1 = u32x4{0u, 0u, 0u, 0u};
      // refill this slot with the step kByteGemvDepth ahead (past the end:
      // re-read the last step, in bounds and unused)
      const int64_t kn = k + kByteGemvDepth < nk ? k + kByteGemvDepth : nk - 1;
      wq[d] = *reinterpret_cast<const u32x4*>(wr + kn * 64);
      sq[d] = scale.load(sb + ((kn * 64) >> a.bs_log2));
      const uint2 a0 = decode4_pk<XT>(w.x, s), a1 = decode4_pk<XT>(w.y, s);
      const uint2 a2 = decode4_pk<XT>(w.z, s), a3 = decode4_pk<XT>(w.w, s);
      acc = mfma16x16x32<XT>(u32x4{a0.x, a0.y, a1.x, a1.y}, xb0, acc);
      acc = mfma16x16x32<XT>(u32x4{a2.x, a2.y, a3.x, a3.y}, xb1, acc);
    }
  }
  // epilogue: lane (i, q), register r -> y[m = i][n0 + 4 q + r]
  if (!mlive) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t no = n0 + 4 * q4 + r;
    if (no >= a.N) continue;
    float v = acc[r];
    if (a.bias) v = __fadd_rn(v, round_x<XT>(load_as_f32(a.bias, no, a.bias_dt)));
    v = round_x<XT>(v);
    a.y[int64_t(i16) * a.ldy + no] = uint16_t(to_x16<XT>(v));
  }
}

// ---------------------------------------------------------------------------
// FP8 per-tensor quantization (fp8_linear.py:37-42): absmax over the whole
// tensor (two deterministic max passes), s = fp32(double(absmax) / 240),
// code = fnuz(RND_dt(float(t) / s)) with the division in fp32 and RND_dt the
// rounding to the tensor's dtype (a 0-dim fp32 divisor keeps bf16/fp16).
// ---------------------------------------------------------------------------
constexpr int kAbsmaxBlocks = 1024;

template <int DT>
__global__ __launch_bounds__(256) void absmax_partial_kernel(const void* __restrict__ t, int64_t rows,
                                                             int64_t cols, int64_t ld, float* __restrict__ part) {
  __shared__ float red[256];
  float m = 0.0f;
  const int64_t total = rows * cols;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / cols, c = i - r * cols;
    const float v = fabsf(ld_f32<DT>(t, r * ld + c));
    m = (v > m || v != v) ? v : m;  // NaN propagates, as torch's max does
  }
  red[threadIdx.x] = m;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      const float b = red[threadIdx.x + o], c = red[threadIdx.x];
      red[threadIdx.x] = (b > c || b != b) ? b : c;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(256) void absmax_final_kernel(const float* __restrict__ part, int n,
                                                           float* __restrict__ scale) {
  __shared__ float red[256];
  float m = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) {
    const float v = part[i];
    m = (v > m || v != v) ? v : m;
  }
  red[threadIdx.x] = m;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      const float b = red[threadIdx.x + o], c = red[threadIdx.x];
      red[threadIdx.x] = (b > c || b != b) ? b : c;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) scale[0] = float(double(red[0]) / 240.0);
}

// codes[r][c] = fnuz(RND_dt(t / s)).
template <int DT>
__global__ __launch_bounds__(256) void fp8_encode_kernel(const void* __restrict__ t, int64_t rows, int64_t cols,
                                                         int64_t ld, const float* __restrict__ scale,
                                                         uint8_t* __restrict__ codes) {
  const float s = *scale;
  const int64_t total = rows * cols;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / cols, c = i - r * cols;
    codes[i] = f32_to_fnuz_rne(round_to(__fdiv_rn(ld_f32<DT>(t, r * ld + c), s), DT));
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct ByteLinearArgs {
  const void* x;
  int x_dtype;
  int64_t M, K, ldx;
  const uint8_t* w;
  int64_t N;
  int64_t block_size;   // 0 = per output row, else blockwise over the flat weight
  const void* scales;   // scales of scales_dtype
  int scales_dtype;
  const void* bias;
  int bias_dtype;
  void* y;
  int64_t ldy;
};

static int validate_byte(const ByteLinearArgs& A) {
  if (!A.x || !A.w || !A.y || !A.scales) return RQ_ERR_NULL_POINTER;
  if (A.x_dtype != RQ_DTYPE_BF16 && A.x_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (A.M < 0 || A.N <= 0 || A.K <= 0 || A.K % 64 != 0) return RQ_ERR_BAD_SHAPE;
  if (A.ldx < A.K || A.ldy < A.N) return RQ_ERR_BAD_SHAPE;
  if (A.scales_dtype != RQ_DTYPE_F32 && A.scales_dtype != RQ_DTYPE_BF16 && A.scales_dtype != RQ_DTYPE_F16)
    return RQ_ERR_BAD_DTYPE;
  if (A.block_size != 0 && (A.block_size < 64 || (A.block_size & (A.block_size - 1)) || A.K % A.block_size))
    return RQ_ERR_BAD_SHAPE;
  if (!aligned(A.x, 16) || A.ldx % 8 != 0 || !aligned(A.w, 16)) return RQ_ERR_BAD_ALIGNMENT;
  if (!offsets_fit(A.M, A.ldx, A.N, 2 * A.K)) return RQ_ERR_UNSUPPORTED;
  return RQ_OK;
}

template <int XT, class Scale>
static int launch_byte(const ByteLinearArgs& A, Scale scale, hipStream_t stream) {
  const uint16_t* x = static_cast<const uint16_t*>(A.x);
  const int64_t bpr = A.block_size ? A.K / A.block_size : 1;
  const int bsl = A.block_size ? pow2_shift(A.block_size) : 62;  // per row: k >> 62 == 0
  if (A.M <= kGemvMaxM) {
    ByteGemvArgs g;
    g.x = x; g.ldx = A.ldx; g.w = A.w; g.M = A.M; g.N = A.N; g.K = A.K;
    g.blocks_per_row = bpr; g.bs_log2 = bsl;
    g.bias = A.bias; g.bias_dt = A.bias_dtype;
    g.y = static_cast<uint16_t*>(A.y); g.ldy = A.ldy;
    byte_gemv_kernel<XT, Scale><<<unsigned((A.N + 63) / 64), 256, 0, stream>>>(g, scale);
    return rq_check_launch();
  }
  const GemmPlan p = plan_gemm(A.M, A.N, A.K, 0, device_cus());
  GemmArgs a{};
  a.x = x; a.ldx = A.ldx; a.M = A.M; a.N = A.N; a.K = A.K;
  a.tiles_m = p.tiles_m; a.tiles_n = p.tiles_n; a.xcd_map = p.xcd_map;
  a.splits = 1; a.lf = p.tiles_m * p.tiles_n / 8;
  GemmEpi e{};
  e.bias = A.bias; e.bias_dt = A.bias_dtype; e.scaling = 1.0f;
  e.y = static_cast<uint16_t*>(A.y); e.ldy = A.ldy;
  ProducerParams pp{A.w, A.K, A.N, bpr, bsl};
  const unsigned grid = unsigned(int64_t(p.tiles_m) * p.tiles_n);
  nf4_gemm8_kernel<XT, Byte8Producer<XT, Scale>, Scale><<<grid, kGemm8Threads, 0, stream>>>(a, pp, scale, e);
  return rq_check_launch();
}

template <int XT>
static int run_byte(const ByteLinearArgs& A, hipStream_t stream) {
  switch (A.scales_dtype) {
    case RQ_DTYPE_F32:
      return launch_byte<XT>(A, ScaleAbsmax<RQ_DTYPE_F32>{A.scales}, stream);
    case RQ_DTYPE_BF16:
      return launch_byte<XT>(A, ScaleAbsmax<RQ_DTYPE_BF16>{A.scales}, stream);
    default:
      return launch_byte<XT>(A, ScaleAbsmax<RQ_DTYPE_F16>{A.scales}, stream);
  }
}

static int byte_linear(const ByteLinearArgs& A, hipStream_t stream) {
  int st = validate_byte(A);
  if (st != RQ_OK) return st;
  if (A.M == 0) return RQ_OK;
  if (A.x_dtype == RQ_DTYPE_BF16) return run_byte<RQ_DTYPE_BF16>(A, stream);
  return run_byte<RQ_DTYPE_F16>(A, stream);
}

template <int DT>
static int fp8_quantize_t(const void* t, int64_t rows, int64_t cols, int64_t ld, float* part, float* scale,
                          uint8_t* codes, hipStream_t stream) {
  absmax_partial_kernel<DT><<<kAbsmaxBlocks, 256, 0, stream>>>(t, rows, cols, ld, part);
  absmax_final_kernel<<<1, 256, 0, stream>>>(part, kAbsmaxBlocks, scale);
  const int64_t blocks = (rows * cols + 255) / 256;
  fp8_encode_kernel<DT><<<unsigned(blocks < 65536 ? blocks : 65536), 256, 0, stream>>>(t, rows, cols, ld, scale,
                                                                                      codes);
  return rq_check_launch();
}

static int fp8_quantize(int dt, const void* t, int64_t rows, int64_t cols, int64_t ld, float* part, float* scale,
                        uint8_t* codes, hipStream_t stream) {
  switch (dt) {
    case RQ_DTYPE_F32: return fp8_quantize_t<RQ_DTYPE_F32>(t, rows, cols, ld, part, scale, codes, stream);
    case RQ_DTYPE_BF16: return fp8_quantize_t<RQ_DTYPE_BF16>(t, rows, cols, ld, part, scale, codes, stream);
    case RQ_DTYPE_F16: return fp8_quantize_t<RQ_DTYPE_F16>(t, rows, cols, ld, part, scale, codes, stream);
    default: return RQ_ERR_BAD_DTYPE;
  }
}

}  // namespace rq

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int rq_int8_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* q,
                              int64_t N, int64_t block_size, const void* scales, int scales_dtype, const void* bias,
                              int bias_dtype, void* y, int64_t ldy, hipStream_t stream) {
  rq::ByteLinearArgs A{};
  A.x = x; A.x_dtype = x_dtype; A.M = M; A.K = K; A.ldx = ldx;
  A.w = reinterpret_cast<const uint8_t*>(q); A.N = N;
  A.block_size = block_size; A.scales = scales; A.scales_dtype = scales_dtype;
  A.bias = bias; A.bias_dtype = bias_dtype; A.y = y; A.ldy = ldy;
  return rq::byte_linear(A, stream);
}

extern "C" int rq_fp8_quantize_workspace_size(int64_t* bytes) {
  if (!bytes) return RQ_ERR_NULL_POINTER;
  *bytes = int64_t(rq::kAbsmaxBlocks) * 4;
  return RQ_OK;
}

extern "C" int rq_fp8_quantize(const void* t, int t_dtype, int64_t rows, int64_t cols, int64_t ld, uint8_t* codes,
                               float* scale, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if (!t || !codes || !scale || !workspace) return RQ_ERR_NULL_POINTER;
  if (rows < 0 || cols < 0 || ld < cols) return RQ_ERR_BAD_SHAPE;
  if (workspace_bytes < int64_t(rq::kAbsmaxBlocks) * 4) return RQ_ERR_WORKSPACE;
  if (rows * cols == 0) return RQ_ERR_BAD_SHAPE;
  return rq::fp8_quantize(t_dtype, t, rows, cols, ld, static_cast<float*>(workspace), scale, codes, stream);
}
