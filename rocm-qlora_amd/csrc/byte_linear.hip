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
#include "rq_fp8.h"
#include "rq_generic.h"

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
  static constexpr bool kLoraRegs = false;  // no LoRA term
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
      *reinterpret_cast<u32x4*>(tile + swzw(tile_row, 2u * quarter + uint32_t(p))) =
          u32x4{S.r[0], S.r[1], S.r[2], S.r[3]};
  }
};

// ---------------------------------------------------------------------------
// Decode GEMV for M <= 16 rows of activations.  Workgroup: 16 weight rows n0
// .. n0 + 15 and all of K, sixteen waves, wave w the k chunks w, w + 16, ...
// of 256 k.  A chunk is 4 pieces of 64 k; lane (i, g) (i = lane % 16, g =
// lane / 16) loads 16 bytes of row n0 + i per piece, k = 64 t + 16 g .. +15,
// and feeds them as two 16x16x32 MFMA steps (h = 0, 1: bytes 8 h .. 8 h + 7);
// the activation operand (row i, zero for i >= M) takes the same k, so step
// (t, h) sums k = 64 t + 16 g + 8 h + e over g and e -- inside one 64-k block
// of the weight's scales.  Weights are decoded exactly, RND(float(q) * s), as
// the MFMA's B operand; D[m][n]: lane (i, g), register r = (row 4 g + r,
// column n0 + i).  The waves' sums meet in LDS and wave 0 adds them in wave
// order.  A wave holds its chunk's activations (32 VGPRs) and weights (16).
// ---------------------------------------------------------------------------
constexpr int kByteGvWaves = 16;
constexpr int kByteGvChunk = 256;   // k per wave chunk
constexpr int kByteGvPieces = kByteGvChunk / 64;

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
__global__ __launch_bounds__(64 * kByteGvWaves) void byte_gemv_kernel(ByteGemvArgs a, Scale scale) {
  __shared__ f32x4 red[kByteGvWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int i16 = lane & 15, g4 = lane >> 4;
  const int64_t n0 = int64_t(blockIdx.x) * 16;
  int64_t n = n0 + i16;
  n = n < a.N ? n : a.N - 1;  // rows past N re-read a live row; never stored
  const bool mlive = i16 < a.M;
  const uint8_t* wr = a.w + n * a.K + 16 * g4;
  const uint16_t* xr = a.x + (mlive ? int64_t(i16) : 0) * a.ldx + 16 * g4;
  const int64_t sb = n * a.blocks_per_row;
  const int64_t nchunks = (a.K + kByteGvChunk - 1) / kByteGvChunk;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t c = wave; c < nchunks; c += kByteGvWaves) {
    const int64_t kb = c * kByteGvChunk;
    // piece t covers k = kb + 64 t .. + 63; a piece at or past K is zero in
    // both operands (its loads stay inside the row)
    u32x4 wq[kByteGvPieces], xa[kByteGvPieces][2];
    typename Scale::Raw sq[kByteGvPieces];
#pragma unroll
    for (int t = 0; t < kByteGvPieces; ++t) {
      const int64_t k = kb + 64 * t;
      const bool live = k < a.K;
      const int64_t ko = live ? k : 0;
      wq[t] = *reinterpret_cast<const u32x4*>(wr + ko);
      sq[t] = scale.load(sb + (ko >> a.bs_log2));
      xa[t][0] = xa[t][1] = u32x4{0u, 0u, 0u, 0u};
      if (mlive && live) {
        xa[t][0] = *reinterpret_cast<const u32x4*>(xr + ko);
        xa[t][1] = *reinterpret_cast<const u32x4*>(xr + ko + 8);
      }
    }
#pragma unroll
    for (int t = 0; t < kByteGvPieces; ++t) {
      if (kb + 64 * t >= a.K) break;
      const float s = scale.value(sq[t]);
      const uint2 p0 = decode4_pk<XT>(wq[t].x, s), p1 = decode4_pk<XT>(wq[t].y, s);
      const uint2 p2 = decode4_pk<XT>(wq[t].z, s), p3 = decode4_pk<XT>(wq[t].w, s);
      acc = mfma16x16x32<XT>(xa[t][0], u32x4{p0.x, p0.y, p1.x, p1.y}, acc);
      acc = mfma16x16x32<XT>(xa[t][1], u32x4{p2.x, p2.y, p3.x, p3.y}, acc);
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4 sum = red[0][lane];
#pragma unroll
  for (int w = 1; w < kByteGvWaves; ++w) {
    const f32x4 v = red[w][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) sum[r] = __fadd_rn(sum[r], v[r]);
  }
  // lane (i, g): outputs y[4 g + r][n0 + i], r = 0..3
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t m = 4 * g4 + r;
    const int64_t no = n0 + i16;
    if (m >= a.M || no >= a.N) continue;
    float v = sum[r];
    if (a.bias) v = __fadd_rn(v, round_x<XT>(load_as_f32(a.bias, no, a.bias_dt)));
    a.y[m * a.ldy + no] = uint16_t(to_x16<XT>(round_x<XT>(v)));
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
  const float rs = recip_rn(s);
  const int64_t total = rows * cols;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / cols, c = i - r * cols;
    codes[i] = f32_to_fnuz_rne(div_round<DT>(ld_f32<DT>(t, r * ld + c), s, rs));
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
  if (!valid_float_dtype(A.x_dtype)) return RQ_ERR_BAD_DTYPE;
  if (A.M < 0 || A.N <= 0 || A.K <= 0 || A.block_size < 0) return RQ_ERR_BAD_SHAPE;
  if (A.ldx < A.K || A.ldy < A.N) return RQ_ERR_BAD_SHAPE;
  if (!valid_float_dtype(A.scales_dtype)) return RQ_ERR_BAD_DTYPE;
  if (A.bias && !valid_float_dtype(A.bias_dtype)) return RQ_ERR_BAD_DTYPE;
  if (!aligned(A.x, dtype_size(A.x_dtype)) || !aligned(A.y, dtype_size(A.x_dtype))) return RQ_ERR_BAD_ALIGNMENT;
  return RQ_OK;
}

// Whether the byte GEMV / MFMA GEMM take the call: 16-bit activations read
// 16 bytes at a time, K a multiple of 64, per-row scales or a power-of-two
// block of at least 64 dividing K, 32-bit offsets.  Every other valid call
// (fp32 activations among them) runs on the generic kernels.
static bool byte_fast_ok(const ByteLinearArgs& A) {
  if (A.x_dtype != RQ_DTYPE_BF16 && A.x_dtype != RQ_DTYPE_F16) return false;
  if (A.K % 64 != 0) return false;
  if (A.block_size != 0 && (A.block_size < 64 || (A.block_size & (A.block_size - 1)) || A.K % A.block_size))
    return false;
  if (!aligned(A.x, 16) || A.ldx % 8 != 0 || !aligned(A.w, 16)) return false;
  return offsets_fit(A.M, A.ldx, A.N, 2 * A.K);
}

static GenericInt8 generic_args(const ByteLinearArgs& A) {
  GenericInt8 g{};
  g.x = A.x; g.x_dtype = A.x_dtype; g.M = A.M; g.K = A.K; g.N = A.N; g.ldx = A.ldx;
  g.q = reinterpret_cast<const int8_t*>(A.w); g.block_size = A.block_size;
  g.scales = A.scales; g.scales_dtype = A.scales_dtype;
  g.bias = A.bias; g.bias_dtype = A.bias_dtype; g.y = A.y; g.ldy = A.ldy;
  return g;
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
    byte_gemv_kernel<XT, Scale><<<unsigned((A.N + 15) / 16), 64 * kByteGvWaves, 0, stream>>>(g, scale);
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
  if (!byte_fast_ok(A)) return run_generic_int8_linear(generic_args(A), stream);
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

int fp8_quantize(int dt, const void* t, int64_t rows, int64_t cols, int64_t ld, float* part, float* scale,
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

extern "C" int rq_int8_linear_dx(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t lddy, const int8_t* q,
                                 int64_t K, int64_t block_size, const void* scales, int scales_dtype, void* dx,
                                 int64_t lddx, hipStream_t stream) {
  if (!dy || !q || !scales || !dx) return RQ_ERR_NULL_POINTER;
  if (!rq::valid_float_dtype(dy_dtype) || !rq::valid_float_dtype(scales_dtype)) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || N <= 0 || K <= 0 || block_size < 0 || lddy < N || lddx < K) return RQ_ERR_BAD_SHAPE;
  if (!rq::aligned(dy, rq::dtype_size(dy_dtype)) || !rq::aligned(dx, rq::dtype_size(dy_dtype)))
    return RQ_ERR_BAD_ALIGNMENT;
  if (M == 0) return RQ_OK;
  rq::GenericInt8 g{};
  g.x = dy; g.x_dtype = dy_dtype; g.M = M; g.K = K; g.N = N; g.ldx = lddy;
  g.q = q; g.block_size = block_size; g.scales = scales; g.scales_dtype = scales_dtype;
  g.y = dx; g.ldy = lddx;
  return rq::run_generic_int8_dx(g, stream);
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
