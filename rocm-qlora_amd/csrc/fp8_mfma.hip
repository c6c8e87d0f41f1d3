// FP8 linears on gfx950's fp8 matrix cores.
//
// _FP8LinearFunc.forward (fp8_linear.py:27-60) quantizes x and W per tensor
// to e4m3fnuz (bias 8, max 240, 0x80 NaN) and multiplies the decoded codes in
// fp32.  gfx950's fp8 MFMA (v_mfma_scale_f32_{32x32x64,16x16x128}_f8f6f4,
// here with unit E8M0 scales) reads the OCP e4m3fn format (bias 7, max 448,
// 0x7F / 0xFF NaN), so both operands are re-encoded value for value:
//   fn(c) = the e4m3fn code of fnuz value v(c)
// which is exact for every code except the 8 odd-mantissa magnitudes below
// 2^-6 (fnuz steps 2^-10, fn steps 2^-9 there), which round to the nearest
// even fn code -- a change of at most 2^-10 in a value whose tensor maximum is
// 240 (torch's own fnuz -> fn conversion gives the same codes).  The fnuz NaN
// becomes the fn NaN.  The products of fn codes are exact and the MFMA sums
// them in fp32; the epilogue is that of the reference:
//   y = RND(RND(acc * s_x * s_w) + RND(bias)).
//
// Kernels:
//   fnuz_to_fn_kernel      bulk re-encoding (rq_fp8_fnuz_to_e4m3fn)
//   fp8_quant_small_kernel per-tensor quantization of a small activation
//                          (absmax, scale and fn codes in one workgroup)
//   fp8_absmax16 / fp8_encode16
//                          the same for large activations, 16-byte vectors
//   byte_mfma_gemv_kernel  M <= 16: 16 weight rows x 1024 k per wave
//   byte_mfma_gemm_kernel  M > 16: 256 x 256 tiles, 5-stage LDS ring
// The GEMV and GEMM are templates on the operand policy: Fp8Mma here, I8Mma
// for the W8A8 int8 mode (int8 activations quantized per row, int32 sums).
#include "rq_fp8.h"
#include "rq_generic.h"
#include "rq_gemm_core.h"

namespace rq {

typedef int i32x8 __attribute__((ext_vector_type(8)));

// D += A B over 64 k (32 x 32 output) / 128 k (16 x 16 output), fn x fn
// operands (format 0 = e4m3 for both), scale exponents 127 (x 1.0).
__device__ __forceinline__ f32x16 mfma_fn_32x32x64(const u32x4& a0, const u32x4& a1, const u32x4& b0,
                                                   const u32x4& b1, const f32x16& c) {
  const i32x8 a = {int(a0.x), int(a0.y), int(a0.z), int(a0.w), int(a1.x), int(a1.y), int(a1.z), int(a1.w)};
  const i32x8 b = {int(b0.x), int(b0.y), int(b0.z), int(b0.w), int(b1.x), int(b1.y), int(b1.z), int(b1.w)};
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}
__device__ __forceinline__ f32x4 mfma_fn_16x16x128(const u32x4& a0, const u32x4& a1, const u32x4& b0,
                                                   const u32x4& b1, const f32x4& c) {
  const i32x8 a = {int(a0.x), int(a0.y), int(a0.z), int(a0.w), int(a1.x), int(a1.y), int(a1.z), int(a1.w)};
  const i32x8 b = {int(b0.x), int(b0.y), int(b0.z), int(b0.w), int(b1.x), int(b1.y), int(b1.z), int(b1.w)};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Operand policies of the byte-operand GEMM / GEMV below.
//   Fp8Mma: e4m3fn x e4m3fn, fp32 sums, per-tensor scales (the FP8 linear);
//   I8Mma:  int8 x int8, exact int32 sums (v_mfma_i32_{32x32x32,16x16x64}_i8,
//           two per step: the lane's first and second 16 bytes), per-row
//           scales of both operands (the W8A8 mode).
// Both take a lane's 32 bytes per step as two 16-byte halves, the same k
// order for both operands.  A step is kParts instructions (FP8: one over
// both halves; int8: one per half): the GEMV keeps one accumulator per part
// (part p of mma16 issues instruction p), the GEMM issues the int8 halves as
// two passes over its tiles (mma32h) and FP8 steps whole (mma32).
struct Fp8Mma {
  static constexpr bool kPerRow = false;
  static constexpr int kParts = 1;
  typedef f32x16 Acc32;
  typedef f32x4 Acc16;
  __device__ static Acc32 mma32(const u32x4& a0, const u32x4& a1, const u32x4& b0, const u32x4& b1, const Acc32& c) {
    return mfma_fn_32x32x64(a0, a1, b0, b1, c);
  }
  template <int P>
  __device__ static Acc16 mma16(const u32x4& a0, const u32x4& a1, const u32x4& b0, const u32x4& b1, const Acc16& c) {
    return mfma_fn_16x16x128(a0, a1, b0, b1, c);
  }
  __device__ static float to_f32(float v) { return v; }
};

struct I8Mma {
  static constexpr bool kPerRow = true;
  static constexpr int kParts = 2;
  typedef i32x16 Acc32;
  typedef i32x4 Acc16;
  __device__ static i32x4 bits(const u32x4& v) { return __builtin_bit_cast(i32x4, v); }
  __device__ static Acc32 mma32h(const u32x4& a, const u32x4& b, const Acc32& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(bits(a), bits(b), c, 0, 0, 0);
  }
  template <int P>
  __device__ static Acc16 mma16(const u32x4& a0, const u32x4& a1, const u32x4& b0, const u32x4& b1, const Acc16& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(bits(P ? a1 : a0), bits(P ? b1 : b0), c, 0, 0, 0);
  }
  __device__ static float to_f32(int v) { return float(v); }  // round to nearest
};

// Output scale of (m, n): FP8 the product of the two per-tensor scales, W8A8
// the activation row's scale times the weight row's.
template <class Op>
__device__ __forceinline__ float out_scale(const Fp8Args& a, int64_t m, int64_t n) {
  if constexpr (Op::kPerRow) return __fmul_rn(a.sx[m], load_as_f32(a.w_row_scale, n, a.w_row_scale_dt));
  else return __fmul_rn(*a.sx, *a.sw);
}

// y = RND(RND(float(acc) * scale) + RND(bias)).  FP8 applies the product of
// its two scalars at once (the reference multiplies by x_scale * w_scale
// folded into its GEMM); W8A8 multiplies by the row scales one at a time.
template <int XT, class Op, class V>
__device__ __forceinline__ float byte_epilogue(const Fp8Args& a, V acc, int64_t m, int64_t n) {
  float v;
  if constexpr (Op::kPerRow)
    v = __fmul_rn(__fmul_rn(Op::to_f32(acc), a.sx[m]), load_as_f32(a.w_row_scale, n, a.w_row_scale_dt));
  else
    v = __fmul_rn(Op::to_f32(acc), out_scale<Op>(a, m, n));
  v = round_x<XT>(v);
  if (a.bias) v = round_x<XT>(__fadd_rn(v, round_x<XT>(load_as_f32(a.bias, n, a.bias_dt))));
  return v;
}

// ---------------------------------------------------------------------------
// Bulk fnuz -> fn re-encoding, 16 bytes per thread (n % 16 == 0 part; the
// tail bytes one per thread).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fnuz_to_fn_kernel(const uint8_t* __restrict__ in, int64_t n,
                                                         uint8_t* __restrict__ out) {
  const int64_t nv = n / 16;
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < nv; i += stride) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(in + 16 * i);
    *reinterpret_cast<u32x4*>(out + 16 * i) = u32x4{fnuz_to_fn4(v.x), fnuz_to_fn4(v.y), fnuz_to_fn4(v.z),
                                                    fnuz_to_fn4(v.w)};
  }
  for (int64_t i = 16 * nv + int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
    out[i] = uint8_t(fnuz_to_fn4(in[i]));
}

// ---------------------------------------------------------------------------
// Activation quantization (fp8_linear.py:37-38): s = fp32(double(max|x|) /
// 240), code = fn(fnuz(RND_dt(x / s))).  x: [rows][cols] 16-bit of dtype DT,
// row stride ld; cols % 8 == 0, ld % 8 == 0, 16-byte aligned rows.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float h2f(uint32_t h) {
  return DT == RQ_DTYPE_BF16 ? bf16_to_f32(uint16_t(h)) : f16_to_f32(uint16_t(h));
}

// 8 elements (one 16-byte vector) -> 8 fn codes (two dwords).
template <int DT>
__device__ __forceinline__ u32x2 encode8_fn(const u32x4& v, float s, float rs) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t c[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = h2f<DT>((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
    const uint32_t code = f32_to_fnuz_rne(div_round<DT>(f, s, rs));
    c[e >> 2] |= code << (8 * (e & 3));
  }
  return u32x2{fnuz_to_fn4(c[0]), fnuz_to_fn4(c[1])};
}

template <int DT>
__device__ __forceinline__ float absmax8(const u32x4& v, float m) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) m = absmax_nan(m, h2f<DT>((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
  return m;
}

// NaN-propagating max over a workgroup of T threads (T a multiple of 64):
// lane shuffles within each wave, then the T / 64 waves' maxima through red
// behind one barrier (a tree through LDS would take log2(T) barriers).  Max
// is exact, so the result does not depend on the order (a NaN when any input
// is one).  Every thread returns it; red is not written again.
template <int T>
__device__ __forceinline__ float block_max_nan(float m, float* red) {
  static_assert(T % 64 == 0 && T <= 1024, "whole waves");
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max_nan(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) r = max_nan(r, red[w]);
  return r;
}

// One workgroup: absmax, the scale (also stored), then the codes.
template <int DT>
__global__ __launch_bounds__(1024) void fp8_quant_small_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                               int64_t cols, int64_t ld, float* __restrict__ scale,
                                                               uint8_t* __restrict__ codes) {
  __shared__ float red[16];
  const int gpr = int(cols / 8);
  const int total = int(rows) * gpr;
  float m = 0.0f;
  for (int i = threadIdx.x; i < total; i += 1024) {
    const int r = i / gpr, c = i - r * gpr;
    m = absmax8<DT>(*reinterpret_cast<const u32x4*>(x + int64_t(r) * ld + 8 * c), m);
  }
  const float s = float(double(block_max_nan<1024>(m, red)) / 240.0);
  if (threadIdx.x == 0) *scale = s;
  const float rs = recip_rn(s);
  for (int i = threadIdx.x; i < total; i += 1024) {
    const int r = i / gpr, c = i - r * gpr;
    const u32x2 q = encode8_fn<DT>(*reinterpret_cast<const u32x4*>(x + int64_t(r) * ld + 8 * c), s, rs);
    *reinterpret_cast<u32x2*>(codes + int64_t(r) * cols + 8 * c) = q;
  }
}

constexpr int kFp8AbsmaxBlocks = 1024;

template <int DT>
__global__ __launch_bounds__(256) void fp8_absmax16_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                           int64_t cols, int64_t ld, float* __restrict__ part) {
  __shared__ float red[4];
  const int64_t gpr = cols / 8, total = rows * gpr;
  float m = 0.0f;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / gpr, c = i - r * gpr;
    m = absmax8<DT>(*reinterpret_cast<const u32x4*>(x + r * ld + 8 * c), m);
  }
  m = block_max_nan<256>(m, red);
  if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// ---------------------------------------------------------------------------
// W8A8 activation quantization, one workgroup of T threads per row: the
// per-row recipe of quantize_int8 (quant_ops.py:29-35) on the row in fp32,
//   s_m = max(fp32(max_k |x[m][k]|) / 127, 1e-12),
//   q[m][k] = RNE(fp32(x[m][k]) / s_m)  (|q| <= 127 for finite rows).
// A NaN in the row makes its scale NaN (max and clamp propagate NaN, as
// torch's amax and clamp do) and its codes 0; codes are clamped to
// [-127, 127], so every output stays defined.  The second pass re-reads the
// row from the cache.
// ---------------------------------------------------------------------------
template <int DT, int T>
__global__ __launch_bounds__(T) void i8_row_quant_kernel(const uint16_t* __restrict__ x, int64_t K, int64_t ld,
                                                         float* __restrict__ scales, int8_t* __restrict__ codes) {
  __shared__ float red[T / 64];
  const int64_t m = blockIdx.x;
  const uint16_t* xr = x + m * ld;
  const int64_t groups = K / 8;
  float mx = 0.0f;
  for (int64_t i = threadIdx.x; i < groups; i += T) mx = absmax8<DT>(*reinterpret_cast<const u32x4*>(xr + 8 * i), mx);
  const float q127 = __fdiv_rn(block_max_nan<T>(mx, red), 127.0f);
  const float s = q127 > 1e-12f ? q127 : (q127 != q127 ? q127 : 1e-12f);  // torch.clamp keeps NaN
  if (threadIdx.x == 0) scales[m] = s;
  int8_t* cr = codes + m * K;
  for (int64_t i = threadIdx.x; i < groups; i += T) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + 8 * i);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t c[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float q = __builtin_rintf(__fdiv_rn(h2f<DT>((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu), s));
      q = q != q ? 0.0f : (q > 127.0f ? 127.0f : (q < -127.0f ? -127.0f : q));
      c[e >> 2] |= (uint32_t(int32_t(q)) & 0xFFu) << (8 * (e & 3));
    }
    *reinterpret_cast<u32x2*>(cr + 8 * i) = u32x2{c[0], c[1]};
  }
}

// Reduces the partial maxima (at most 1024, read from L2); every workgroup
// of the encode kernel does this for itself, so the scale needs no launch of
// its own.
__device__ __forceinline__ float scale_from_parts(const float* __restrict__ part, int nparts, float* red) {
  float m = 0.0f;
  for (int i = threadIdx.x; i < nparts; i += 256) {
    const float v = part[i];
    m = (v > m || v != v) ? v : m;
  }
  return float(double(block_max_nan<256>(m, red)) / 240.0);
}

template <int DT>
__global__ __launch_bounds__(256) void fp8_encode16_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                           int64_t cols, int64_t ld, const float* __restrict__ part,
                                                           int nparts, float* __restrict__ scale,
                                                           uint8_t* __restrict__ codes) {
  __shared__ float red[4];
  const float s = scale_from_parts(part, nparts, red);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale = s;
  const float rs = recip_rn(s);
  const int64_t gpr = cols / 8, total = rows * gpr;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / gpr, c = i - r * gpr;
    *reinterpret_cast<u32x2*>(codes + r * cols + 8 * c) =
        encode8_fn<DT>(*reinterpret_cast<const u32x4*>(x + r * ld + 8 * c), s, rs);
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV (M <= 16).  Workgroup: 16 weight rows n0 .. n0 + 15, eight
// waves, wave w the k chunks w, w + 8, ... of `chunk` k (a multiple of 128,
// at most 1024).  Lane (i, g) (i = lane % 16, g = lane / 16) feeds the
// 16x16x128 MFMA with bytes k = 16 g .. +15 and 64 + 16 g .. +15 of a 128-k
// step: weight row n0 + i as operand A, activation row i as operand B (zero
// for i >= M); D[n][m]: lane (i, g), register r = (row 4 g + r, activation
// i).  A wave holds its chunk's activations (8 steps x 8 VGPRs) and keeps 4
// steps of weights in flight.  The waves' sums meet in LDS and wave 0 adds
// them in wave order.
// ---------------------------------------------------------------------------
constexpr int kF8GvWaves = 8;
constexpr int kF8GvSteps = 8;   // 128-k steps per chunk, at most
constexpr int kF8GvDepth = 4;   // weight steps in flight

template <int XT, class Op>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
void byte_mfma_gemv_kernel(Fp8Args a) {
  typedef typename Op::Acc16 Acc;
  __shared__ Acc red[kF8GvWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int i16 = lane & 15, g = lane >> 4;
  const int64_t n0 = int64_t(blockIdx.x) * 16;
  int64_t n = n0 + i16;
  n = n < a.N ? n : a.N - 1;  // rows past N re-read a live row; never stored
  const bool xlive = i16 < a.M;
  const uint8_t* wr = a.w + n * a.K + 16 * g;
  const uint8_t* xr = a.x + (xlive ? int64_t(i16) : 0) * a.K + 16 * g;
  const int steps = a.gv_steps;  // per chunk
  const int64_t chunk = int64_t(steps) * 128;
  const int64_t nchunks = (a.K + chunk - 1) / chunk;

  Acc acc = {}, acc1 = {};  // acc1: the int8 policy's second part
  for (int64_t c = wave; c < nchunks; c += kF8GvWaves) {
    const int64_t kb = c * chunk;
    // half h of step s covers k = kb + 128 s + 64 h .. + 63; halves at or
    // past K are zero in both operands (their load addresses stay in the row)
    auto live = [&](int s, int h) -> bool { return kb + 128 * s + 64 * h < a.K; };
    auto koff = [&](int s, int h) -> int64_t { return live(s, h) ? kb + 128 * s + 64 * h : 0; };
    u32x4 xa[kF8GvSteps][2];
#pragma unroll
    for (int s = 0; s < kF8GvSteps; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        xa[s][h] = u32x4{0u, 0u, 0u, 0u};
        if (s < steps && xlive && live(s, h)) xa[s][h] = *reinterpret_cast<const u32x4*>(xr + koff(s, h));
      }
    u32x4 wq[kF8GvDepth][2];
#pragma unroll
    for (int d = 0; d < kF8GvDepth; ++d)
#pragma unroll
      for (int h = 0; h < 2; ++h) wq[d][h] = *reinterpret_cast<const u32x4*>(wr + koff(d < steps ? d : 0, h));
#pragma unroll
    for (int s = 0; s < kF8GvSteps; ++s) {
      if (s >= steps) break;
      u32x4 w0 = wq[s % kF8GvDepth][0], w1 = wq[s % kF8GvDepth][1];
      if (!live(s, 0)) w0 = u32x4{0u, 0u, 0u, 0u};
      if (!live(s, 1)) w1 = u32x4{0u, 0u, 0u, 0u};
      if (s + kF8GvDepth < steps) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          wq[s % kF8GvDepth][h] = *reinterpret_cast<const u32x4*>(wr + koff(s + kF8GvDepth, h));
      }
      acc = Op::template mma16<0>(w0, w1, xa[s][0], xa[s][1], acc);
      if constexpr (Op::kParts == 2) acc1 = Op::template mma16<1>(w0, w1, xa[s][0], xa[s][1], acc1);
    }
  }
  if constexpr (Op::kParts == 2) acc += acc1;  // exact int32 sums
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0 || !xlive) return;
  Acc sum = red[0][lane];
#pragma unroll
  for (int w = 1; w < kF8GvWaves; ++w) {
    const Acc v = red[w][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (Op::kPerRow) sum[r] += v[r];  // exact int32 sums
      else sum[r] = __fadd_rn(sum[r], v[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t no = n0 + 4 * g + r;
    if (no >= a.N) continue;
    const float v = byte_epilogue<XT, Op>(a, sum[r], int64_t(i16), no);
    a.y[int64_t(i16) * a.ldy + no] = uint16_t(to_x16<XT>(v));
  }
}

// ---------------------------------------------------------------------------
// GEMM (M > 16): out[M, N] = x[M, K] W[N, K]^T on 256 x 256 workgroup tiles,
// 64 k per stage, a ring of 5 LDS stages (x tile then W tile, 16 KiB each,
// rows of 64 bytes with 16-byte chunk c of row r at chunk c ^ ((r / 4) % 4),
// so that any 16 consecutive lanes reading one chunk of 16 consecutive rows
// hit 16 distinct 16-byte bank groups).  Both operands move by direct-to-LDS
// loads, issued four stages ahead of their MFMAs.  Eight waves, two per SIMD:
// wave w owns rows 128 (w % 2) .. +127 and columns 64 (w / 2) .. +63 of the
// tile as 4 x 2 blocks of the 32x32x64 MFMA; lane (i, h) (i = lane % 32, h =
// lane / 32) feeds bytes k = 32 h .. 32 h + 31 of the stage.  The weights
// are the MFMAs' A operand: lane (i, h), register r holds row i of the block,
// column 8 (r / 4) + 4 h + r % 4.
//
// Iteration j: wait until stages j and j + 1 have landed (this wave's loads;
// j + 2 and j + 3 may be in flight), barrier (every wave's loads of them too,
// and every wave is done reading stage j - 1), loads of stage j + 4 into
// stage j - 1's buffer, then the MFMAs of stage j on operands read in
// iteration j - 1 while the operands of stage j + 1 are read from LDS.  The
// matrix cores so never wait for an LDS read after the barrier.  Stages past
// the end re-load the last stage (in bounds, never used).
//
// With xcd_map, XCD x (= workgroup id % 8) takes tiles x T / 8 .. +T / 8 of
// the m-fastest tile order: the 32 workgroups an XCD runs at a time share
// their weight columns in its L2.
// ---------------------------------------------------------------------------
constexpr int kF8BM = 256, kF8BN = 256, kF8BK = 64;
constexpr int kF8Stages = 5;
constexpr int kF8Threads = 512;
constexpr int kF8TileBytes = kF8BM * kF8BK;       // 16 KiB
constexpr int kF8StageBytes = 2 * kF8TileBytes;   // x tile, W tile
static_assert(kF8BM == kF8BN, "one DMA lane map serves both operands");
static_assert(kF8Stages * kF8StageBytes <= 160 * 1024, "LDS plan");

// Output staging of a wave's 128 x 64 block after the main loop (144-byte
// rows, in the ring's LDS)
constexpr int kF8EpiPitch = 144;
constexpr int kF8EpiWaveBytes = 128 * kF8EpiPitch;
static_assert(8 * kF8EpiWaveBytes <= kF8Stages * kF8StageBytes, "output staging");

__device__ __forceinline__ uint32_t swz64(uint32_t r, uint32_t c) { return r * 64u + ((c ^ ((r >> 2) & 3u)) << 4); }

struct Fp8Frags {
  u32x4 a[4][2], b[2][2];
};

template <int XT, class Op>
__global__ __launch_bounds__(kF8Threads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void byte_mfma_gemm_kernel(Fp8Args a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kF8Stages * kF8StageBytes];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int i32 = lane & 31, h = lane >> 5;

  const int64_t T = int64_t(a.tiles_m) * a.tiles_n, g = blockIdx.x;
  const int64_t t = a.xcd_map ? (g % 8) * (T / 8) + g / 8 : g;
  const int64_t mt = t % a.tiles_m, nt = t / a.tiles_m;
  const int64_t m0 = mt * kF8BM, n0 = nt * kF8BN;

  // direct-to-LDS lanes: wave w loads rows 32 w .. +31 of both tiles, 16
  // rows per instruction; lane l of instruction tt: row 32 w + 16 tt + l / 4,
  // stored at chunk l % 4, which holds logical chunk (l % 4) ^ ((row / 4) % 4)
  uint32_t xo[2], wo[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const uint32_t r = uint32_t(32 * wave + 16 * tt + (lane >> 2));
    const uint32_t c = uint32_t(lane & 3) ^ ((r >> 2) & 3u);
    int64_t m = m0 + r, n = n0 + r;
    m = m < a.M ? m : a.M - 1;  // rows past M / N re-read a live row; never stored
    n = n < a.N ? n : a.N - 1;
    xo[tt] = uint32_t(m * a.K) + 16u * c;  // the host keeps both operands under 4 GiB
    wo[tt] = uint32_t(n * a.K) + 16u * c;
  }
  const uint32_t dst = __builtin_amdgcn_readfirstlane(uint32_t(32 * wave * kF8BK));
  const int nk = int(a.K / kF8BK);
  auto issue = [&](int ks) {
    ks = ks < nk ? ks : nk - 1;
    const uint32_t sb = uint32_t((ks % kF8Stages) * kF8StageBytes) + dst;
    const uint32_t ko = uint32_t(ks) * uint32_t(kF8BK);
    dma16(a.x, xo[0] + ko, sb);
    dma16(a.x, xo[1] + ko, sb + 1024);
    dma16(a.w, wo[0] + ko, sb + kF8TileBytes);
    dma16(a.w, wo[1] + ko, sb + kF8TileBytes + 1024);
  };
  // the buffer of stage j is j % kF8Stages; stages past the end sit in the
  // last stage's buffer
  const uint32_t arow = uint32_t(128 * wm + i32), brow = uint32_t(64 * wn + i32);
  auto read = [&](Fp8Frags& f, int j) {
    j = j < nk ? j : nk - 1;
    const uint8_t* xt = lds + (j % kF8Stages) * kF8StageBytes;
    const uint8_t* wt = xt + kF8TileBytes;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        f.b[nb][e] = *reinterpret_cast<const u32x4*>(wt + swz64(brow + 32 * nb, uint32_t(2 * h + e)));
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        f.a[mb][e] = *reinterpret_cast<const u32x4*>(xt + swz64(arow + 32 * mb, uint32_t(2 * h + e)));
  };

  typename Op::Acc32 acc[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0;

  // prologue: stages 0 .. 3 in flight, stage 0 read once it has landed
#pragma unroll
  for (int s = 0; s < kF8Stages - 1; ++s) issue(s);
  step_barrier<4 * (kF8Stages - 2)>();
  // the next stage's fragments are read while this stage's MFMAs run; int8
  // issues the first k-half of all eight blocks before the second, so no
  // MFMA waits on the one just issued to its accumulator (a half-stage
  // double buffer for int8 measured the same)
  Fp8Frags cur;
  read(cur, 0);
  for (int j = 0; j < nk; ++j) {
    step_barrier<4 * (kF8Stages - 3)>();
    issue(j + kF8Stages - 1);
    Fp8Frags nxt;
    read(nxt, j + 1);
    if constexpr (Op::kParts == 2) {
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = Op::mma32h(cur.b[nb][e], cur.a[mb][e], acc[mb][nb]);
    } else {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[mb][nb] = Op::mma32(cur.b[nb][0], cur.b[nb][1], cur.a[mb][0], cur.a[mb][1], acc[mb][nb]);
    }
    cur = nxt;
  }
  wait_vmcnt<0>();  // no load may still be landing in LDS when it holds the output
  __syncthreads();   // and every wave is done reading the last stage

  // Output.  The weights are the MFMAs' A operand, so lane (i32, h) holds row
  // m0 + 128 wm + 32 mb + i32 of block (mb, nb) and its columns 8 g + 4 h ..
  // + 3 in acc[mb][nb][4 g ..] (g < 4).  The values go, two per dword, into
  // the wave's LDS region (its 128 x 64 block, 144-byte rows), are read back
  // as 16-byte row pieces and stored eight 128-byte row pieces per
  // instruction.  (With the activations as A, a lane held one column and
  // stored 128 two-byte values, each behind its own bounds checks and scale
  // loads.)  y = RND(RND(float(acc) * scale) + RND(bias)), bias -0.0 where
  // there is none (x + -0.0 == x for every x).
  uint8_t* ws = lds + wave * kF8EpiWaveBytes;
  const float s_tensor = Op::kPerRow ? 0.0f : __fmul_rn(*a.sx, *a.sw);
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    float bias[4][4], wsc[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t n = n0 + 64 * wn + 32 * nb + 8 * g + 4 * h + c;
        bias[g][c] = a.bias && n < a.N ? round_x<XT>(load_as_f32(a.bias, n, a.bias_dt)) : -0.0f;
        wsc[g][c] = Op::kPerRow && n < a.N ? load_as_f32(a.w_row_scale, n, a.w_row_scale_dt) : 0.0f;
      }
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int64_t m = m0 + 128 * wm + 32 * mb + i32;
      const float sxm = Op::kPerRow && m < a.M ? a.sx[m] : 0.0f;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          v[c] = Op::kPerRow ? __fmul_rn(__fmul_rn(Op::to_f32(acc[mb][nb][4 * g + c]), sxm), wsc[g][c])
                             : __fmul_rn(Op::to_f32(acc[mb][nb][4 * g + c]), s_tensor);
        round2<XT>(v[0], v[1]);
        round2<XT>(v[2], v[3]);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = __fadd_rn(v[c], bias[g][c]);
        *reinterpret_cast<u32x2*>(ws + (32 * mb + i32) * kF8EpiPitch + (32 * nb + 8 * g + 4 * h) * 2) =
            u32x2{cvt_pk<XT>(v[0], v[1]), cvt_pk<XT>(v[2], v[3])};
      }
    }
  }
  // the wave reads back only its own region
  const bool full = m0 + kF8BM <= a.M && n0 + kF8BN <= a.N && (reinterpret_cast<uintptr_t>(a.y) & 15u) == 0 &&
                    (a.ldy & 7) == 0;
  const int64_t col = n0 + 64 * wn + 8 * (lane & 7);
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int r = 8 * it + (lane >> 3);
    const int64_t m = m0 + 128 * wm + r;
    const u32x4 o = *reinterpret_cast<const u32x4*>(ws + r * kF8EpiPitch + 16 * (lane & 7));
    uint16_t* yp = a.y + m * a.ldy + col;
    if (full) {
      *reinterpret_cast<u32x4*>(yp) = o;
    } else if (m < a.M) {
      const uint32_t w4[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int c = 0; c < 8; ++c)
        if (col + c < a.N) yp[c] = uint16_t(w4[c >> 1] >> (16 * (c & 1)));
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
int fp8_fnuz_to_fn(const uint8_t* in, int64_t n, uint8_t* out, hipStream_t stream) {
  if (n <= 0) return RQ_OK;
  if (!aligned(in, 16) || !aligned(out, 16)) return RQ_ERR_BAD_ALIGNMENT;
  const int64_t blocks = (n / 16 + 255) / 256;
  const unsigned grid = unsigned(blocks < 1 ? 1 : (blocks < 8192 ? blocks : 8192));
  fnuz_to_fn_kernel<<<grid, 256, 0, stream>>>(in, n, out);
  return rq_check_launch();
}

size_t fp8_act_ws_bytes(int64_t M, int64_t K) {
  // [absmax partials][scale][fn codes M x K]
  return size_t(kFp8AbsmaxBlocks) * 4 + 256 + ((size_t(M) * size_t(K) + 255) & ~size_t(255));
}

template <int XT>
static int fp8_quantize_act(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, float* part, float* scale,
                            uint8_t* codes, hipStream_t stream) {
  // one workgroup when each of its threads has at most 2 vectors to encode
  if (M * K <= 16384) {
    fp8_quant_small_kernel<XT><<<1, 1024, 0, stream>>>(x, M, K, ldx, scale, codes);
    return rq_check_launch();
  }
  const int64_t groups = M * (K / 8);
  const int64_t blocks = (groups + 255) / 256;
  const int nparts = int(blocks < kFp8AbsmaxBlocks ? blocks : kFp8AbsmaxBlocks);
  fp8_absmax16_kernel<XT><<<unsigned(nparts), 256, 0, stream>>>(x, M, K, ldx, part);
  fp8_encode16_kernel<XT><<<unsigned(blocks < 4096 ? blocks : 4096), 256, 0, stream>>>(x, M, K, ldx, part, nparts,
                                                                                      scale, codes);
  return rq_check_launch();
}

template <int XT>
static int fp8_linear_t(const Fp8LinearCall& c, void* workspace, hipStream_t stream) {
  char* ws = static_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(ws);
  float* xs = reinterpret_cast<float*>(ws + size_t(kFp8AbsmaxBlocks) * 4);
  uint8_t* xq = reinterpret_cast<uint8_t*>(ws + size_t(kFp8AbsmaxBlocks) * 4 + 256);
  int st = fp8_quantize_act<XT>(static_cast<const uint16_t*>(c.x), c.M, c.K, c.ldx, part, xs, xq, stream);
  if (st != RQ_OK) return st;
  Fp8Args a{};
  a.x = xq; a.w = c.w; a.M = c.M; a.N = c.N; a.K = c.K;
  a.sx = xs; a.sw = c.w_scale; a.bias = c.bias; a.bias_dt = c.bias_dtype;
  a.y = static_cast<uint16_t*>(c.y); a.ldy = c.ldy;
  if (c.M <= 16) {
    const int64_t steps128 = (c.K + 127) / 128;
    const int64_t per = (steps128 + kF8GvWaves - 1) / kF8GvWaves;
    a.gv_steps = int(per < 1 ? 1 : (per > kF8GvSteps ? kF8GvSteps : per));
    byte_mfma_gemv_kernel<XT, Fp8Mma><<<unsigned((c.N + 15) / 16), 512, 0, stream>>>(a);
    return rq_check_launch();
  }
  a.tiles_m = int((c.M + kF8BM - 1) / kF8BM);
  a.tiles_n = int((c.N + kF8BN - 1) / kF8BN);
  const int64_t T = int64_t(a.tiles_m) * a.tiles_n;
  a.xcd_map = T % 8 == 0;
  byte_mfma_gemm_kernel<XT, Fp8Mma><<<unsigned(T), kF8Threads, 0, stream>>>(a);
  return rq_check_launch();
}

int fp8_linear_run(const Fp8LinearCall& c, void* workspace, hipStream_t stream) {
  if (c.x_dtype == RQ_DTYPE_BF16) return fp8_linear_t<RQ_DTYPE_BF16>(c, workspace, stream);
  return fp8_linear_t<RQ_DTYPE_F16>(c, workspace, stream);
}

// ---------------------------------------------------------------------------
// W8A8: int8 activations (per row) x int8 weights (per row) on the int8
// matrix cores.  Workspace: [M row scales, fp32][M x K int8 codes].
// ---------------------------------------------------------------------------
static size_t w8a8_scales_bytes(int64_t M) { return (size_t(M) * 4 + 255) & ~size_t(255); }

size_t w8a8_ws_bytes(int64_t M, int64_t K) {
  return w8a8_scales_bytes(M) + ((size_t(M) * size_t(K) + 255) & ~size_t(255));
}

template <int XT>
static int i8_quantize_rows_t(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, float* scales, int8_t* codes,
                              hipStream_t stream) {
  // few rows: 1024 threads per row shorten the row's two passes
  if (M <= 64) i8_row_quant_kernel<XT, 1024><<<unsigned(M), 1024, 0, stream>>>(x, K, ldx, scales, codes);
  else i8_row_quant_kernel<XT, 256><<<unsigned(M), 256, 0, stream>>>(x, K, ldx, scales, codes);
  return rq_check_launch();
}

int i8_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, float* scales, int8_t* codes,
                     hipStream_t stream) {
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (x_dtype == RQ_DTYPE_BF16) return i8_quantize_rows_t<RQ_DTYPE_BF16>(xp, M, K, ldx, scales, codes, stream);
  return i8_quantize_rows_t<RQ_DTYPE_F16>(xp, M, K, ldx, scales, codes, stream);
}

template <int XT>
static int w8a8_linear_t(const W8A8LinearCall& c, void* workspace, hipStream_t stream) {
  char* ws = static_cast<char*>(workspace);
  float* xs = reinterpret_cast<float*>(ws);
  int8_t* xq = reinterpret_cast<int8_t*>(ws + w8a8_scales_bytes(c.M));
  int st = i8_quantize_rows_t<XT>(static_cast<const uint16_t*>(c.x), c.M, c.K, c.ldx, xs, xq, stream);
  if (st != RQ_OK) return st;
  Fp8Args a{};
  a.x = reinterpret_cast<const uint8_t*>(xq); a.w = reinterpret_cast<const uint8_t*>(c.w);
  a.M = c.M; a.N = c.N; a.K = c.K;
  a.sx = xs; a.w_row_scale = c.w_scales; a.w_row_scale_dt = c.w_scales_dtype;
  a.bias = c.bias; a.bias_dt = c.bias_dtype;
  a.y = static_cast<uint16_t*>(c.y); a.ldy = c.ldy;
  if (c.M <= 16) {
    const int64_t steps128 = (c.K + 127) / 128;
    const int64_t per = (steps128 + kF8GvWaves - 1) / kF8GvWaves;
    a.gv_steps = int(per < 1 ? 1 : (per > kF8GvSteps ? kF8GvSteps : per));
    byte_mfma_gemv_kernel<XT, I8Mma><<<unsigned((c.N + 15) / 16), 512, 0, stream>>>(a);
    return rq_check_launch();
  }
  a.tiles_m = int((c.M + kF8BM - 1) / kF8BM);
  a.tiles_n = int((c.N + kF8BN - 1) / kF8BN);
  const int64_t T = int64_t(a.tiles_m) * a.tiles_n;
  a.xcd_map = T % 8 == 0;
  byte_mfma_gemm_kernel<XT, I8Mma><<<unsigned(T), kF8Threads, 0, stream>>>(a);
  return rq_check_launch();
}

int w8a8_linear_run(const W8A8LinearCall& c, void* workspace, hipStream_t stream) {
  if (c.x_dtype == RQ_DTYPE_BF16) return w8a8_linear_t<RQ_DTYPE_BF16>(c, workspace, stream);
  return w8a8_linear_t<RQ_DTYPE_F16>(c, workspace, stream);
}

}  // namespace rq

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int rq_fp8_fnuz_to_e4m3fn(const uint8_t* codes, int64_t n, uint8_t* out, hipStream_t stream) {
  if (!codes || !out) return RQ_ERR_NULL_POINTER;
  if (n < 0) return RQ_ERR_BAD_SHAPE;
  return rq::fp8_fnuz_to_fn(codes, n, out, stream);
}

extern "C" int rq_fp8_linear_workspace_size(int64_t M, int64_t K, int64_t* bytes) {
  if (!bytes) return RQ_ERR_NULL_POINTER;
  if (M < 0 || K <= 0) return RQ_ERR_BAD_SHAPE;
  *bytes = int64_t(rq::fp8_act_ws_bytes(M, K));
  return RQ_OK;
}

extern "C" int rq_fp8_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_codes,
                             int64_t N, const float* w_scale, const void* bias, int bias_dtype, void* y, int64_t ldy,
                             void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if (!x || !w_codes || !w_scale || !y) return RQ_ERR_NULL_POINTER;
  if (!rq::valid_float_dtype(x_dtype)) return RQ_ERR_BAD_DTYPE;
  if (bias && !rq::valid_float_dtype(bias_dtype)) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || N <= 0 || K <= 0 || ldx < K || ldy < N) return RQ_ERR_BAD_SHAPE;
  if (!rq::aligned(x, rq::dtype_size(x_dtype)) || !rq::aligned(y, rq::dtype_size(x_dtype)))
    return RQ_ERR_BAD_ALIGNMENT;
  if (M == 0) return RQ_OK;
  if (!workspace) return RQ_ERR_NULL_POINTER;
  if (workspace_bytes < int64_t(rq::fp8_act_ws_bytes(M, K))) return RQ_ERR_WORKSPACE;
  if (!rq::aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  // the fp8 matrix cores take 16-bit activations read 16 bytes at a time, K a
  // multiple of 64 and code matrices within 32-bit byte offsets; every other
  // call (fp32 activations among them) quantizes x the same way and runs on
  // the generic kernels, which decode both code matrices and sum the fp32
  // products (fp8_linear.py:44-52)
  const bool fast = x_dtype != RQ_DTYPE_F32 && K % 64 == 0 && rq::aligned(x, 16) && ldx % 8 == 0 &&
                    rq::aligned(w_codes, 16) && double(M) * double(K) < 4294967296.0 &&
                    double(N) * double(K) < 4294967296.0;
  if (!fast) {
    char* ws = static_cast<char*>(workspace);
    float* part = reinterpret_cast<float*>(ws);
    float* xs = reinterpret_cast<float*>(ws + size_t(rq::kFp8AbsmaxBlocks) * 4);
    uint8_t* xq = reinterpret_cast<uint8_t*>(ws + size_t(rq::kFp8AbsmaxBlocks) * 4 + 256);
    int st = rq::fp8_quantize(x_dtype, x, M, K, ldx, part, xs, xq, stream);
    if (st != RQ_OK) return st;
    return rq::run_generic_fp8(x_dtype, xq, xs, M, K, w_codes, w_scale, N, bias, bias_dtype, y, ldy, stream);
  }
  rq::Fp8LinearCall c{};
  c.x = x; c.x_dtype = x_dtype; c.M = M; c.K = K; c.ldx = ldx;
  c.w = w_codes; c.N = N; c.w_scale = w_scale; c.bias = bias; c.bias_dtype = bias_dtype;
  c.y = y; c.ldy = ldy;
  return rq::fp8_linear_run(c, workspace, stream);
}

extern "C" int rq_int8_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int8_t* codes,
                                     float* scales, hipStream_t stream) {
  if (!x || !codes || !scales) return RQ_ERR_NULL_POINTER;
  if (x_dtype != RQ_DTYPE_BF16 && x_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || K <= 0 || K % 8 != 0 || ldx < K) return RQ_ERR_BAD_SHAPE;
  if (!rq::aligned(x, 16) || ldx % 8 != 0 || !rq::aligned(codes, 8)) return RQ_ERR_BAD_ALIGNMENT;
  if (M > 0x7FFFFFFF) return RQ_ERR_UNSUPPORTED;
  if (M == 0) return RQ_OK;
  return rq::i8_quantize_rows(x, x_dtype, M, K, ldx, scales, codes, stream);
}

extern "C" int rq_int8_linear_w8a8_workspace_size(int64_t M, int64_t K, int64_t* bytes) {
  if (!bytes) return RQ_ERR_NULL_POINTER;
  if (M < 0 || K <= 0) return RQ_ERR_BAD_SHAPE;
  *bytes = int64_t(rq::w8a8_ws_bytes(M, K));
  return RQ_OK;
}

extern "C" int rq_int8_linear_w8a8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* w,
                                   int64_t N, const void* w_scales, int w_scales_dtype, const void* bias,
                                   int bias_dtype, void* y, int64_t ldy, void* workspace, int64_t workspace_bytes,
                                   hipStream_t stream) {
  if (!x || !w || !w_scales || !y) return RQ_ERR_NULL_POINTER;
  if (x_dtype != RQ_DTYPE_BF16 && x_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (!rq::valid_float_dtype(w_scales_dtype)) return RQ_ERR_BAD_DTYPE;
  if (bias && !rq::valid_float_dtype(bias_dtype)) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || N <= 0 || K <= 0 || K % 64 != 0 || ldx < K || ldy < N) return RQ_ERR_BAD_SHAPE;
  if (!rq::aligned(x, 16) || ldx % 8 != 0 || !rq::aligned(w, 16)) return RQ_ERR_BAD_ALIGNMENT;
  // the GEMM addresses both code matrices with 32-bit byte offsets
  if (double(M) * double(K) >= 4294967296.0 || double(N) * double(K) >= 4294967296.0) return RQ_ERR_UNSUPPORTED;
  if (M > 0x7FFFFFFF) return RQ_ERR_UNSUPPORTED;
  if (M == 0) return RQ_OK;
  if (!workspace) return RQ_ERR_NULL_POINTER;
  if (workspace_bytes < int64_t(rq::w8a8_ws_bytes(M, K))) return RQ_ERR_WORKSPACE;
  if (!rq::aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  rq::W8A8LinearCall c{};
  c.x = x; c.x_dtype = x_dtype; c.M = M; c.K = K; c.ldx = ldx;
  c.w = w; c.N = N; c.w_scales = w_scales; c.w_scales_dtype = w_scales_dtype;
  c.bias = bias; c.bias_dtype = bias_dtype; c.y = y; c.ldy = ldy;
  return rq::w8a8_linear_run(c, workspace, stream);
}
