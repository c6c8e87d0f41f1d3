// Generic dequantize-and-multiply kernels: the calls the specialized
// kernels do not take -- any K, any block size (blocks may straddle weight
// rows, as quantize_int4 / quantize_int8 lay them over the flat weight,
// quant_ops.py:80-126 / :20-53), operands at any alignment, fp32
// activations with any LoRA rank, fp32 dY, and FP8 with fp32 activations.
// The reference runs these through its dequantize-then-F.linear path
// (quantization/quant_linear.py:168-197, kernels/dequant_matmul.py:308-351,
// fp8/fp8_linear.py:27-60); here every element of the weight is decoded from
// its codes inside the multiply, with the same roundings.
//
// One kernel shape serves every operand format: a workgroup of 256 threads
// computes a 64 x 64 output tile.  Each reduction step, every thread decodes
// 8 (16-bit operands) or 4 (fp32) elements of the activation tile and of the
// weight tile with bounds checks, rounds them to the operand dtype and
// stages them in LDS; 16-bit operands then run on the 16x16x32 MFMA (each
// wave a 32 x 32 quadrant), fp32 operands on fp32 FMA (4 x 4 outputs per
// thread).  A second reduction over the LoRA rank (the same tile loop,
// operands u or v and RND(B) or RND(A)) feeds the epilogue.  Element loads
// are scalar: these shapes are the exceptions, and a tile's loads stay in
// the L1/L2 lines its neighbours use.
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"
#include "rq_generic.h"
#include "rq_fp8.h"

namespace rq {
namespace {

constexpr int kGenThreads = 256;
constexpr int kGenTile = 64;     // output rows and columns per workgroup
constexpr int kGenK16 = 32;      // reduction step of 16-bit operands (one MFMA k)
constexpr int kGenK32 = 16;      // reduction step of fp32 operands
constexpr int kGenPitch16 = 40;  // LDS row pitch (elements) of a 16-bit tile: 80 bytes
constexpr int kGenPitch32 = 68;  // LDS row pitch (floats) of an fp32 tile

// RND: rounding to the result dtype (fp32: none)
template <int XT>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (XT == RQ_DTYPE_F32) return v;
  else return round_x<XT>(v);
}

// e4m3fn: the bits of fnuz value v encode 2v (bias 7 against 8), but for
// 0x80 (-0 here, NaN in fnuz) and the NaNs 0x7F / 0xFF.
__device__ __forceinline__ float fn_to_f32(uint8_t c) {
  if ((c & 0x7Fu) == 0x7Fu) return __builtin_nanf("");
  if (c == 0x80u) return -0.0f;
  return 2.0f * fnuz_to_f32(c);
}

// ---- activation operands: the fp32 value of element (m, r), before the
// rounding to the operand dtype --------------------------------------------
template <int DT>
struct XPlain {
  const void* p;
  int64_t ld;
  float pre;     // RND(x * pre) when has_pre (dY * scaling of the LoRA dX term)
  bool has_pre;
  __device__ __forceinline__ float operator()(int64_t m, int64_t r) const {
    const float v = ld_f32<DT>(p, m * ld + r);
    return has_pre ? __fmul_rn(v, pre) : v;
  }
};

// FP8 activations: fnuz code times the per-tensor scale (fp8_linear.py:44-52's
// x_fp8.float() * x_scale)
struct XFnuz {
  const uint8_t* p;
  int64_t ld;
  const float* scale;
  __device__ __forceinline__ float operator()(int64_t m, int64_t r) const {
    return __fmul_rn(fnuz_to_f32(p[m * ld + r]), *scale);
  }
};

// ---- weight operands: the fp32 value of W[n, k] ---------------------------
// NF4: T[code] * scale of the code's flat block (quant_ops.py:144-148), the
// code at flat index f = n K + k (byte f / 2, low nibble first)
template <class Scale>
struct WNF4 {
  const uint8_t* packed;
  int64_t K, bs;
  Scale sc;
  __device__ __forceinline__ float operator()(int64_t n, int64_t k) const {
    const int64_t f = n * K + k;
    const uint32_t byte = packed[f >> 1];
    const uint32_t code = (f & 1) ? (byte >> 4) : (byte & 15u);
    return __fmul_rn(u2f(nf4_bits(int(code))), sc(f / bs));
  }
};

// INT8: float(q) * scale, one scale per row (bs 0) or per flat block
// (quant_ops.py:55-78)
template <int SDT>
struct WInt8 {
  const int8_t* q;
  int64_t K, bs;
  const void* s;
  __device__ __forceinline__ float operator()(int64_t n, int64_t k) const {
    const int64_t f = n * K + k;
    return __fmul_rn(float(q[f]), ld_f32<SDT>(s, bs > 0 ? f / bs : n));
  }
};

// FP8 weight: e4m3fn code times the per-tensor scale
struct WFn {
  const uint8_t* p;
  int64_t K;
  const float* scale;
  __device__ __forceinline__ float operator()(int64_t n, int64_t k) const {
    return __fmul_rn(fn_to_f32(p[n * K + k]), *scale);
  }
};

// A dense matrix of a runtime float dtype, element (n, k) at n sn + k sk
struct WDense {
  const void* p;
  int dt;
  int64_t sn, sk;
  __device__ __forceinline__ float operator()(int64_t n, int64_t k) const {
    return load_as_f32(p, n * sn + k * sk, dt);
  }
};

// ---- epilogue --------------------------------------------------------------
enum GenEpiMode {
  kEpiRound = 0,  // y = RND(acc)
  kEpiFwd = 1,    // y = RND(RND(acc + RND(bias)) + RND(RND(l) * scaling))
  kEpiDx = 2,     // y = RND(RND(acc) + RND(RND(l) * d)), d = mask ? mask_scale : 0 (1 without a mask)
  kEpiFp8 = 3,    // y = RND(RND(acc) + RND(bias))
};

struct GenEpi {
  const void* bias;
  int bias_dt;
  int rank;        // LoRA: l[m, c] = sum_j u[m, j] RND(lf(c, j))
  const void* u;   // [M, rank] in the result dtype, row stride ldu
  int64_t ldu;
  WDense lf;       // the second LoRA factor, element (c, j)
  float scaling;
  const uint8_t* mask;  // dropout keep-mask of the dX term, [M, C] bytes, row stride ldm
  int64_t ldm;
  float mask_scale;
  void* y;
  int64_t ldy;
};

template <int XT, int EPI>
__device__ __forceinline__ void gen_store(const GenEpi& e, int64_t m, int64_t c, float acc, float l) {
  float v;
  if constexpr (EPI == kEpiFwd) {
    v = acc;
    if (e.bias) v = __fadd_rn(v, rnd<XT>(load_as_f32(e.bias, c, e.bias_dt)));
    v = rnd<XT>(v);
    if (e.rank > 0) v = rnd<XT>(__fadd_rn(v, rnd<XT>(__fmul_rn(rnd<XT>(l), e.scaling))));
  } else if constexpr (EPI == kEpiDx) {
    v = rnd<XT>(acc);
    if (e.rank > 0) {
      float t = rnd<XT>(l);
      if (e.mask) t = rnd<XT>(__fmul_rn(t, e.mask[m * e.ldm + c] ? e.mask_scale : 0.0f));
      v = rnd<XT>(__fadd_rn(v, t));
    }
  } else if constexpr (EPI == kEpiFp8) {
    v = rnd<XT>(acc);
    if (e.bias) v = rnd<XT>(__fadd_rn(v, rnd<XT>(load_as_f32(e.bias, c, e.bias_dt))));
  } else {
    v = rnd<XT>(acc);
  }
  if constexpr (XT == RQ_DTYPE_F32) static_cast<float*>(e.y)[m * e.ldy + c] = v;
  else static_cast<uint16_t*>(e.y)[m * e.ldy + c] = uint16_t(to_x16<XT>(v));
}

// ---- reduction loops ---------------------------------------------------------
// 16-bit operands on the MFMA: acc[mt][nt] of wave (wm, wn), lane (i16, q),
// register r is output (m0 + 32 wm + 16 mt + 4 q + r, c0 + 32 wn + 16 nt + i16).
// Operand (c, r) of the weight is W[c, r], or W[r, c] when TRANS (dX).
template <int XT, bool TRANS, class XOp, class WOp>
__device__ __forceinline__ void reduce16(const XOp& x, const WOp& w, int64_t M, int64_t C, int64_t R, int64_t m0,
                                         int64_t c0, uint16_t* xs, uint16_t* ws, f32x4 (&acc)[2][2]) {
  const int t = threadIdx.x, row = t >> 2, c8 = (t & 3) * 8;
  const int lane = t & 63, wave = t >> 6, i16 = lane & 15, q = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t m = m0 + row, c = c0 + row;
  const bool mlive = m < M, clive = c < C;
  for (int64_t r0 = 0; r0 < R; r0 += kGenK16) {
    float xv[8], wv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t r = r0 + c8 + j;
      const bool rlive = r < R;
      xv[j] = mlive && rlive ? x(m, r) : 0.0f;
      wv[j] = clive && rlive ? (TRANS ? w(r, c) : w(c, r)) : 0.0f;
    }
    const u32x4 xp = {cvt_pk<XT>(xv[0], xv[1]), cvt_pk<XT>(xv[2], xv[3]), cvt_pk<XT>(xv[4], xv[5]),
                      cvt_pk<XT>(xv[6], xv[7])};
    const u32x4 wp = {cvt_pk<XT>(wv[0], wv[1]), cvt_pk<XT>(wv[2], wv[3]), cvt_pk<XT>(wv[4], wv[5]),
                      cvt_pk<XT>(wv[6], wv[7])};
    *reinterpret_cast<u32x4*>(xs + row * kGenPitch16 + c8) = xp;
    *reinterpret_cast<u32x4*>(ws + row * kGenPitch16 + c8) = wp;
    __syncthreads();
    u32x4 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      a[i] = *reinterpret_cast<const u32x4*>(xs + (32 * wm + 16 * i + i16) * kGenPitch16 + 8 * q);
      b[i] = *reinterpret_cast<const u32x4*>(ws + (32 * wn + 16 * i + i16) * kGenPitch16 + 8 * q);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma16x16x32<XT>(a[i], b[j], acc[i][j]);
    __syncthreads();
  }
}

// fp32 operands on FMA: acc[i][j] of thread (tx, ty) = (t % 16, t / 16) is
// output (m0 + ty + 16 i, c0 + tx + 16 j).
template <bool TRANS, class XOp, class WOp>
__device__ __forceinline__ void reduce32(const XOp& x, const WOp& w, int64_t M, int64_t C, int64_t R, int64_t m0,
                                         int64_t c0, float* xs, float* ws, float (&acc)[4][4]) {
  const int t = threadIdx.x, row = t >> 2, k4 = (t & 3) * 4, tx = t & 15, ty = t >> 4;
  const int64_t m = m0 + row, c = c0 + row;
  const bool mlive = m < M, clive = c < C;
  for (int64_t r0 = 0; r0 < R; r0 += kGenK32) {
    float xv[4], wv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t r = r0 + k4 + j;
      const bool rlive = r < R;
      xv[j] = mlive && rlive ? x(m, r) : 0.0f;
      wv[j] = clive && rlive ? (TRANS ? w(r, c) : w(c, r)) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xs[(k4 + j) * kGenPitch32 + row] = xv[j];
      ws[(k4 + j) * kGenPitch32 + row] = wv[j];
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < kGenK32; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = xs[kk * kGenPitch32 + ty + 16 * i];
        b[i] = ws[kk * kGenPitch32 + tx + 16 * i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
}

// out[m, c] = epi(sum_r RND(x(m, r)) RND(w(c, r)), sum_j u[m, j] RND(lf(c, j)))
// for m < M, c < C; XT is the result and rounding dtype; F32OPS keeps the
// operands in fp32 (FMA path) even when XT is 16-bit (FP8 operands).
template <int XT, bool F32OPS, bool TRANS, int EPI, class XOp, class WOp>
__global__ __launch_bounds__(kGenThreads) void generic_linear_kernel(XOp x, WOp w, int64_t M, int64_t C, int64_t R,
                                                                    GenEpi e) {
  const int64_t c0 = int64_t(blockIdx.x) * kGenTile, m0 = int64_t(blockIdx.y) * kGenTile;
  constexpr bool kLora = EPI == kEpiFwd || EPI == kEpiDx;
  if constexpr (F32OPS || XT == RQ_DTYPE_F32) {
    __shared__ float xs[kGenK32 * kGenPitch32], ws[kGenK32 * kGenPitch32];
    float acc[4][4], lacc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = lacc[i][j] = 0.0f;
    reduce32<TRANS>(x, w, M, C, R, m0, c0, xs, ws, acc);
    if constexpr (kLora) {
      if (e.rank > 0) reduce32<false>(XPlain<XT>{e.u, e.ldu, 1.0f, false}, e.lf, M, C, e.rank, m0, c0, xs, ws, lacc);
    }
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t m = m0 + ty + 16 * i, c = c0 + tx + 16 * j;
        if (m < M && c < C) gen_store<XT, EPI>(e, m, c, acc[i][j], lacc[i][j]);
      }
  } else {
    __shared__ __attribute__((aligned(16))) uint16_t xs[kGenTile * kGenPitch16], ws[kGenTile * kGenPitch16];
    f32x4 acc[2][2], lacc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = lacc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    reduce16<XT, TRANS>(x, w, M, C, R, m0, c0, xs, ws, acc);
    if constexpr (kLora) {
      if (e.rank > 0) reduce16<XT, false>(XPlain<XT>{e.u, e.ldu, 1.0f, false}, e.lf, M, C, e.rank, m0, c0, xs, ws, lacc);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, i16 = lane & 15, q = lane >> 4;
    const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = m0 + 32 * wm + 16 * i + 4 * q + r, c = c0 + 32 * wn + 16 * j + i16;
          if (m < M && c < C) gen_store<XT, EPI>(e, m, c, acc[i][j][r], lacc[i][j][r]);
        }
  }
}

template <int XT, bool F32OPS, bool TRANS, int EPI, class XOp, class WOp>
int launch_generic(const XOp& x, const WOp& w, int64_t M, int64_t C, int64_t R, const GenEpi& e,
                   hipStream_t stream) {
  if (M == 0 || C == 0) return RQ_OK;
  const int64_t gx = ceil_div(C, kGenTile), gy = ceil_div(M, kGenTile);
  if (gy > 65535 || gx > int64_t(INT32_MAX)) return RQ_ERR_UNSUPPORTED;
  generic_linear_kernel<XT, F32OPS, TRANS, EPI>
      <<<dim3(unsigned(gx), unsigned(gy)), kGenThreads, 0, stream>>>(x, w, M, C, R, e);
  return rq_check_launch();
}

// ---- NF4 forward -------------------------------------------------------------
template <int XT, class Scale>
int gen_nf4_fwd(const LinearArgs& L, Scale sc, void* u, hipStream_t stream) {
  GenEpi e{};
  e.bias = L.bias;
  e.bias_dt = L.bias_dtype;
  e.scaling = L.scaling;
  e.y = L.y;
  e.ldy = L.ldy;
  if (L.rank > 0) {
    // u = RND(xl . RND(A)^T), A [rank, K] row-major (lora_layer.py:67)
    GenEpi eu{};
    eu.y = u;
    eu.ldy = L.rank;
    const int st = launch_generic<XT, false, false, kEpiRound>(XPlain<XT>{L.lora_x, L.ld_lora_x, 1.0f, false},
                                                               WDense{L.lora_a, L.lora_dtype, L.K, 1}, L.M, L.rank,
                                                               L.K, eu, stream);
    if (st != RQ_OK) return st;
    e.rank = int(L.rank);
    e.u = u;
    e.ldu = L.rank;
    e.lf = WDense{L.lora_b, L.lora_dtype, L.ld_lora_b, 1};  // RND(B)[n, j]
  }
  return launch_generic<XT, false, false, kEpiFwd>(XPlain<XT>{L.x, L.ldx, 1.0f, false},
                                                   WNF4<Scale>{L.w_packed, L.K, L.block_size, sc}, L.M, L.N, L.K, e,
                                                   stream);
}

template <int XT>
int gen_nf4_fwd_x(const LinearArgs& L, void* u, hipStream_t stream) {
  if (L.c2) {
    const int sh = (L.block2 & (L.block2 - 1)) == 0 ? pow2_shift(L.block2) : -1;
    switch (L.absmax_dtype) {
      case RQ_DTYPE_F32:
        return gen_nf4_fwd<XT>(L, ScaleDQ<RQ_DTYPE_F32>{L.c2, L.absmax, L.c2_format, sh, L.block2}, u, stream);
      case RQ_DTYPE_BF16:
        return gen_nf4_fwd<XT>(L, ScaleDQ<RQ_DTYPE_BF16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, u, stream);
      default:
        return gen_nf4_fwd<XT>(L, ScaleDQ<RQ_DTYPE_F16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, u, stream);
    }
  }
  switch (L.absmax_dtype) {
    case RQ_DTYPE_F32: return gen_nf4_fwd<XT>(L, ScaleAbsmax<RQ_DTYPE_F32>{L.absmax}, u, stream);
    case RQ_DTYPE_BF16: return gen_nf4_fwd<XT>(L, ScaleAbsmax<RQ_DTYPE_BF16>{L.absmax}, u, stream);
    default: return gen_nf4_fwd<XT>(L, ScaleAbsmax<RQ_DTYPE_F16>{L.absmax}, u, stream);
  }
}

// ---- NF4 dX ------------------------------------------------------------------
template <int XT, class Scale>
int gen_nf4_dx(const DxArgs& D, Scale sc, void* v, hipStream_t stream) {
  GenEpi e{};
  e.y = D.dx;
  e.ldy = D.lddx;
  const int64_t rank = D.rank > 0 ? D.rank : 0;
  if (rank > 0) {
    // v = RND(RND(dY * s) . RND(B)), B [N, rank] of row stride ld_lora_b:
    // output j, reduced over n
    GenEpi ev{};
    ev.y = v;
    ev.ldy = rank;
    const int st = launch_generic<XT, false, true, kEpiRound>(XPlain<XT>{D.dy, D.lddy, D.scaling, true},
                                                              WDense{D.lora_b, D.lora_dtype, D.ld_lora_b, 1}, D.M,
                                                              rank, D.N, ev, stream);
    if (st != RQ_OK) return st;
    e.rank = int(rank);
    e.u = v;
    e.ldu = rank;
    e.lf = WDense{D.lora_a, D.lora_dtype, 1, D.K};  // RND(A)[j, k] as element (k, j)
    e.mask = D.lora_mask;
    e.ldm = D.ld_lora_mask;
    e.mask_scale = D.mask_scale;
  }
  // dX[m, k] = sum_n dY[m, n] RND(W[n, k])
  return launch_generic<XT, false, true, kEpiDx>(XPlain<XT>{D.dy, D.lddy, 1.0f, false},
                                                 WNF4<Scale>{D.w_packed, D.K, D.block_size, sc}, D.M, D.K, D.N, e,
                                                 stream);
}

template <int XT>
int gen_nf4_dx_x(const DxArgs& D, void* v, hipStream_t stream) {
  if (D.c2) {
    const int sh = (D.block2 & (D.block2 - 1)) == 0 ? pow2_shift(D.block2) : -1;
    switch (D.absmax_dtype) {
      case RQ_DTYPE_F32:
        return gen_nf4_dx<XT>(D, ScaleDQ<RQ_DTYPE_F32>{D.c2, D.absmax, D.c2_format, sh, D.block2}, v, stream);
      case RQ_DTYPE_BF16:
        return gen_nf4_dx<XT>(D, ScaleDQ<RQ_DTYPE_BF16>{D.c2, D.absmax, D.c2_format, sh, D.block2}, v, stream);
      default:
        return gen_nf4_dx<XT>(D, ScaleDQ<RQ_DTYPE_F16>{D.c2, D.absmax, D.c2_format, sh, D.block2}, v, stream);
    }
  }
  switch (D.absmax_dtype) {
    case RQ_DTYPE_F32: return gen_nf4_dx<XT>(D, ScaleAbsmax<RQ_DTYPE_F32>{D.absmax}, v, stream);
    case RQ_DTYPE_BF16: return gen_nf4_dx<XT>(D, ScaleAbsmax<RQ_DTYPE_BF16>{D.absmax}, v, stream);
    default: return gen_nf4_dx<XT>(D, ScaleAbsmax<RQ_DTYPE_F16>{D.absmax}, v, stream);
  }
}

// ---- INT8 ----------------------------------------------------------------------
template <int XT, int SDT>
int gen_int8(const GenericInt8& A, bool dx, hipStream_t stream) {
  GenEpi e{};
  e.y = A.y;
  e.ldy = A.ldy;
  const WInt8<SDT> w{A.q, A.K, A.block_size, A.scales};
  const XPlain<XT> x{A.x, A.ldx, 1.0f, false};
  if (dx) return launch_generic<XT, false, true, kEpiRound>(x, w, A.M, A.K, A.N, e, stream);
  e.bias = A.bias;
  e.bias_dt = A.bias_dtype;
  return launch_generic<XT, false, false, kEpiFwd>(x, w, A.M, A.N, A.K, e, stream);
}

template <int XT>
int gen_int8_x(const GenericInt8& A, bool dx, hipStream_t stream) {
  switch (A.scales_dtype) {
    case RQ_DTYPE_F32: return gen_int8<XT, RQ_DTYPE_F32>(A, dx, stream);
    case RQ_DTYPE_BF16: return gen_int8<XT, RQ_DTYPE_BF16>(A, dx, stream);
    default: return gen_int8<XT, RQ_DTYPE_F16>(A, dx, stream);
  }
}

int gen_int8_dispatch(const GenericInt8& A, bool dx, hipStream_t stream) {
  switch (A.x_dtype) {
    case RQ_DTYPE_F32: return gen_int8_x<RQ_DTYPE_F32>(A, dx, stream);
    case RQ_DTYPE_BF16: return gen_int8_x<RQ_DTYPE_BF16>(A, dx, stream);
    default: return gen_int8_x<RQ_DTYPE_F16>(A, dx, stream);
  }
}

}  // namespace

size_t generic_lora_bytes(int x_dtype, int64_t M, int64_t rank) {
  if (rank <= 0 || M <= 0) return 0;
  return (size_t(M) * size_t(rank) * dtype_size(x_dtype) + 255) & ~size_t(255);
}

int run_generic_nf4_linear(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (L.M == 0) return RQ_OK;
  void* u = nullptr;
  if (L.rank > 0) {
    const size_t need = kLinearSyncBytes + generic_lora_bytes(L.x_dtype, L.M, L.rank);
    if (!workspace || ws_bytes < need) return RQ_ERR_WORKSPACE;
    u = static_cast<char*>(workspace) + kLinearSyncBytes;
  }
  switch (L.x_dtype) {
    case RQ_DTYPE_F32: return gen_nf4_fwd_x<RQ_DTYPE_F32>(L, u, stream);
    case RQ_DTYPE_BF16: return gen_nf4_fwd_x<RQ_DTYPE_BF16>(L, u, stream);
    default: return gen_nf4_fwd_x<RQ_DTYPE_F16>(L, u, stream);
  }
}

int run_generic_nf4_dx(const DxArgs& D, void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (D.M == 0) return RQ_OK;
  void* v = nullptr;
  if (D.rank > 0) {
    if (!workspace || ws_bytes < generic_lora_bytes(D.dy_dtype, D.M, D.rank)) return RQ_ERR_WORKSPACE;
    v = workspace;
  }
  switch (D.dy_dtype) {
    case RQ_DTYPE_F32: return gen_nf4_dx_x<RQ_DTYPE_F32>(D, v, stream);
    case RQ_DTYPE_BF16: return gen_nf4_dx_x<RQ_DTYPE_BF16>(D, v, stream);
    default: return gen_nf4_dx_x<RQ_DTYPE_F16>(D, v, stream);
  }
}

int run_generic_int8_linear(const GenericInt8& A, hipStream_t stream) { return gen_int8_dispatch(A, false, stream); }

int run_generic_int8_dx(const GenericInt8& A, hipStream_t stream) { return gen_int8_dispatch(A, true, stream); }

int run_generic_fp8(int x_dtype, const uint8_t* x_codes, const float* x_scale, int64_t M, int64_t K,
                    const uint8_t* w_codes, const float* w_scale, int64_t N, const void* bias, int bias_dtype,
                    void* y, int64_t ldy, hipStream_t stream) {
  GenEpi e{};
  e.bias = bias;
  e.bias_dt = bias_dtype;
  e.y = y;
  e.ldy = ldy;
  const XFnuz x{x_codes, K, x_scale};
  const WFn w{w_codes, K, w_scale};
  switch (x_dtype) {
    case RQ_DTYPE_F32: return launch_generic<RQ_DTYPE_F32, true, false, kEpiFp8>(x, w, M, N, K, e, stream);
    case RQ_DTYPE_BF16: return launch_generic<RQ_DTYPE_BF16, true, false, kEpiFp8>(x, w, M, N, K, e, stream);
    default: return launch_generic<RQ_DTYPE_F16, true, false, kEpiFp8>(x, w, M, N, K, e, stream);
  }
}

}  // namespace rq
