// NF4 quantized linear (+ bias, + LoRA) for gfx950: the decode-shaped
// dequant-GEMV (M <= 16 rows of activations), the LoRA down-projection
// u = x . A^T, and the split-K epilogue.  The prefill / training GEMM and the
// dX kernels live in nf4_gemm.hip and share the epilogue defined here.
//
// Math (rocm_qlora's QuantLinear.forward + LoRALinear.forward,
// quant_linear.py:182-197, lora_layer.py:60-70), with RND = rounding to the
// activation dtype:
//   base[m,n] = RND( sum_k x[m,k] * W[n,k] + RND(bias[n]) ),  W = T[code] * absmax
//   u[m,j]    = RND( sum_k xl[m,k] * RND(A[j,k]) )           (xl = dropout(x) or x)
//   lora[m,n] = RND( RND( sum_j u[m,j] * RND(B[n,j]) ) * scaling )
//   y[m,n]    = RND( base[m,n] + lora[m,n] )
// The weight operand is RND(T[code] * scale), the very value the reference's
// dequantize_int4 + .to(x.dtype) produces (fp32 product, one RNE rounding);
// only the order of the fp32 sums differs from the CPU GEMM.
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"

namespace rq {

// ---------------------------------------------------------------------------
// Scale providers: fp32 scale of flat 64-aligned block b.
// ---------------------------------------------------------------------------
struct ScaleAbsmax {
  const void* p;
  int dt;
  __device__ __forceinline__ float operator()(int64_t b) const { return load_as_f32(p, b, dt); }
};

struct ScaleDQ {
  const uint8_t* c2;
  const void* c2s;
  int c2s_dt;
  int fmt;
  int64_t bs2;
  __device__ __forceinline__ float operator()(int64_t b) const {
    const float hi = load_as_f32(c2s, b / bs2, c2s_dt);
    const float lo = fmt == RQ_C2_FP8_E4M3FNUZ ? fnuz_to_f32(c2[b])
                                               : __fdiv_rn(float(int8_t(c2[b])), 127.0f);
    return __fmul_rn(lo, hi);
  }
};

// 16 consecutive activations of one row as two 8-element operands.
template <int XT>
__device__ __forceinline__ void load_x16(const uint16_t* __restrict__ p, bool vec, u32x4& a0, u32x4& a1) {
  if (vec) {
    a0 = *reinterpret_cast<const u32x4*>(p);
    a1 = *reinterpret_cast<const u32x4*>(p + 8);
  } else {
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = uint32_t(p[2 * j]) | (uint32_t(p[2 * j + 1]) << 16);
    a0 = u32x4{w[0], w[1], w[2], w[3]};
    a1 = u32x4{w[4], w[5], w[6], w[7]};
  }
}

// ---------------------------------------------------------------------------
// Epilogue shared by the GEMV, the split-K finisher and the GEMM.
// ---------------------------------------------------------------------------
template <int XT>
__device__ __forceinline__ float lora_term(const LinearEpi& e, const float* __restrict__ u_row, int64_t n) {
  float l = 0.0f;
  for (int j = 0; j < e.rank; ++j)
    l = __fmaf_rn(u_row[j], round_x<XT>(load_as_f32(e.lora_b, n * e.ld_lora_b + j, e.lora_dt)), l);
  return round_x<XT>(__fmul_rn(round_x<XT>(l), e.scaling));
}

template <int XT>
__device__ __forceinline__ float epilogue_value(const LinearEpi& e, const float* __restrict__ u_row,
                                                int64_t n, float acc) {
  float v = acc;
  if (e.bias) v = __fadd_rn(v, round_x<XT>(load_as_f32(e.bias, n, e.bias_dt)));
  v = round_x<XT>(v);
  if (e.rank > 0) v = round_x<XT>(__fadd_rn(v, lora_term<XT>(e, u_row, n)));
  return v;
}

// Stage RND(u[m, :]) for rows [m0, m0 + rows) into LDS (sums the u_splits
// partial products written by lora_u_kernel).
template <int XT>
__device__ __forceinline__ void stage_u(const LinearEpi& e, int64_t M, int64_t m0, int rows, float* us,
                                        int tid, int nthreads) {
  if (e.rank <= 0) return;
  const int total = rows * e.rank;
  for (int i = tid; i < total; i += nthreads) {
    const int64_t m = m0 + i / e.rank;
    const int j = i % e.rank;
    float s = 0.0f;
    if (m < M)
      for (int k = 0; k < e.u_splits; ++k) s = __fadd_rn(s, e.u[(int64_t(k) * M + m) * e.rank + j]);
    us[i] = round_x<XT>(s);
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV: y[M <= 16, N] = x[M, K] . W^T, W NF4 (block size multiple of
// 64, K % 64 == 0).
//
// One 16x16x32 MFMA step: A = 16 activation rows (rows >= M are zero), B =
// 16 weight rows x 32 k.  Lane (i = l % 16, q = l / 16) feeds row i of both
// operands with k = 64 kb + 16 q + 8 s + (0..7), s = 0, 1: each lane loads 8
// packed bytes of its weight row per 64-block (a whole wave load covers 16
// rows x 32 contiguous bytes) and one scale.  D row m = 4 (l / 16) + r,
// column = weight row l % 16.
//
// Work item = (group of R 16-row tiles, K split s).  The waves of a
// workgroup split the item's blocks; their fp32 partials are summed in a
// fixed order through LDS, so results are deterministic.
// ---------------------------------------------------------------------------
struct GemvArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* packed;
  int64_t M, N, K;
  int64_t blocks_per_row;  // K / block_size
  int64_t bs_shift;        // log2(block_size / 64)
  int S;                   // K splits
  int R;                   // row tiles per item (runtime copy of the template value)
  bool xvec;
  float* ws;               // [S, M, N] partials when S > 1
};

template <int XT, int R, class Scale>
__global__ __launch_bounds__(1024) void nf4_gemv_kernel(GemvArgs a, Scale scale, LinearEpi e) {
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x, nthreads = blockDim.x;
  const int nw = nthreads >> 6, wave = tid >> 6, lane = tid & 63;
  u32x2* lut = reinterpret_cast<u32x2*>(smem);
  float* red = reinterpret_cast<float*>(lut + kF32PairLutQwords);  // [nw][R][16][16]
  float* us = red + nw * R * 256;                                   // [16][rank]
  fill_f32pair_lut(lut, tid, nthreads);
  if (a.S == 1) stage_u<XT>(e, a.M, 0, 16, us, tid, nthreads);
  __syncthreads();

  const int i16 = lane & 15, q = lane >> 4;
  const uint32_t lane_off = uint32_t(lane & 31) * 8u;
  const int64_t KB = a.K >> 6;
  const int64_t half_k = a.K >> 1;
  const bool xlive = i16 < a.M;
  const uint16_t* xrow = a.x + (xlive ? i16 : 0) * a.ldx + 16 * q;
  const int64_t rows_per_item = 16 * R;
  const int64_t n_groups = (a.N + rows_per_item - 1) / rows_per_item;
  const int64_t n_items = n_groups * a.S;

  for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int64_t g = item / a.S;
    const int s = int(item % a.S);
    const int64_t kb0 = (KB * s) / a.S, kb1 = (KB * (s + 1)) / a.S;
    const int64_t wb0 = kb0 + ((kb1 - kb0) * wave) / nw;
    const int64_t wb1 = kb0 + ((kb1 - kb0) * (wave + 1)) / nw;
    const int64_t nbase = g * rows_per_item;

    const uint8_t* wrow[R];
    int64_t srow[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {
      int64_t n = nbase + 16 * t + i16;
      n = n < a.N ? n : a.N - 1;  // dead rows re-read a live row; never stored
      wrow[t] = a.packed + n * half_k + 8 * q;
      srow[t] = n * a.blocks_per_row;
    }
    f32x4 acc[R];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    int64_t kb = wb0;
    // two blocks per iteration: all loads first, then the math
    for (; kb + 2 <= wb1; kb += 2) {
      u32x4 xa[2][2];
      u32x2 wv[2][R];
      float sc[2][R];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (xlive) load_x16<XT>(xrow + 64 * (kb + u), a.xvec, xa[u][0], xa[u][1]);
        else xa[u][0] = xa[u][1] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int t = 0; t < R; ++t) {
          wv[u][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(wrow[t] + 32 * (kb + u)));
          sc[u][t] = scale(srow[t] + ((kb + u) >> a.bs_shift));
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int t = 0; t < R; ++t) {
          acc[t] = mfma16x16x32<XT>(xa[u][0], expand8_scaled<XT>(lut, wv[u][t].x, lane_off, sc[u][t]), acc[t]);
          acc[t] = mfma16x16x32<XT>(xa[u][1], expand8_scaled<XT>(lut, wv[u][t].y, lane_off, sc[u][t]), acc[t]);
        }
      }
    }
    for (; kb < wb1; ++kb) {
      u32x4 xa0, xa1;
      if (xlive) load_x16<XT>(xrow + 64 * kb, a.xvec, xa0, xa1);
      else xa0 = xa1 = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < R; ++t) {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(wrow[t] + 32 * kb));
        const float sc = scale(srow[t] + (kb >> a.bs_shift));
        acc[t] = mfma16x16x32<XT>(xa0, expand8_scaled<XT>(lut, w.x, lane_off, sc), acc[t]);
        acc[t] = mfma16x16x32<XT>(xa1, expand8_scaled<XT>(lut, w.y, lane_off, sc), acc[t]);
      }
    }

    // ordered cross-wave reduction and epilogue
#pragma unroll
    for (int t = 0; t < R; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((wave * R + t) * 16 + 4 * q + r) * 16 + i16] = acc[t][r];
    __syncthreads();
    for (int idx = tid; idx < R * 256; idx += nthreads) {
      const int t = idx >> 8, m = (idx >> 4) & 15, nn = idx & 15;
      const int64_t n = nbase + 16 * t + nn;
      if (m < a.M && n < a.N) {
        float v = 0.0f;
        for (int w = 0; w < nw; ++w) v = __fadd_rn(v, red[((w * R + t) * 16 + m) * 16 + nn]);
        if (a.S == 1) {
          v = epilogue_value<XT>(e, us + m * e.rank, n, v);
          static_cast<uint16_t*>(e.y)[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
        } else {
          a.ws[(int64_t(s) * a.M + m) * a.N + n] = v;
        }
      }
    }
    __syncthreads();
  }
}

// Split-K finisher: y = epilogue(sum_s ws[s]).  One workgroup per 16 rows of
// activations x 256 columns.
template <int XT>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(const float* __restrict__ ws, int S, int64_t M,
                                                              int64_t N, LinearEpi e) {
  extern __shared__ float us[];
  const int64_t m0 = int64_t(blockIdx.y) * 16;
  stage_u<XT>(e, M, m0, 16, us, threadIdx.x, blockDim.x);
  __syncthreads();
  const int64_t n = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (n >= N) return;
  for (int mm = 0; mm < 16 && m0 + mm < M; ++mm) {
    const int64_t m = m0 + mm;
    float v = 0.0f;
    for (int s = 0; s < S; ++s) v = __fadd_rn(v, ws[(int64_t(s) * M + m) * N + n]);
    v = epilogue_value<XT>(e, us + mm * e.rank, n, v);
    static_cast<uint16_t*>(e.y)[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
  }
}

// ---------------------------------------------------------------------------
// LoRA down-projection partials: up[ks, m, j] = sum_{k in split ks}
// xl[m, k] * RND(A[j, k]).  A (rank x K) is the trainable fp32 (or
// activation-dtype) parameter; it is rounded to the activation dtype on load,
// as lora_layer.py:67's `self.lora_A.to(x.dtype)` does.  One workgroup per
// (16 rows of xl, 16 rows of A, K split); its 4 waves split the K range and
// reduce through LDS.
// ---------------------------------------------------------------------------
template <int XT>
__device__ __forceinline__ u32x4 load_a8(const void* p, int dt, int64_t off, int64_t k, int64_t K, bool live) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t k0 = k + 2 * j, k1 = k + 2 * j + 1;
    const float v0 = (live && k0 < K) ? load_as_f32(p, off + k0, dt) : 0.0f;
    const float v1 = (live && k1 < K) ? load_as_f32(p, off + k1, dt) : 0.0f;
    w[j] = to_x16<XT>(v0) | (to_x16<XT>(v1) << 16);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

template <int XT>
__global__ __launch_bounds__(256) void lora_u_kernel(const uint16_t* __restrict__ xl, int64_t ldxl,
                                                     const void* __restrict__ A, int a_dt, int64_t M,
                                                     int64_t K, int rank, int KS, float* __restrict__ up) {
  __shared__ float red[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i16 = lane & 15, q = lane >> 4;
  const int64_t m = int64_t(blockIdx.x) * 16 + i16;
  const int64_t j = int64_t(blockIdx.y) * 16 + i16;
  const int ks = blockIdx.z;
  const int64_t nsteps = (K + 31) / 32;
  const int64_t s0 = (nsteps * ks) / KS, s1 = (nsteps * (ks + 1)) / KS;
  const int64_t w0 = s0 + ((s1 - s0) * wave) / 4, w1 = s0 + ((s1 - s0) * (wave + 1)) / 4;
  const bool mlive = m < M, jlive = j < rank;
  f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t st = w0; st < w1; ++st) {
    const int64_t k = 32 * st + 8 * q;
    u32x4 av, bv;
    {
      uint32_t w[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t k0 = k + 2 * t, k1 = k0 + 1;
        const uint32_t lo = (mlive && k0 < K) ? xl[m * ldxl + k0] : 0u;
        const uint32_t hi = (mlive && k1 < K) ? xl[m * ldxl + k1] : 0u;
        w[t] = lo | (hi << 16);
      }
      av = u32x4{w[0], w[1], w[2], w[3]};
    }
    bv = load_a8<XT>(A, a_dt, j * K, k, K, jlive);
    d = mfma16x16x32<XT>(av, bv, d);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][(4 * q + r) * 16 + i16] = d[r];
  __syncthreads();
  const int idx = threadIdx.x;  // 256 outputs: (row mm, col jj)
  const int mm = idx >> 4, jj = idx & 15;
  const int64_t om = int64_t(blockIdx.x) * 16 + mm, oj = int64_t(blockIdx.y) * 16 + jj;
  if (om < M && oj < rank) {
    float v = 0.0f;
    for (int w = 0; w < 4; ++w) v = __fadd_rn(v, red[w][idx]);
    up[(int64_t(ks) * M + om) * rank + oj] = v;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

GemvPlan plan_gemv(int64_t M, int64_t N, int64_t K, int64_t rank, int cus) {
  GemvPlan p{};
  const int64_t KB = K / 64;
  const int64_t tiles = (N + 15) / 16;
  p.R = 1;
  int S = 1;
  while (S < 8 && tiles * S < cus && KB / (S * 2) >= 4) S *= 2;
  p.S = S;
  const int64_t blocks_per_item = KB / S;
  int64_t nw = blocks_per_item / 4;
  p.nw = int(nw < 1 ? 1 : (nw > 16 ? 16 : nw));
  p.lds_bytes = size_t(kF32PairLutQwords) * 8 + size_t(p.nw) * p.R * 256 * 4 + size_t(16) * (rank > 0 ? rank : 0) * 4;
  const int per_cu = int(160 * 1024 / p.lds_bytes) > 0 ? int(160 * 1024 / p.lds_bytes) : 1;
  const int64_t items = ((N + 16 * p.R - 1) / (16 * p.R)) * S;
  p.grid = int(items < int64_t(cus) * per_cu ? items : int64_t(cus) * per_cu);
  p.u_splits = 0;
  if (rank > 0) {
    const int64_t mt = (M + 15) / 16, jt = (rank + 15) / 16;
    int ks = 1;
    while (ks < 16 && mt * jt * ks < cus && (K / 32) / (ks * 2) >= 16) ks *= 2;
    p.u_splits = ks;
  }
  p.ws_bytes = 0;
  if (S > 1) p.ws_bytes += size_t(S) * M * N * 4;
  p.u_offset = (p.ws_bytes + 255) & ~size_t(255);
  if (rank > 0) p.ws_bytes = p.u_offset + size_t(p.u_splits) * M * rank * 4;
  return p;
}

template <int XT>
static int launch_lora_u(const LinearArgs& L, int ks, float* up, hipStream_t stream) {
  dim3 grid(unsigned((L.M + 15) / 16), unsigned((L.rank + 15) / 16), unsigned(ks));
  lora_u_kernel<XT><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(L.lora_x), L.ld_lora_x,
                                              L.lora_a, L.lora_dtype, L.M, L.K, int(L.rank), ks, up);
  return rq_check_launch();
}

template <int XT, int R, class Scale>
static int launch_gemv_t(const LinearArgs& L, const GemvPlan& p, Scale scale, const LinearEpi& e,
                         float* ws, hipStream_t stream) {
  GemvArgs a;
  a.x = static_cast<const uint16_t*>(L.x);
  a.ldx = L.ldx;
  a.packed = L.w_packed;
  a.M = L.M;
  a.N = L.N;
  a.K = L.K;
  a.blocks_per_row = L.K / L.block_size;
  int sh = 0;
  while ((int64_t(64) << sh) < L.block_size) ++sh;
  a.bs_shift = sh;
  a.S = p.S;
  a.R = R;
  a.xvec = aligned(L.x, 16) && (L.ldx % 8 == 0);
  a.ws = ws;
  auto kern = nf4_gemv_kernel<XT, R, Scale>;
  static bool attr_set = false;  // one instantiation per (XT, R, Scale)
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess)
      return RQ_ERR_HIP;
    attr_set = true;
  }
  kern<<<p.grid, p.nw * 64, p.lds_bytes, stream>>>(a, scale, e);
  return rq_check_launch();
}

template <int XT>
static int run_gemv(const LinearArgs& L, const GemvPlan& p, const LinearEpi& e, float* ws, hipStream_t stream) {
  if (L.c2) {
    ScaleDQ sc{L.c2, L.absmax, L.absmax_dtype, L.c2_format, L.block2};
    return launch_gemv_t<XT, 1>(L, p, sc, e, ws, stream);
  }
  ScaleAbsmax sc{L.absmax, L.absmax_dtype};
  return launch_gemv_t<XT, 1>(L, p, sc, e, ws, stream);
}

template <int XT>
static int launch_splitk_epilogue(const LinearArgs& L, const GemvPlan& p, const LinearEpi& e, const float* ws,
                                  hipStream_t stream) {
  dim3 grid(unsigned((L.N + 255) / 256), unsigned((L.M + 15) / 16));
  const size_t lds = size_t(16) * (L.rank > 0 ? L.rank : 1) * 4;
  splitk_epilogue_kernel<XT><<<grid, 256, lds, stream>>>(ws, p.S, L.M, L.N, e);
  return rq_check_launch();
}

int validate_linear(const LinearArgs& L) {
  if (L.x_dtype != RQ_DTYPE_BF16 && L.x_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (!valid_float_dtype(L.absmax_dtype)) return RQ_ERR_BAD_DTYPE;
  if (L.bias && !valid_float_dtype(L.bias_dtype)) return RQ_ERR_BAD_DTYPE;
  if (L.rank > 0 && !valid_float_dtype(L.lora_dtype)) return RQ_ERR_BAD_DTYPE;
  if (L.c2 && L.c2_format != RQ_C2_FP8_E4M3FNUZ && L.c2_format != RQ_C2_INT8) return RQ_ERR_BAD_DTYPE;
  if (L.M < 0 || L.N < 1 || L.K < 64 || L.K % 64 != 0) return RQ_ERR_BAD_SHAPE;
  if (L.block_size < 64 || L.block_size % 64 != 0 || L.K % L.block_size != 0) return RQ_ERR_BAD_SHAPE;
  if ((L.block_size & (L.block_size - 1)) != 0) return RQ_ERR_BAD_SHAPE;
  if (L.c2 && L.block2 < 1) return RQ_ERR_BAD_SHAPE;
  if (L.ldx < L.K || L.ldy < L.N) return RQ_ERR_BAD_SHAPE;
  if (L.rank < 0 || L.rank > 256) return RQ_ERR_BAD_SHAPE;
  if (L.rank > 0 && (L.ld_lora_x < L.K || L.ld_lora_b < L.rank)) return RQ_ERR_BAD_SHAPE;
  if (L.M == 0) return RQ_OK;
  if (!L.x || !L.w_packed || !L.absmax || !L.y) return RQ_ERR_NULL_POINTER;
  if (L.rank > 0 && (!L.lora_x || !L.lora_a || !L.lora_b)) return RQ_ERR_NULL_POINTER;
  if (!aligned(L.w_packed, 8)) return RQ_ERR_BAD_ALIGNMENT;
  if (!aligned(L.x, 2) || !aligned(L.y, 2)) return RQ_ERR_BAD_ALIGNMENT;
  return RQ_OK;
}

LinearEpi make_epi(const LinearArgs& L, float* u_parts, int u_splits) {
  LinearEpi e;
  e.bias = L.bias;
  e.bias_dt = L.bias_dtype;
  e.rank = int(L.rank);
  e.u = u_parts;
  e.u_splits = u_splits;
  e.lora_b = L.lora_b;
  e.ld_lora_b = L.ld_lora_b;
  e.lora_dt = L.lora_dtype;
  e.scaling = L.scaling;
  e.y = L.y;
  e.ldy = L.ldy;
  return e;
}

int run_lora_u(const LinearArgs& L, int ks, float* up, hipStream_t stream) {
  if (L.x_dtype == RQ_DTYPE_BF16) return launch_lora_u<RQ_DTYPE_BF16>(L, ks, up, stream);
  return launch_lora_u<RQ_DTYPE_F16>(L, ks, up, stream);
}

int gemv_workspace(const LinearArgs& L, size_t* bytes) {
  GemvPlan p = plan_gemv(L.M, L.N, L.K, L.rank, device_cus());
  *bytes = p.ws_bytes;
  return RQ_OK;
}

int run_nf4_gemv(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  const GemvPlan p = plan_gemv(L.M, L.N, L.K, L.rank, device_cus());
  if (p.ws_bytes > 0 && (!workspace || ws_bytes < p.ws_bytes)) return RQ_ERR_WORKSPACE;
  if (workspace && !aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  float* ws = static_cast<float*>(workspace);
  float* up = L.rank > 0 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.u_offset) : nullptr;
  int st;
  if (L.rank > 0 && (st = run_lora_u(L, p.u_splits, up, stream)) != RQ_OK) return st;
  const LinearEpi e = make_epi(L, up, p.u_splits);
  if (L.x_dtype == RQ_DTYPE_BF16) st = run_gemv<RQ_DTYPE_BF16>(L, p, e, ws, stream);
  else st = run_gemv<RQ_DTYPE_F16>(L, p, e, ws, stream);
  if (st != RQ_OK || p.S == 1) return st;
  if (L.x_dtype == RQ_DTYPE_BF16) return launch_splitk_epilogue<RQ_DTYPE_BF16>(L, p, e, ws, stream);
  return launch_splitk_epilogue<RQ_DTYPE_F16>(L, p, e, ws, stream);
}

}  // namespace rq

// ===========================================================================
// C ABI
// ===========================================================================
using namespace rq;

static LinearArgs pack_linear_args(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                                   const uint8_t* w_packed, int64_t N, int64_t block_size,
                                   const void* absmax, int absmax_dtype, const uint8_t* c2, int c2_format,
                                   int64_t block2, const void* bias, int bias_dtype, const void* lora_x,
                                   int64_t ld_lora_x, const void* lora_a, const void* lora_b,
                                   int64_t ld_lora_b, int lora_dtype, int64_t rank, float scaling, void* y,
                                   int64_t ldy) {
  LinearArgs L;
  L.x = x; L.x_dtype = x_dtype; L.M = M; L.K = K; L.ldx = ldx;
  L.w_packed = w_packed; L.N = N; L.block_size = block_size;
  L.absmax = absmax; L.absmax_dtype = absmax_dtype;
  L.c2 = c2; L.c2_format = c2_format; L.block2 = block2;
  L.bias = bias; L.bias_dtype = bias_dtype;
  L.lora_x = lora_x ? lora_x : x; L.ld_lora_x = lora_x ? ld_lora_x : ldx;
  L.lora_a = lora_a; L.lora_b = lora_b; L.ld_lora_b = ld_lora_b; L.lora_dtype = lora_dtype;
  L.rank = (lora_a && lora_b) ? rank : 0; L.scaling = scaling;
  L.y = y; L.ldy = ldy;
  return L;
}

extern "C" int rq_nf4_linear_workspace_size(int x_dtype, int64_t M, int64_t K, int64_t N, int64_t rank,
                                            int64_t* bytes) {
  if (!bytes) return RQ_ERR_NULL_POINTER;
  if (x_dtype != RQ_DTYPE_BF16 && x_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || N < 1 || K < 64 || K % 64 || rank < 0 || rank > 256) return RQ_ERR_BAD_SHAPE;
  size_t b = 0;
  LinearArgs L{};
  L.x_dtype = x_dtype; L.M = M; L.K = K; L.N = N; L.rank = rank;
  int st = M <= kGemvMaxM ? gemv_workspace(L, &b) : gemm_workspace(L, &b);
  *bytes = int64_t(b);
  return st;
}

extern "C" int rq_nf4_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                             const uint8_t* w_packed, int64_t N, int64_t block_size, const void* absmax,
                             int absmax_dtype, const uint8_t* c2, int c2_format, int64_t block2,
                             const void* bias, int bias_dtype, const void* lora_x, int64_t ld_lora_x,
                             const void* lora_a, const void* lora_b, int64_t ld_lora_b, int lora_dtype,
                             int64_t rank, float scaling, void* y, int64_t ldy, void* workspace,
                             int64_t workspace_bytes, hipStream_t stream) {
  const LinearArgs L = pack_linear_args(x, x_dtype, M, K, ldx, w_packed, N, block_size, absmax, absmax_dtype,
                                        c2, c2_format, block2, bias, bias_dtype, lora_x, ld_lora_x, lora_a,
                                        lora_b, ld_lora_b, lora_dtype, rank, scaling, y, ldy);
  int st = validate_linear(L);
  if (st != RQ_OK || M == 0) return st;
  if (workspace_bytes < 0) return RQ_ERR_BAD_SHAPE;
  if (M <= kGemvMaxM) return run_nf4_gemv(L, workspace, size_t(workspace_bytes), stream);
  return run_nf4_gemm(L, workspace, size_t(workspace_bytes), stream);
}
