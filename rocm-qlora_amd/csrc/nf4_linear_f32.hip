// NF4 quantized linear with fp32 activations (+ bias, + LoRA) for gfx950, on
// the fp32 matrix cores (v_mfma_f32_16x16x4_f32).
//
// For fp32 inputs the reference computes everything in fp32
// (quant_linear.py:189-197: W = dequantize_int4(...) is fp32 and .to(x.dtype)
// keeps it; F.linear(x, W, bias); lora_layer.py:67: (x @ A^T) @ B^T * s with
// A, B in fp32):
//   base[m,n] = sum_k x[m,k] * W[n,k] + bias[n],  W = T[code] * scale (fp32)
//   u[m,j]    = sum_k x[m,k] * A[j,k]
//   y[m,n]    = base[m,n] + (sum_j u[m,j] * B[n,j]) * scaling
// The weight operand is T[code] * scale rounded once to fp32 -- the value
// dequantize_int4 produces -- and every product and sum is an fp32 MFMA
// operation, so the result differs from the reference's only in the order of
// the fp32 sums.
//
// Layout of one 16 x 16 x 4 step (checked by the parity tests): lane l holds
// A[l % 16][l / 16] (activation row m, k group q = l / 16), B[l / 16][l % 16]
// (k group q, weight row n), and D[4 (l / 16) + r][l % 16] in register r.
// Within a chunk of 128 k, lane group q owns k = 128 i + 32 q + 8 d + e
// (d = 0..3 code dword, e = 0..7 code in the dword): each lane reads one 16-byte
// piece of packed codes (32 codes of its row) and 32 activations of its row,
// and step (d, e) of the 32 steps multiplies the k set {32 q + 8 d + e}.
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"

namespace rq {

constexpr int kF32Threads = 1024;  // sixteen waves; wave w takes chunks w, w + 16, ...
constexpr int kF32Waves = kF32Threads / 64;
constexpr int kF32ChunkK = 128;

__device__ __forceinline__ f32x4 mfma16x16x4_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// 32 consecutive values of a row (fp32 or 16-bit, widened exactly to fp32),
// zeros where the row or the k range is past the end.
template <int DT>
__device__ __forceinline__ void load32_f32(const void* p, int64_t off, bool live, float (&v)[32]) {
  if (!live) {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = 0.0f;
    return;
  }
  if constexpr (DT == RQ_DTYPE_F32) {
    const f32x4* s = reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + off);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f32x4 t = s[i];
      v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
  } else {
    const u32x4* s = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 t = s[i];
      const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        v[8 * i + 2 * h] = DT == RQ_DTYPE_BF16 ? bf16_to_f32(uint16_t(w[h])) : f16_to_f32(uint16_t(w[h]));
        v[8 * i + 2 * h + 1] = DT == RQ_DTYPE_BF16 ? bf16_to_f32(uint16_t(w[h] >> 16))
                                                   : f16_to_f32(uint16_t(w[h] >> 16));
      }
    }
  }
}

// y rows [m0, m0 + 16) (fewer when M is shorter) of one 16-row weight tile.
// The sixteen waves take the tile's 128-k chunks in turn, two chunks' loads
// in flight per wave; their partials are summed in wave order.
// u: fp32 LoRA operand partials [usplits][M][rank] (rank 0: none), summed in
// split order.
template <class Scale>
__global__ __launch_bounds__(kF32Threads) void nf4_gemv_f32_kernel(const float* __restrict__ x, int64_t ldx,
                                                                   int64_t M, int64_t K,
                                                                   const uint8_t* __restrict__ packed, int64_t N,
                                                                   int bs_log2, Scale scale, LinearEpi e,
                                                                   int usplits) {
  __shared__ float tab[16];
  __shared__ float red[kF32Waves][16][16];
  __shared__ float us[16][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, q = lane >> 4;
  const int64_t n0 = int64_t(blockIdx.x) * 16;
  if (tid < 16) tab[tid] = u2f(kNF4Bits[tid]);
  __syncthreads();
  const int64_t n = n0 + i16;               // weight row of this lane's B operands
  const bool nlive = n < N;
  const int64_t row_bytes = K / 2;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int64_t nchunks = (K + kF32ChunkK - 1) / kF32ChunkK;
  struct Chunk {
    u32x4 codes;
    float s;
    float xv[32];
  };
  auto load = [&](Chunk& ch, int64_t c) {
    const int64_t k0 = c * kF32ChunkK + 32 * q;  // this lane group's 32 k
    const bool live = c < nchunks && k0 < K;
    ch.codes = u32x4{0u, 0u, 0u, 0u};
    ch.s = 0.0f;
    if (nlive && live) {
      ch.codes = *reinterpret_cast<const u32x4*>(packed + n * row_bytes + k0 / 2);
      ch.s = scale((n * K + k0) >> bs_log2);
    }
    load32_f32<RQ_DTYPE_F32>(x, i16 * ldx + k0, i16 < M && live, ch.xv);
  };
  auto compute = [&](const Chunk& ch) {
    const uint32_t w[4] = {ch.codes.x, ch.codes.y, ch.codes.z, ch.codes.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int ee = 0; ee < 8; ++ee) {
        const float wv = __fmul_rn(tab[(w[d] >> (4 * ee)) & 15u], ch.s);
        acc = mfma16x16x4_f32(ch.xv[8 * d + ee], wv, acc);
      }
    }
  };
  for (int64_t c = wave; c < nchunks; c += 2 * kF32Waves) {
    Chunk c0, c1;
    load(c0, c);
    load(c1, c + kF32Waves);
    compute(c0);
    compute(c1);  // a chunk past the end has zero codes, scale and activations
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][4 * q + r][i16] = acc[r];
  // the LoRA operand rows of this launch's activation rows: the splits'
  // partials summed in split order
  const int rank = e.rank;
  for (int idx = tid; idx < 16 * rank; idx += kF32Threads) {
    const int m = idx / rank, j = idx - m * rank;
    float v = 0.0f;
    if (m < M)
      for (int sp = 0; sp < usplits; ++sp) v = __fadd_rn(v, e.u[(int64_t(sp) * M + m) * rank + j]);
    us[m][j] = v;
  }
  __syncthreads();
  // one thread per output (row m = tid / 16, column n0 + tid % 16)
  if (tid >= 256) return;
  const int m = tid >> 4, nn = tid & 15;
  const int64_t on = n0 + nn;
  if (m >= M || on >= N) return;
  float v = 0.0f;
#pragma unroll
  for (int w2 = 0; w2 < kF32Waves; ++w2) v = __fadd_rn(v, red[w2][m][nn]);
  if (e.bias) v = __fadd_rn(v, load_as_f32(e.bias, on, e.bias_dt));
  if (rank > 0) {
    float l = 0.0f;
    for (int j = 0; j < rank; ++j) l = __fmaf_rn(us[m][j], load_as_f32(e.lora_b, on * e.ld_lora_b + j, e.lora_dt), l);
    v = __fadd_rn(v, __fmul_rn(l, e.scaling));
  }
  static_cast<float*>(e.y)[m * e.ldy + on] = v;
}

// A few activation rows (M <= 4) on the vector ALUs: the 16 x 16 x 4 MFMA
// spends sixteen rows' work whatever M is, so at decode sizes the products are
// plain fp32 FMAs.  One workgroup of eight waves takes 16 weight rows; wave w
// takes the K segments s = w, w + 8, ... of 512 k, and in a segment lane l
// owns weight rows 4 i + l / 16 (i = 0..3) and k = 512 s + 32 (l % 16) + [0, 32):
// four 16-byte code loads, one scale each, and the 32 activations of each of
// the MR rows, shared by the four weight rows.  Per lane the products are
// summed in k order, the 16 lanes of a row by DPP swaps, the waves in wave
// order; the weight value is RND(T[code] * scale), as the MFMA kernel uses.
// v from the lane that DPP control CTRL names within the 16-lane row
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v),
                                                               CTRL, 0xF, 0xF, false));
}

// Sum over a 16-lane DPP row (lanes 16 r .. 16 r + 15): xor 1, xor 2, then
// lane 7 - i and lane 15 - i within the row; lane 16 r holds the row's sum.
__device__ __forceinline__ float row16_sum(float v) {
  v = __fadd_rn(v, dpp_f32<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = __fadd_rn(v, dpp_f32<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = __fadd_rn(v, dpp_f32<0x141>(v));  // row_half_mirror
  return __fadd_rn(v, dpp_f32<0x140>(v));  // row_mirror
}

constexpr int kF32vThreads = 512;
constexpr int kF32vWaves = kF32vThreads / 64;
constexpr int kF32vSegK = 512;
constexpr int kF32vPre = 2;  // epilogue operands requested per thread before the weight stream

template <class Scale, int MR>
__global__ __launch_bounds__(kF32vThreads) void nf4_gemv_f32v_kernel(const float* __restrict__ x, int64_t ldx,
                                                                     int64_t M, int64_t K,
                                                                     const uint8_t* __restrict__ packed, int64_t N,
                                                                     int bs_log2, Scale scale, LinearEpi e,
                                                                     int usplits) {
  __shared__ float tab[16];
  __shared__ float red[kF32vWaves][16][MR];
  __shared__ float us[MR][64];
  __shared__ float bsh[16];                         // bias of the tile's columns
  __shared__ float lbs[16 * 64];                    // LoRA B rows of the tile's columns
  __shared__ float ups[kF32vPre * kF32vThreads];    // u partials as laid out in e.u
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j16 = lane & 15, g = lane >> 4;
  const int64_t n0 = int64_t(blockIdx.x) * 16;
  if (tid < 16) tab[tid] = u2f(kNF4Bits[tid]);
  // The epilogue's operands are requested before the weight stream so that
  // their latency hides under it: B rows [16][rank], the bias, and (when they
  // fit kF32vPre per thread) the u partials [usplits][M][rank].
  const int rank = e.rank;
  const int nb = 16 * rank;
  const int64_t nu = int64_t(usplits) * M * rank;
  const bool u_pre = nu <= int64_t(kF32vPre) * kF32vThreads;
  float bpre[kF32vPre], upre[kF32vPre];
#pragma unroll
  for (int p = 0; p < kF32vPre; ++p) {
    const int idx = tid + p * kF32vThreads;
    const int64_t bn = n0 + (rank > 0 ? idx / rank : 0);
    bpre[p] = idx < nb && bn < N ? load_as_f32(e.lora_b, bn * e.ld_lora_b + (idx - (idx / rank) * rank), e.lora_dt)
                                 : 0.0f;
    upre[p] = u_pre && idx < nu ? e.u[idx] : 0.0f;
  }
  const float bias_v = e.bias && tid < 16 && n0 + tid < N ? load_as_f32(e.bias, n0 + tid, e.bias_dt) : 0.0f;
  __syncthreads();
  const int64_t row_bytes = K / 2;
  const int64_t nseg = (K + kF32vSegK - 1) / kF32vSegK;
  float acc[4][MR];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[i][m] = 0.0f;
  for (int64_t s = wave; s < nseg; s += kF32vWaves) {
    const int64_t k0 = s * kF32vSegK + 32 * j16;  // K % 64 == 0: a live lane's 32 k are all in range
    const bool klive = k0 < K;
    // activations first: row group i can then start as soon as its own
    // codes and scale arrive, while later groups' loads are still in flight
    float xv[MR][32];
#pragma unroll
    for (int m = 0; m < MR; ++m) load32_f32<RQ_DTYPE_F32>(x, m * ldx + k0, m < M && klive, xv[m]);
    u32x4 codes[4];
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = n0 + 4 * i + g;
      codes[i] = u32x4{0u, 0u, 0u, 0u};
      sc[i] = 0.0f;
      if (klive && n < N) {
        codes[i] = *reinterpret_cast<const u32x4*>(packed + n * row_bytes + k0 / 2);
        sc[i] = scale((n * K + k0) >> bs_log2);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w[4] = {codes[i].x, codes[i].y, codes[i].z, codes[i].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int ee = 0; ee < 8; ++ee) {
          const float wv = __fmul_rn(tab[(w[d] >> (4 * ee)) & 15u], sc[i]);
#pragma unroll
          for (int m = 0; m < MR; ++m) acc[i][m] = __fmaf_rn(xv[m][8 * d + ee], wv, acc[i][m]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float v = row16_sum(acc[i][m]);
      if (j16 == 0) red[wave][4 * i + g][m] = v;
    }
#pragma unroll
  for (int p = 0; p < kF32vPre; ++p) {
    lbs[tid + p * kF32vThreads] = bpre[p];
    ups[tid + p * kF32vThreads] = upre[p];
  }
  if (tid < 16) bsh[tid] = bias_v;
  if (!u_pre)  // more partials than the prefetch holds: summed here from memory
    for (int idx = tid; idx < MR * rank; idx += kF32vThreads) {
      const int m = idx / rank, j = idx - m * rank;
      float v = 0.0f;
      if (m < M)
        for (int sp = 0; sp < usplits; ++sp) v = __fadd_rn(v, e.u[(int64_t(sp) * M + m) * rank + j]);
      us[m][j] = v;
    }
  __syncthreads();
  if (u_pre)  // the partials in split order, as above
    for (int idx = tid; idx < MR * rank; idx += kF32vThreads) {
      const int m = idx / rank, j = idx - m * rank;
      float v = 0.0f;
      if (m < M)
        for (int sp = 0; sp < usplits; ++sp) v = __fadd_rn(v, ups[(sp * int(M) + m) * rank + j]);
      us[m][j] = v;
    }
  __syncthreads();
  // one thread per output (row m = tid / 16, column n0 + tid % 16)
  if (tid >= 16 * MR) return;
  const int m = tid >> 4, nn = tid & 15;
  const int64_t on = n0 + nn;
  if (m >= M || on >= N) return;
  float v = 0.0f;
#pragma unroll
  for (int w2 = 0; w2 < kF32vWaves; ++w2) v = __fadd_rn(v, red[w2][nn][m]);
  if (e.bias) v = __fadd_rn(v, bsh[nn]);
  if (rank > 0) {
    float l = 0.0f;
    for (int j = 0; j < rank; ++j) l = __fmaf_rn(us[m][j], lbs[nn * rank + j], l);
    v = __fadd_rn(v, __fmul_rn(l, e.scaling));
  }
  static_cast<float*>(e.y)[m * e.ldy + on] = v;
}

// Partials of u[m, j] = sum_k xl[m, k] * A[j, k] in fp32 for m < M <= 16:
// workgroup (j0 / 16, sp) takes ranks [j0, j0 + 16) over K split sp (chunks
// 2 sp and 2 sp + 1 of 128 k, one per wave); the two waves' products are
// summed in wave order into u[sp][m][j].
constexpr int kLuThreads = 128;
constexpr int kLuWaves = kLuThreads / 64;

template <int ADT>
__global__ __launch_bounds__(kLuThreads) void lora_u_f32_kernel(const float* __restrict__ xl, int64_t ldxl,
                                                                int64_t M, int64_t K, const void* __restrict__ A,
                                                                int rank, float* __restrict__ u) {
  __shared__ float red[kLuWaves][16][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, q = lane >> 4;
  const int j = int(blockIdx.x) * 16 + i16;
  const int64_t c = int64_t(blockIdx.y) * kLuWaves + wave;
  const int64_t k0 = c * kF32ChunkK;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (k0 < K) {
    float xv[32], av[32];
    const int64_t kq = k0 + 32 * q;
    load32_f32<RQ_DTYPE_F32>(xl, i16 * ldxl + kq, i16 < M && kq < K, xv);
    load32_f32<ADT>(A, int64_t(j) * K + kq, j < rank && kq < K, av);
#pragma unroll
    for (int t = 0; t < 32; ++t) acc = mfma16x16x4_f32(xv[t], av[t], acc);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][4 * q + r][i16] = acc[r];
  __syncthreads();
  for (int o = tid; o < 256; o += kLuThreads) {
    const int m = o >> 4, jj = int(blockIdx.x) * 16 + (o & 15);
    if (m >= M || jj >= rank) continue;
    float v = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < kLuWaves; ++w2) v = __fadd_rn(v, red[w2][m][o & 15]);
    u[(int64_t(blockIdx.y) * M + m) * rank + jj] = v;
  }
}

// K splits of the LoRA operand: one chunk of 128 k per wave of lora_u_f32_kernel.
inline int f32_usplits(int64_t K) { return int((K + kLuWaves * kF32ChunkK - 1) / (kLuWaves * kF32ChunkK)); }

template <class Scale>
static int launch_f32_gemv(const LinearArgs& L, int64_t m0, int64_t rows, Scale scale, const LinearEpi& e,
                           hipStream_t stream) {
  const int usplits = L.rank > 0 ? f32_usplits(L.K) : 0;
  const float* x = static_cast<const float*>(L.x) + m0 * L.ldx;
  LinearEpi ec = e;
  ec.y = static_cast<float*>(L.y) + m0 * L.ldy;
  const unsigned grid = unsigned((L.N + 15) / 16);
  const int bs = pow2_shift(L.block_size);
  if (rows <= 4) {  // vector-ALU kernel: MR = rows rounded up to 1, 2 or 4
    if (rows == 1)
      nf4_gemv_f32v_kernel<Scale, 1><<<grid, kF32vThreads, 0, stream>>>(x, L.ldx, rows, L.K, L.w_packed, L.N, bs,
                                                                       scale, ec, usplits);
    else if (rows == 2)
      nf4_gemv_f32v_kernel<Scale, 2><<<grid, kF32vThreads, 0, stream>>>(x, L.ldx, rows, L.K, L.w_packed, L.N, bs,
                                                                       scale, ec, usplits);
    else
      nf4_gemv_f32v_kernel<Scale, 4><<<grid, kF32vThreads, 0, stream>>>(x, L.ldx, rows, L.K, L.w_packed, L.N, bs,
                                                                       scale, ec, usplits);
    return rq_check_launch();
  }
  nf4_gemv_f32_kernel<Scale><<<grid, kF32Threads, 0, stream>>>(x, L.ldx, rows, L.K, L.w_packed, L.N,
                                                               pow2_shift(L.block_size), scale, ec, usplits);
  return rq_check_launch();
}

template <class Scale>
static int run_f32_rows(const LinearArgs& L, int64_t m0, int64_t rows, Scale scale, float* u, hipStream_t stream) {
  LinearEpi e = make_epi(L, u, 1);
  if (L.rank > 0) {
    const float* xl = static_cast<const float*>(L.lora_x) + m0 * L.ld_lora_x;
    const dim3 grid(unsigned((L.rank + 15) / 16), unsigned(f32_usplits(L.K)));
    switch (L.lora_dtype) {
      case RQ_DTYPE_F32:
        lora_u_f32_kernel<RQ_DTYPE_F32><<<grid, kLuThreads, 0, stream>>>(xl, L.ld_lora_x, rows, L.K, L.lora_a,
                                                                          int(L.rank), u);
        break;
      case RQ_DTYPE_BF16:
        lora_u_f32_kernel<RQ_DTYPE_BF16><<<grid, kLuThreads, 0, stream>>>(xl, L.ld_lora_x, rows, L.K, L.lora_a,
                                                                           int(L.rank), u);
        break;
      default:
        lora_u_f32_kernel<RQ_DTYPE_F16><<<grid, kLuThreads, 0, stream>>>(xl, L.ld_lora_x, rows, L.K, L.lora_a,
                                                                          int(L.rank), u);
        break;
    }
    if (int st = rq_check_launch(); st != RQ_OK) return st;
  }
  return launch_f32_gemv(L, m0, rows, scale, e, stream);
}

template <class Scale>
static int run_f32_all(const LinearArgs& L, Scale scale, float* u, hipStream_t stream) {
  // 16 activation rows per launch pair (the MFMA's row count); larger M runs
  // as consecutive row blocks
  for (int64_t m0 = 0; m0 < L.M; m0 += 16) {
    const int64_t rows = L.M - m0 < 16 ? L.M - m0 : 16;
    if (int st = run_f32_rows(L, m0, rows, scale, u, stream); st != RQ_OK) return st;
  }
  return RQ_OK;
}

// The LoRA operand partials [usplits][16][rank] lie after the workspace's
// synchronization area (which every rq_nf4_linear call leaves zero for the
// decode GEMV).
int f32_linear_workspace(const LinearArgs& L, size_t* bytes) {
  *bytes = L.rank > 0 ? kLinearSyncBytes + size_t(f32_usplits(L.K)) * 16 * size_t(L.rank) * 4 : 0;
  return RQ_OK;
}

int run_nf4_linear_f32(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  size_t need = 0;
  f32_linear_workspace(L, &need);
  if (need > 0 && (!workspace || ws_bytes < need)) return RQ_ERR_WORKSPACE;
  if (L.rank > 64) return RQ_ERR_UNSUPPORTED;  // the epilogue stages 64 ranks per activation row
  // 16-byte loads of activations, codes and (fp32) LoRA A rows
  if (!aligned(L.x, 16) || L.ldx % 4 != 0 || !aligned(L.w_packed, 16) || L.K % 64 != 0) return RQ_ERR_BAD_ALIGNMENT;
  if (L.rank > 0 && (!aligned(L.lora_x, 16) || L.ld_lora_x % 4 != 0 || !aligned(L.lora_a, 16)))
    return RQ_ERR_BAD_ALIGNMENT;
  float* u = L.rank > 0 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kLinearSyncBytes) : nullptr;
  if (L.c2) {
    const int sh = pow2_shift(L.block2);
    switch (L.absmax_dtype) {
      case RQ_DTYPE_F32: return run_f32_all(L, ScaleDQ<RQ_DTYPE_F32>{L.c2, L.absmax, L.c2_format, sh, L.block2}, u, stream);
      case RQ_DTYPE_BF16: return run_f32_all(L, ScaleDQ<RQ_DTYPE_BF16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, u, stream);
      default: return run_f32_all(L, ScaleDQ<RQ_DTYPE_F16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, u, stream);
    }
  }
  switch (L.absmax_dtype) {
    case RQ_DTYPE_F32: return run_f32_all(L, ScaleAbsmax<RQ_DTYPE_F32>{L.absmax}, u, stream);
    case RQ_DTYPE_BF16: return run_f32_all(L, ScaleAbsmax<RQ_DTYPE_BF16>{L.absmax}, u, stream);
    default: return run_f32_all(L, ScaleAbsmax<RQ_DTYPE_F16>{L.absmax}, u, stream);
  }
}

}  // namespace rq
