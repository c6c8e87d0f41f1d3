// LoRA operand preparation for the prefill GEMM and the dX kernel (many
// activation rows).  lora_layer.py:67-70 rounds every intermediate to the
// activation dtype:
//   forward  u = RND(xl . RND(A)^T)                   [M, r]
//   backward g = RND(RND(dY * s) . RND(B))            [M, r] (lora_layer.py:67
//            differentiated: dX += RND(g . RND(A)))
// The kernels here produce u / g as [rows, r16] 16-bit operands (r16 = r
// rounded up to 16, zero padded) that the GEMM epilogues stage into LDS:
//   lora_rows_kernel     fp32 partial sums of a split-K MFMA product
//                        X[rows, K] . RND(S)[r, K]^T; S is rounded as it is
//                        staged, from contiguous rows (A) or, transposed in
//                        LDS, from contiguous columns (S = B^T);
//   lora_finish_kernel   sum of the partials in split order, rounded.
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"
#include "rq_lora.h"

namespace rq {

constexpr int kLoraChunkK = 256;   // k per LDS stage of S
constexpr int kLoraSPitch = kLoraChunkK + 8;
constexpr int kLoraMaxSplits = 16;

// X[m, k] (16-bit, row stride ldx) times RND(S)[j, k] over k in this split's
// range, for the 16 W activation rows (W waves of 16) and the 16 JB ranks
// j0 .. j0 + 16 JB - 1 of this workgroup, where
// S[j][k] = s[j * s_j + k * s_k] (dtype sdt) and j < R (zeros past R).
// s_rows: s_k == 1 (each rank's row contiguous); otherwise s_j == 1 and each
// k holds the ranks contiguously, and the staging transposes them.
// PRESCALE multiplies each x element by `prescale` and rounds it to XT
// first.  Output: part[ks][m][j] fp32 for m < M, j < R.  At most 128 VGPRs
// (four waves per SIMD), so that two 8-wave workgroups share a compute unit.
template <int XT, bool PRESCALE, int JB, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(4))) void lora_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M,
                                                        int64_t K, const void* __restrict__ s, int sdt, int64_t s_j,
                                                        int64_t s_k, bool s_rows, bool svec, int R, float prescale,
                                                        int64_t k_per_split, float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint16_t ss[16 * JB * kLoraSPitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, q4 = lane >> 4;
  constexpr int NT = 64 * W;
  const int64_t m0 = int64_t(blockIdx.x) * 16 * W;
  const int j0 = blockIdx.y * 16 * JB;
  const int ks = blockIdx.z;
  const int64_t k0 = int64_t(ks) * k_per_split;
  const int64_t k1 = k0 + k_per_split < K ? k0 + k_per_split : K;
  int64_t m = m0 + 16 * wave + i16;
  m = m < M ? m : M - 1;
  const uint16_t* xr = x + m * ldx;
  f32x4 acc[JB];
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) acc[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t kc = k0; kc < k1; kc += kLoraChunkK) {
    const int len = int(k1 - kc < kLoraChunkK ? k1 - kc : kLoraChunkK);  // multiple of 64
    // this lane's activation fragments of the whole chunk, issued before the
    // staging so that their latency overlaps it
    u32x4 xf[kLoraChunkK / 32];
#pragma unroll
    for (int t = 0; t < kLoraChunkK / 32; ++t)
      if (32 * t < len) xf[t] = *reinterpret_cast<const u32x4*>(xr + kc + 32 * t + 8 * q4);
    __syncthreads();
    if (s_rows) {
      // 16 JB ranks x len in 16-byte chunks, CPR per rank: thread tid takes
      // chunk tid % CPR of ranks tid / CPR + (NT / CPR) i
      constexpr int CPR = kLoraChunkK / 8;
      const int c = tid % CPR;
#pragma unroll
      for (int i = 0; i < 16 * JB / (NT / CPR); ++i) {
        const int jj = tid / CPR + (NT / CPR) * i, j = j0 + jj;
        if (8 * c < len) {
          const u32x4 v = load_a8<XT>(s, sdt, int64_t(j) * s_j + kc + 8 * c, j < R, svec);
          *reinterpret_cast<u32x4*>(ss + jj * kLoraSPitch + 8 * c) = v;
        }
      }
    } else {
      // len k x 16 JB ranks: thread tid takes k = tid % 256, ranks 8 i ..
      // 8 i + 7 for i = tid / 256 + (NT / 256) n (eight contiguous values,
      // stored down one LDS column)
      static_assert(kLoraChunkK == 256 && NT % 256 == 0, "one k of the chunk per thread");
      const int kk = tid % 256;
      if (kk < len) {
#pragma unroll
        for (int n = 0; n < (2 * JB + NT / 256 - 1) / (NT / 256); ++n) {
          const int i = tid / 256 + (NT / 256) * n;
          if (i >= 2 * JB) break;
          const int j = j0 + 8 * i;
          const u32x4 v = j < R ? load_a8_masked<XT>(s, sdt, (kc + kk) * s_k + j, R - j, svec)
                                : u32x4{0u, 0u, 0u, 0u};
          const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            ss[(8 * i + e) * kLoraSPitch + kk] = uint16_t(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xFFFFu);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < kLoraChunkK / 32; ++t) {
      if (32 * t >= len) break;
      u32x4 xa = xf[t];
      if constexpr (PRESCALE) {
        uint32_t w[4] = {xa.x, xa.y, xa.z, xa.w};
#pragma unroll
        for (int h = 0; h < 4; ++h)
          w[h] = cvt_pk<XT>(__fmul_rn(from_x16<XT>(w[h] & 0xFFFFu), prescale),
                            __fmul_rn(from_x16<XT>(w[h] >> 16), prescale));
        xa = u32x4{w[0], w[1], w[2], w[3]};
      }
#pragma unroll
      for (int jb = 0; jb < JB; ++jb) {
        const u32x4 b = *reinterpret_cast<const u32x4*>(ss + (16 * jb + i16) * kLoraSPitch + 32 * t + 8 * q4);
        acc[jb] = mfma16x16x32<XT>(xa, b, acc[jb]);
      }
    }
  }
  // D[r][c] of block jb: row 4 q4 + r of the wave's 16, rank 16 jb + i16
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) {
    const int j = j0 + 16 * jb + i16;
    if (j >= R) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t mo = m0 + 16 * wave + 4 * q4 + r;
      if (mo < M) part[(int64_t(ks) * M + mo) * R + j] = acc[jb][r];
    }
  }
}

// out[m][j] = RND(0 + part[0][m][j] + part[1][m][j] + ...) for j < R, 0
// for R <= j < R16; each thread produces 4 consecutive outputs (one 8-byte
// store) and keeps up to 16 splits' loads in flight.
template <int XT>
__global__ __launch_bounds__(256) void lora_finish_kernel(const float* __restrict__ part, int KS, int64_t M, int R,
                                                          int R16, uint16_t* __restrict__ out) {
  const int64_t i4 = int64_t(blockIdx.x) * 256 + threadIdx.x;  // index of 4 outputs
  const int per_row = R16 / 4;
  if (i4 >= M * per_row) return;
  const int64_t m = i4 / per_row;
  const int j0 = int(i4 - m * per_row) * 4;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (R % 4 == 0) {
    if (j0 < R) {
      const f32x4* src = reinterpret_cast<const f32x4*>(part + m * R + j0);
      const int64_t step = M * R / 4;  // one split, in f32x4
      for (int k = 0; k < KS; k += 16) {
        f32x4 a[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) a[t] = src[int64_t(k + t < KS ? k + t : k) * step];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          if (k + t < KS) {
            v[0] = __fadd_rn(v[0], a[t].x);
            v[1] = __fadd_rn(v[1], a[t].y);
            v[2] = __fadd_rn(v[2], a[t].z);
            v[3] = __fadd_rn(v[3], a[t].w);
          }
        }
      }
    }
  } else {
    for (int k = 0; k < KS; ++k) {
      const float* src = part + (int64_t(k) * M + m) * R;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (j0 + e < R) v[e] = __fadd_rn(v[e], src[j0 + e]);
    }
  }
  *reinterpret_cast<uint2*>(out + m * R16 + j0) = uint2{cvt_pk<XT>(v[0], v[1]), cvt_pk<XT>(v[2], v[3])};
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
LoraRowsPlan plan_lora_rows(int64_t M, int64_t K, int64_t R, int cus) {
  LoraRowsPlan p{};
  const int64_t r16 = (R + 15) / 16 * 16;
  p.jb = r16 <= 16 ? 1 : (r16 <= 32 ? 2 : 4);
  // 128 activation rows per workgroup with 64 ranks (each rank block read
  // for twice the rows), else 64
  p.waves = p.jb == 4 ? 8 : 4;
  const int64_t rows = 16 * p.waves;
  const int64_t tiles = ((M + rows - 1) / rows) * ((r16 + 16 * p.jb - 1) / (16 * p.jb));
  const int64_t steps = K / 64;
  // about two workgroups per compute unit, at most 8 steps (two LDS chunks)
  // per split and at least 2 unless that leaves too many splits for the
  // partials
  int64_t ks = (2 * cus + tiles - 1) / tiles;
  const int64_t ks_len = (steps + 7) / 8;
  ks = ks < ks_len ? ks_len : ks;
  ks = ks > steps / 2 ? steps / 2 : ks;
  ks = ks > kLoraMaxSplits ? (ks_len > kLoraMaxSplits ? ks_len : int64_t(kLoraMaxSplits)) : ks;
  ks = ks < 1 ? 1 : ks;
  const int64_t steps_per = (steps + ks - 1) / ks;
  p.k_per_split = steps_per * 64;
  p.splits = int((K + p.k_per_split - 1) / p.k_per_split);
  p.part_bytes = (size_t(p.splits) * M * R * 4 + 255) & ~size_t(255);
  return p;
}

template <int XT, bool PRESCALE, int JB, int W>
static void launch_rows_jb(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const void* s, int sdt,
                           int64_t s_j, int64_t s_k, bool s_rows, bool svec, int R, float prescale,
                           const LoraRowsPlan& p, float* part, hipStream_t stream) {
  dim3 grid(unsigned((M + 16 * W - 1) / (16 * W)), unsigned((R + 16 * JB - 1) / (16 * JB)), unsigned(p.splits));
  lora_rows_kernel<XT, PRESCALE, JB, W><<<grid, 64 * W, 0, stream>>>(x, ldx, M, K, s, sdt, s_j, s_k, s_rows, svec, R,
                                                               prescale, p.k_per_split, part);
}

template <int XT, bool PRESCALE>
static void launch_rows_t(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const void* s, int sdt, int64_t s_j,
                          int64_t s_k, bool s_rows, bool svec, int R, float prescale, const LoraRowsPlan& p,
                          float* part, hipStream_t stream) {
  if (p.jb == 1)
    launch_rows_jb<XT, PRESCALE, 1, 4>(x, ldx, M, K, s, sdt, s_j, s_k, s_rows, svec, R, prescale, p, part, stream);
  else if (p.jb == 2)
    launch_rows_jb<XT, PRESCALE, 2, 4>(x, ldx, M, K, s, sdt, s_j, s_k, s_rows, svec, R, prescale, p, part, stream);
  else
    launch_rows_jb<XT, PRESCALE, 4, 8>(x, ldx, M, K, s, sdt, s_j, s_k, s_rows, svec, R, prescale, p, part, stream);
}

int run_lora_rows(int xt, const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const void* s, int s_dt,
                  int64_t s_j, int64_t s_k, int R, bool prescale, float scale, const LoraRowsPlan& p, float* part,
                  uint16_t* out, int R16, hipStream_t stream) {
  if (!aligned(x, 16) || ldx % 8 != 0 || K % 64 != 0) return RQ_ERR_BAD_ALIGNMENT;
  if (s_k != 1 && s_j != 1) return RQ_ERR_BAD_SHAPE;
  // contiguous runs of S are read 16 bytes at a time when aligned
  const bool s_rows = s_k == 1;
  const int64_t run_stride = s_rows ? s_j : s_k;
  const bool svec = aligned(s, 16) && (s_dt != RQ_DTYPE_F32 || run_stride % 4 == 0);
  if (xt == RQ_DTYPE_BF16) {
    if (prescale)
      launch_rows_t<RQ_DTYPE_BF16, true>(x, ldx, M, K, s, s_dt, s_j, s_k, s_rows, svec, R, scale, p, part, stream);
    else
      launch_rows_t<RQ_DTYPE_BF16, false>(x, ldx, M, K, s, s_dt, s_j, s_k, s_rows, svec, R, scale, p, part, stream);
  } else {
    if (prescale)
      launch_rows_t<RQ_DTYPE_F16, true>(x, ldx, M, K, s, s_dt, s_j, s_k, s_rows, svec, R, scale, p, part, stream);
    else
      launch_rows_t<RQ_DTYPE_F16, false>(x, ldx, M, K, s, s_dt, s_j, s_k, s_rows, svec, R, scale, p, part, stream);
  }
  int st = rq_check_launch();
  if (st != RQ_OK) return st;
  const unsigned blocks = unsigned((M * (R16 / 4) + 255) / 256);
  if (xt == RQ_DTYPE_BF16)
    lora_finish_kernel<RQ_DTYPE_BF16><<<blocks, 256, 0, stream>>>(part, p.splits, M, R, R16, out);
  else
    lora_finish_kernel<RQ_DTYPE_F16><<<blocks, 256, 0, stream>>>(part, p.splits, M, R, R16, out);
  return rq_check_launch();
}

}  // namespace rq
