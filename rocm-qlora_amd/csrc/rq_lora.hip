// LoRA operand preparation for the prefill GEMM and the dX kernel (many
// activation rows).  lora_layer.py:67-70 rounds every intermediate to the
// activation dtype:
//   forward  u = RND(xl . RND(A)^T)                   [M, r]
//   backward g = RND(RND(dY * s) . RND(B))            [M, r] (lora_layer.py:67
//            differentiated: dX += RND(g . RND(A)))
// The kernels here produce u / g as [rows, r16] 16-bit operands (r16 = r
// rounded up to 16, zero padded) that the GEMM epilogues stage into LDS:
//   lora_rows_kernel     fp32 partial sums of a split-K MFMA product
//                        X[rows, K] . RND(S)[r, K]^T; S with contiguous rows
//                        (A) is rounded as it is staged, S with strided rows
//                        (B^T) is first gathered into a contiguous 16-bit
//                        [r, K] scratch;
//   lora_finish_kernel   sum of the partials, rounded;
//   lora_round_kernel    RND of a strided matrix into a contiguous 16-bit
//                        copy (B^T for the dX's lora_rows, whose rows are
//                        strided in B).
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"
#include "rq_lora.h"

namespace rq {

constexpr int kLoraRowsM = 64;    // activation rows per workgroup (4 waves x 16)
constexpr int kLoraRowsR = 64;    // LoRA ranks per workgroup
constexpr int kLoraChunkK = 256;  // k per LDS stage of S
constexpr int kLoraSPitch = kLoraChunkK + 8;

// X[m, k] (16-bit, row stride ldx) times S16[j, k] (16-bit, already rounded
// to XT, rows j < R of a [R][K] array) over k in this split's range;
// PRESCALE multiplies each x element by `prescale` and rounds it to XT
// first.  Output: part[ks][m][j] fp32 for m < M, j < R.
template <int XT, bool PRESCALE>
__global__ __launch_bounds__(256) void lora_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M,
                                                        int64_t K, const uint16_t* __restrict__ s16, int R,
                                                        const void* __restrict__ sraw, int sdt, int64_t ldsr,
                                                        bool svec, float prescale, int64_t k_per_split,
                                                        float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint16_t ss[kLoraRowsR * kLoraSPitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, q4 = lane >> 4;
  const int64_t m0 = int64_t(blockIdx.x) * kLoraRowsM;
  const int j0 = blockIdx.y * kLoraRowsR;
  const int ks = blockIdx.z;
  const int64_t k0 = int64_t(ks) * k_per_split;
  const int64_t k1 = k0 + k_per_split < K ? k0 + k_per_split : K;
  int64_t m = m0 + 16 * wave + i16;
  m = m < M ? m : M - 1;
  const uint16_t* xr = x + m * ldx;
  f32x4 acc[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) acc[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t kc = k0; kc < k1; kc += kLoraChunkK) {
    const int len = int(k1 - kc < kLoraChunkK ? k1 - kc : kLoraChunkK);  // multiple of 64
    const int c16 = len / 8;                                             // 16-byte chunks per row
    // this lane's activation fragments of the whole chunk, issued before the
    // staging so that their latency overlaps it (steps past len re-read the
    // chunk's first step: in bounds, unused)
    u32x4 xf[kLoraChunkK / 32];
#pragma unroll
    for (int t = 0; t < kLoraChunkK / 32; ++t)
      xf[t] = *reinterpret_cast<const u32x4*>(xr + kc + (32 * t < len ? 32 * t : 0) + 8 * q4);
    __syncthreads();
    // 64 rows x len: thread tid takes chunk (tid % 32) of rows tid / 32 + 8 i
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int jj = tid / 32 + 8 * i, c = tid % 32;
      const int j = j0 + jj;
      if (c < c16) {
        // RND(S) from the rounded copy, or from S itself (rows of stride ldsr)
        const u32x4 v = j >= R ? u32x4{0u, 0u, 0u, 0u}
                        : sraw ? load_a8<XT>(sraw, sdt, int64_t(j) * ldsr + kc + 8 * c, true, svec)
                               : *reinterpret_cast<const u32x4*>(s16 + int64_t(j) * K + kc + 8 * c);
        *reinterpret_cast<u32x4*>(ss + jj * kLoraSPitch + 8 * c) = v;
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
      for (int jb = 0; jb < 4; ++jb) {
        const u32x4 b = *reinterpret_cast<const u32x4*>(ss + (16 * jb + i16) * kLoraSPitch + 32 * t + 8 * q4);
        acc[jb] = mfma16x16x32<XT>(xa, b, acc[jb]);
      }
    }
  }
  // D[r][c] of block jb: row 4 q4 + r of the wave's 16, rank 16 jb + i16
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    const int j = j0 + 16 * jb + i16;
    if (j >= R) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t mo = m0 + 16 * wave + 4 * q4 + r;
      if (mo < M) part[(int64_t(ks) * M + mo) * R + j] = acc[jb][r];
    }
  }
}

// out[m][j] = RND(sum over splits of part[k][m][j]) for j < R, 0 for
// R <= j < R16; each thread produces 8 consecutive outputs (one 16-byte
// store).
template <int XT>
__global__ __launch_bounds__(256) void lora_finish_kernel(const float* __restrict__ part, int KS, int64_t M, int R,
                                                          int R16, uint16_t* __restrict__ out) {
  const int64_t i8 = int64_t(blockIdx.x) * 256 + threadIdx.x;  // index of 8 outputs
  const int per_row = R16 / 8;
  if (i8 >= M * per_row) return;
  const int64_t m = i8 / per_row;
  const int j0 = int(i8 - m * per_row) * 8;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = 0.0f;
  if (R % 8 == 0) {
    // two 16-byte loads per split, four splits in flight
    int k = 0;
    for (; k + 4 <= KS; k += 4) {
      f32x4 a[4], b[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f32x4* src = reinterpret_cast<const f32x4*>(part + (int64_t(k + t) * M + m) * R + j0);
        a[t] = src[0];
        b[t] = src[1];
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v[0] = __fadd_rn(v[0], a[t].x); v[1] = __fadd_rn(v[1], a[t].y);
        v[2] = __fadd_rn(v[2], a[t].z); v[3] = __fadd_rn(v[3], a[t].w);
        v[4] = __fadd_rn(v[4], b[t].x); v[5] = __fadd_rn(v[5], b[t].y);
        v[6] = __fadd_rn(v[6], b[t].z); v[7] = __fadd_rn(v[7], b[t].w);
      }
    }
    for (; k < KS; ++k) {
      const f32x4* src = reinterpret_cast<const f32x4*>(part + (int64_t(k) * M + m) * R + j0);
      const f32x4 a = src[0], b = src[1];
      v[0] = __fadd_rn(v[0], a.x); v[1] = __fadd_rn(v[1], a.y);
      v[2] = __fadd_rn(v[2], a.z); v[3] = __fadd_rn(v[3], a.w);
      v[4] = __fadd_rn(v[4], b.x); v[5] = __fadd_rn(v[5], b.y);
      v[6] = __fadd_rn(v[6], b.z); v[7] = __fadd_rn(v[7], b.w);
    }
  } else {
    for (int k = 0; k < KS; ++k) {
      const float* src = part + (int64_t(k) * M + m) * R;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (j0 + e < R) v[e] = __fadd_rn(v[e], src[j0 + e]);
    }
  }
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) w[h] = cvt_pk<XT>(v[2 * h], v[2 * h + 1]);
  *reinterpret_cast<u32x4*>(out + m * R16 + j0) = u32x4{w[0], w[1], w[2], w[3]};
}

// out[n][j] = RND(src[n * s_n + j * s_j]) for j < R, 0 for R <= j < R16;
// each thread produces 8 consecutive outputs (one 16-byte store).
template <int XT, int DT>
__global__ __launch_bounds__(256) void lora_round_kernel(const void* __restrict__ src, int64_t s_n, int64_t s_j,
                                                         int64_t rows, int R, int R16, uint16_t* __restrict__ out) {
  const int64_t i8 = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int per_row = R16 / 8;
  if (i8 >= rows * per_row) return;
  const int64_t n = i8 / per_row;
  const int j0 = int(i8 - n * per_row) * 8;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = j0 + e < R ? ld_f32<DT>(src, n * s_n + int64_t(j0 + e) * s_j) : 0.0f;
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) w[h] = cvt_pk<XT>(v[2 * h], v[2 * h + 1]);
  *reinterpret_cast<u32x4*>(out + n * R16 + j0) = u32x4{w[0], w[1], w[2], w[3]};
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
LoraRowsPlan plan_lora_rows(int64_t M, int64_t K, int64_t R, int cus) {
  LoraRowsPlan p{};
  const int64_t tiles = ((M + kLoraRowsM - 1) / kLoraRowsM) * ((R + kLoraRowsR - 1) / kLoraRowsR);
  const int64_t steps = K / 64;
  // enough splits to fill the compute units, and at most 8 steps (two LDS
  // chunks) per split: a workgroup's chunks run one after another
  int64_t ks = (cus + tiles - 1) / tiles;
  const int64_t ks_len = (steps + 7) / 8;
  ks = ks < ks_len ? ks_len : ks;
  ks = ks < 1 ? 1 : (ks > steps ? steps : ks);
  const int64_t steps_per = (steps + ks - 1) / ks;
  p.k_per_split = steps_per * 64;
  p.splits = int((K + p.k_per_split - 1) / p.k_per_split);
  p.part_bytes = (size_t(p.splits) * M * R * 4 + 255) & ~size_t(255);
  p.s16_bytes = (size_t(R) * K * 2 + 255) & ~size_t(255);
  return p;
}

template <int XT, bool PRESCALE>
static int launch_rows_t(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const uint16_t* s16, int R,
                         const void* sraw, int sdt, int64_t ldsr, bool svec, float prescale, const LoraRowsPlan& p,
                         float* part, hipStream_t stream) {
  dim3 grid(unsigned((M + kLoraRowsM - 1) / kLoraRowsM), unsigned((R + kLoraRowsR - 1) / kLoraRowsR),
            unsigned(p.splits));
  lora_rows_kernel<XT, PRESCALE><<<grid, 256, 0, stream>>>(x, ldx, M, K, s16, R, sraw, sdt, ldsr, svec, prescale,
                                                           p.k_per_split, part);
  return rq_check_launch();
}

int run_lora_rows(int xt, const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const void* s, int s_dt,
                  int64_t s_j, int64_t s_k, int R, bool prescale, float scale, const LoraRowsPlan& p, float* part,
                  uint16_t* s16, uint16_t* out, int R16, hipStream_t stream) {
  if (!aligned(x, 16) || ldx % 8 != 0 || K % 64 != 0) return RQ_ERR_BAD_ALIGNMENT;
  // S with contiguous rows is rounded as it is staged; otherwise RND(S) is
  // first gathered into a contiguous [R][K] 16-bit copy: S[j][k] = s[j * s_j + k * s_k]
  int st = RQ_OK;
  const bool direct = s_k == 1;
  const bool svec = direct && aligned(s, 16) && (s_dt != RQ_DTYPE_F32 || s_j % 4 == 0);
  if (!direct && (st = run_lora_round(xt, s, s_dt, s_j, s_k, R, int(K), int(K), s16, stream)) != RQ_OK) return st;
  const void* sraw = direct ? s : nullptr;
  if (xt == RQ_DTYPE_BF16)
    st = prescale ? launch_rows_t<RQ_DTYPE_BF16, true>(x, ldx, M, K, s16, R, sraw, s_dt, s_j, svec, scale, p, part,
                                                       stream)
                  : launch_rows_t<RQ_DTYPE_BF16, false>(x, ldx, M, K, s16, R, sraw, s_dt, s_j, svec, scale, p, part,
                                                        stream);
  else
    st = prescale ? launch_rows_t<RQ_DTYPE_F16, true>(x, ldx, M, K, s16, R, sraw, s_dt, s_j, svec, scale, p, part,
                                                      stream)
                  : launch_rows_t<RQ_DTYPE_F16, false>(x, ldx, M, K, s16, R, sraw, s_dt, s_j, svec, scale, p, part,
                                                       stream);
  if (st != RQ_OK) return st;
  const unsigned blocks = unsigned((M * (R16 / 8) + 255) / 256);
  if (xt == RQ_DTYPE_BF16)
    lora_finish_kernel<RQ_DTYPE_BF16><<<blocks, 256, 0, stream>>>(part, p.splits, M, R, R16, out);
  else
    lora_finish_kernel<RQ_DTYPE_F16><<<blocks, 256, 0, stream>>>(part, p.splits, M, R, R16, out);
  return rq_check_launch();
}

template <int XT>
static int launch_round_t(const void* src, int dt, int64_t s_n, int64_t s_j, int64_t rows, int R, int R16,
                          uint16_t* out, hipStream_t stream) {
  const unsigned blocks = unsigned((rows * (R16 / 8) + 255) / 256);
  switch (dt) {
    case RQ_DTYPE_F32:
      lora_round_kernel<XT, RQ_DTYPE_F32><<<blocks, 256, 0, stream>>>(src, s_n, s_j, rows, R, R16, out);
      break;
    case RQ_DTYPE_BF16:
      lora_round_kernel<XT, RQ_DTYPE_BF16><<<blocks, 256, 0, stream>>>(src, s_n, s_j, rows, R, R16, out);
      break;
    default:
      lora_round_kernel<XT, RQ_DTYPE_F16><<<blocks, 256, 0, stream>>>(src, s_n, s_j, rows, R, R16, out);
  }
  return rq_check_launch();
}

int run_lora_round(int xt, const void* src, int dt, int64_t s_n, int64_t s_j, int64_t rows, int R, int R16,
                   uint16_t* out, hipStream_t stream) {
  if (R16 % 8 != 0 || !aligned(out, 16)) return RQ_ERR_BAD_ALIGNMENT;
  if (xt == RQ_DTYPE_BF16) return launch_round_t<RQ_DTYPE_BF16>(src, dt, s_n, s_j, rows, R, R16, out, stream);
  return launch_round_t<RQ_DTYPE_F16>(src, dt, s_n, s_j, rows, R, R16, out, stream);
}

}  // namespace rq
