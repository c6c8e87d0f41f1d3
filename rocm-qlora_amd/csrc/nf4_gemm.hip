// NF4 prefill / training GEMM (M > 16 rows of activations) for gfx950:
//   y[M, N] = RND(RND(x W^T + RND(bias)) + RND(RND(RND(u) RND(B)^T) * scaling))
// with W = T[code] * scale dequantized exactly as the reference does
// (quant_ops.py:144-148 then .to(x.dtype), quant_linear.py:191-193) and the
// LoRA term of lora_layer.py:67-70 fused into the epilogue (u = RND(xl A^T)
// comes from lora_u_kernel).
//
// Workgroup tile 256 (tokens) x BN (features), 4 waves in a 2 x 2 grid, each
// owning 128 x BN/2 of the tile as 32x32 MFMA blocks (v_mfma_f32_32x32x16
// bf16/f16).  K advances 64 at a time -- one NF4 block per weight row, so one
// scale per row per step:
//   * activation operands go from global memory (L2) straight into
//     registers in the MFMA A layout, one k-step ahead;
//   * the BN x 64 weight slice is loaded packed (two k-steps ahead),
//     dequantized once per workgroup through the LDS pair table, rounded to
//     the activation dtype and written to a padded LDS tile (double
//     buffered), from which each wave reads its B operands.
// Tiles are numbered so that the workgroups of one XCD (workgroup id mod 8)
// share 256-row activation slices, which then stay in that XCD's L2.
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"

namespace rq {

constexpr int kGemmThreads = 256;
constexpr int kGemmBM = 256;
constexpr int kGemmBK = 64;
constexpr int kWPitch = kGemmBK + 8;  // operand elements per LDS weight row: the pad spreads rows over banks
constexpr int kGemmRankChunk = 64;  // LoRA ranks staged per epilogue pass
constexpr int kLoraPitch = kGemmRankChunk + 8;

struct GemmArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* packed;
  int64_t M, N, K;
  int64_t blocks_per_row;  // K / block_size
  int bs_log2;             // log2(block_size)
  int tiles_m, tiles_n;
  bool xcd_map;            // tiles of one 256-row slice on one XCD
  bool xvec;
};

// One k-step's packed weights for this thread: BN rows x 32 bytes over 256
// threads -- 16 bytes (BN = 128) or 32 bytes (BN = 256) of one row.
template <int BN, class Scale>
struct GemmWLoads {
  static constexpr int kChunks = BN / 128;  // 16-byte chunks per thread
  u32x4 w[kChunks];
  typename Scale::Raw s;
};

template <int BN, class Scale>
__device__ __forceinline__ void gemm_issue_w(GemmWLoads<BN, Scale>& L, const GemmArgs& a, const Scale& scale,
                                             int64_t n0, int64_t kt, int tid) {
  constexpr int C = GemmWLoads<BN, Scale>::kChunks;
  const int row = BN == 128 ? (tid >> 1) : tid;
  const int c0 = BN == 128 ? (tid & 1) : 0;
  int64_t n = n0 + row;
  n = n < a.N ? n : a.N - 1;  // rows past N re-read a live row; never stored
  const uint8_t* p = a.packed + n * (a.K >> 1) + kt * 32 + 16 * c0;
#pragma unroll
  for (int c = 0; c < C; ++c) L.w[c] = *reinterpret_cast<const u32x4*>(p + 16 * c);
  L.s = scale.load(n * a.blocks_per_row + ((kt * kGemmBK) >> a.bs_log2));
}

// Dequantize one k-step into the LDS weight tile (row-major, kWPitch).
template <int XT, int BN, class Scale>
__device__ __forceinline__ void gemm_dequant_w(const GemmWLoads<BN, Scale>& L, const Scale& scale, uint16_t* wt,
                                               const u32x2* lut, uint32_t lane_off, int tid) {
  constexpr int C = GemmWLoads<BN, Scale>::kChunks;
  const int row = BN == 128 ? (tid >> 1) : tid;
  const int c0 = BN == 128 ? (tid & 1) : 0;
  const float s = scale.value(L.s);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const u32x4 v = L.w[c];
    uint16_t* dst = wt + row * kWPitch + 32 * (c0 + c);
    *reinterpret_cast<u32x4*>(dst) = expand8_scaled<XT>(lut, v.x, lane_off, s);
    *reinterpret_cast<u32x4*>(dst + 8) = expand8_scaled<XT>(lut, v.y, lane_off, s);
    *reinterpret_cast<u32x4*>(dst + 16) = expand8_scaled<XT>(lut, v.z, lane_off, s);
    *reinterpret_cast<u32x4*>(dst + 24) = expand8_scaled<XT>(lut, v.w, lane_off, s);
  }
}

// Activation operands: lane (i, q) of a wave feeds row i of each 32-row
// block; within a 64-k step, sub-step s of the MFMA chain takes k = 32 q +
// 8 s + e (e = 0..7), so a lane's four sub-steps are 64 contiguous bytes of
// its row.  The weight operands read from LDS use the same k order (any
// consistent permutation of k leaves the dot product unchanged).
struct XRows {
  const uint16_t* p[4];  // row pointers at this lane's 32 q offset
};

__device__ __forceinline__ XRows gemm_x_rows(const GemmArgs& a, int64_t m0w, int i32, int q) {
  XRows r;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    int64_t m = m0w + 32 * mb + i32;
    m = m < a.M ? m : a.M - 1;  // rows past M re-read a live row; never stored
    r.p[mb] = a.x + m * a.ldx + 32 * q;
  }
  return r;
}

// One 64-k step of MFMAs for a wave's 128 x (32 NB) tile.  Each activation
// operand register set is refilled with the next step's values (k offset
// knext) as soon as its sub-step's MFMAs are issued, so the activations
// need one register set and still arrive a full step ahead.
template <int XT, int NB>
__device__ __forceinline__ void gemm_mfma_step(f32x16 (&acc)[4][NB], u32x4 (&xa)[4][4], const uint16_t* wt,
                                               int nrow0, int i32, int q, const XRows& xr, int64_t knext,
                                               bool xvec) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    u32x4 b[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      b[nb] = *reinterpret_cast<const u32x4*>(wt + (nrow0 + 32 * nb + i32) * kWPitch + 32 * q + 8 * s);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma32x32x16<XT>(xa[mb][s], b[nb], acc[mb][nb]);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) xa[mb][s] = load_x8(xr.p[mb] + knext * kGemmBK + 8 * s, xvec);
  }
}

template <int XT, int BN, class Scale>
__global__ __launch_bounds__(kGemmThreads) void nf4_gemm_kernel(GemmArgs a, Scale scale, LinearEpi e) {
  constexpr int NB = BN / 64;  // 32-wide column blocks per wave
  // The pair table is the only static LDS array (address 0, so lookups fold
  // their base into the instruction offset); in the epilogue its space holds
  // RND(u) rows.
  __shared__ u32x2 lut[kF32PairLutQwords];
  extern __shared__ uint32_t smem[];
  uint16_t* wtile = reinterpret_cast<uint16_t*>(smem);  // [2][BN][kWPitch]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int i32 = lane & 31, q = lane >> 5;

  // tile of this workgroup
  const int64_t T = int64_t(a.tiles_m) * a.tiles_n;
  const int64_t g = blockIdx.x;
  const int64_t t = a.xcd_map ? (g % 8) * (T / 8) + g / 8 : g;
  const int64_t mt = t / a.tiles_n, nt = t % a.tiles_n;
  const int64_t m0 = mt * kGemmBM, n0 = nt * BN;
  const int64_t m0w = m0 + 128 * wm;
  const int nrow0 = (BN / 2) * wn;
  const int64_t nk = a.K / kGemmBK;
  const XRows xr = gemm_x_rows(a, m0w, i32, q);

  GemmWLoads<BN, Scale> wl0, wl1;
  gemm_issue_w<BN>(wl0, a, scale, n0, 0, tid);
  gemm_issue_w<BN>(wl1, a, scale, n0, nk > 1 ? 1 : 0, tid);
  u32x4 xa[4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int s = 0; s < 4; ++s) xa[mb][s] = load_x8(xr.p[mb] + 8 * s, a.xvec);

  fill_f32pair_lut<kGemmThreads * 2>(lut, tid);  // the 512-thread fill pattern, in two halves
  fill_f32pair_lut<kGemmThreads * 2>(lut, tid + kGemmThreads);
  __syncthreads();
  const uint32_t lane_off = uint32_t(lane & 31) * 8u;
  gemm_dequant_w<XT, BN>(wl0, scale, wtile, lut, lane_off, tid);
  __syncthreads();

  f32x16 acc[4][NB];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

  // Two k-steps per iteration so the double buffers are indexed statically.
  // Loads past the last step re-read the last step (in bounds, unused).
  for (int64_t kt = 0; kt < nk; kt += 2) {
    {
      // step kt: weights in tile 0; packed step kt + 1 waits in wl1
      gemm_issue_w<BN>(wl0, a, scale, n0, kt + 2 < nk ? kt + 2 : nk - 1, tid);
      gemm_mfma_step<XT, NB>(acc, xa, wtile, nrow0, i32, q, xr, kt + 1 < nk ? kt + 1 : kt, a.xvec);
      if (kt + 1 < nk) gemm_dequant_w<XT, BN>(wl1, scale, wtile + BN * kWPitch, lut, lane_off, tid);
      __syncthreads();
    }
    if (kt + 1 >= nk) break;
    {
      // step kt + 1: weights in tile 1; packed step kt + 2 waits in wl0
      gemm_issue_w<BN>(wl1, a, scale, n0, kt + 3 < nk ? kt + 3 : nk - 1, tid);
      gemm_mfma_step<XT, NB>(acc, xa, wtile + BN * kWPitch, nrow0, i32, q, xr, kt + 2 < nk ? kt + 2 : kt + 1,
                             a.xvec);
      if (kt + 2 < nk) gemm_dequant_w<XT, BN>(wl0, scale, wtile, lut, lane_off, tid);
      __syncthreads();
    }
  }

  // ---- epilogue.  base = RND(acc + RND(bias)) in place; the LoRA product
  // RND(u) RND(B)^T accumulates by MFMA over rank chunks of 64 staged in LDS
  // (u rows in the table's space, B rows in the weight tiles' space); then
  // y = RND(base + RND(RND(lora) * scaling)).
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = n0 + nrow0 + 32 * nb + i32;
    const float bias = (e.bias && n < a.N) ? round_x<XT>(load_as_f32(e.bias, n, e.bias_dt)) : 0.0f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[mb][nb][r] = round_x<XT>(e.bias ? __fadd_rn(acc[mb][nb][r], bias) : acc[mb][nb][r]);
  }
  const int rank = e.rank > 0 ? e.rank : 0;
  f32x16 lo[4][NB];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) lo[mb][nb][r] = 0.0f;
  uint16_t* us = reinterpret_cast<uint16_t*>(lut);  // [256][kLoraPitch]
  uint16_t* bs = wtile;                             // [BN][kLoraPitch]
  for (int j0 = 0; j0 < rank; j0 += kGemmRankChunk) {
    const int w = rank - j0 < kGemmRankChunk ? ((rank - j0 + 15) & ~15) : kGemmRankChunk;
    if (j0 > 0) __syncthreads();  // previous chunk's operands fully read
    for (int idx = tid; idx < kGemmBM * w; idx += kGemmThreads) {
      const int r = idx / w, j = j0 + idx % w;
      const int64_t m = m0 + r;
      float v = 0.0f;
      if (j < rank && m < a.M) {
        for (int k = 0; k < e.u_splits; ++k) v = __fadd_rn(v, e.u[(int64_t(k) * a.M + m) * rank + j]);
      }
      us[r * kLoraPitch + (j - j0)] = uint16_t(to_x16<XT>(v));
    }
    for (int idx = tid; idx < BN * w; idx += kGemmThreads) {
      const int r = idx / w, j = j0 + idx % w;
      const int64_t n = n0 + r;
      const float v = (j < rank && n < a.N) ? load_as_f32(e.lora_b, n * e.ld_lora_b + j, e.lora_dt) : 0.0f;
      bs[r * kLoraPitch + (j - j0)] = uint16_t(to_x16<XT>(v));
    }
    __syncthreads();
    for (int s = 0; s < w / 16; ++s) {
      u32x4 ub[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        ub[nb] = *reinterpret_cast<const u32x4*>(bs + (nrow0 + 32 * nb + i32) * kLoraPitch + 16 * s + 8 * q);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const u32x4 ua = *reinterpret_cast<const u32x4*>(us + (128 * wm + 32 * mb + i32) * kLoraPitch + 16 * s + 8 * q);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) lo[mb][nb] = mfma32x32x16<XT>(ua, ub[nb], lo[mb][nb]);
      }
    }
  }

  uint16_t* y = static_cast<uint16_t*>(e.y);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = n0 + nrow0 + 32 * nb + i32;
    if (n >= a.N) continue;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0w + 32 * mb + 8 * (r >> 2) + 4 * q + (r & 3);
        if (m >= a.M) continue;
        float v = acc[mb][nb][r];
        if (rank > 0) v = round_x<XT>(__fadd_rn(v, round_x<XT>(__fmul_rn(round_x<XT>(lo[mb][nb][r]), e.scaling))));
        y[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct GemmPlan {
  int BN;
  int tiles_m, tiles_n;
  bool xcd_map;
  int u_splits;
  size_t lds_bytes, ws_bytes, u_offset;
};

static GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t rank, int cus) {
  GemmPlan p{};
  p.tiles_m = int((M + kGemmBM - 1) / kGemmBM);
  p.BN = 128;
  p.tiles_n = int((N + p.BN - 1) / p.BN);
  const int64_t T = int64_t(p.tiles_m) * p.tiles_n;
  p.xcd_map = T % 8 == 0;
  p.u_splits = rank > 0 ? 1 : 0;
  const size_t wtiles = size_t(2) * p.BN * kWPitch * 2;
  const size_t lora_b = size_t(p.BN) * kLoraPitch * 2;
  p.lds_bytes = wtiles > lora_b ? wtiles : lora_b;
  p.ws_bytes = 0;
  p.u_offset = 0;
  if (rank > 0) p.ws_bytes = size_t(p.u_splits) * M * rank * 4;
  return p;
}

int gemm_workspace(const LinearArgs& L, size_t* bytes) {
  const GemmPlan p = plan_gemm(L.M, L.N, L.K, L.rank, device_cus());
  *bytes = p.ws_bytes;
  return RQ_OK;
}

template <int XT, int BN, class Scale>
static int launch_gemm_t(const LinearArgs& L, const GemmPlan& p, Scale scale, const LinearEpi& e,
                         hipStream_t stream) {
  GemmArgs a;
  a.x = static_cast<const uint16_t*>(L.x);
  a.ldx = L.ldx;
  a.packed = L.w_packed;
  a.M = L.M;
  a.N = L.N;
  a.K = L.K;
  a.blocks_per_row = L.K / L.block_size;
  a.bs_log2 = pow2_shift(L.block_size);
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  a.xcd_map = p.xcd_map;
  a.xvec = aligned(L.x, 16) && (L.ldx % 8 == 0);
  auto kern = nf4_gemm_kernel<XT, BN, Scale>;
  static bool attr_set = false;  // one flag per instantiation
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024 - kF32PairLutQwords * 8) != hipSuccess)
      return RQ_ERR_HIP;
    attr_set = true;
  }
  const unsigned grid = unsigned(int64_t(p.tiles_m) * p.tiles_n);
  kern<<<grid, kGemmThreads, p.lds_bytes, stream>>>(a, scale, e);
  return rq_check_launch();
}

template <int XT, class Scale>
static int launch_gemm_bn(const LinearArgs& L, const GemmPlan& p, Scale scale, const LinearEpi& e,
                          hipStream_t stream) {
  return launch_gemm_t<XT, 128>(L, p, scale, e, stream);
}

template <int XT>
static int run_gemm(const LinearArgs& L, const GemmPlan& p, const LinearEpi& e, hipStream_t stream) {
  if (L.c2) {
    const int sh = pow2_shift(L.block2);
    switch (L.absmax_dtype) {
      case RQ_DTYPE_F32:
        return launch_gemm_bn<XT>(L, p, ScaleDQ<RQ_DTYPE_F32>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, stream);
      case RQ_DTYPE_BF16:
        return launch_gemm_bn<XT>(L, p, ScaleDQ<RQ_DTYPE_BF16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, stream);
      default:
        return launch_gemm_bn<XT>(L, p, ScaleDQ<RQ_DTYPE_F16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, stream);
    }
  }
  switch (L.absmax_dtype) {
    case RQ_DTYPE_F32: return launch_gemm_bn<XT>(L, p, ScaleAbsmax<RQ_DTYPE_F32>{L.absmax}, e, stream);
    case RQ_DTYPE_BF16: return launch_gemm_bn<XT>(L, p, ScaleAbsmax<RQ_DTYPE_BF16>{L.absmax}, e, stream);
    default: return launch_gemm_bn<XT>(L, p, ScaleAbsmax<RQ_DTYPE_F16>{L.absmax}, e, stream);
  }
}

int run_nf4_gemm(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  const GemmPlan p = plan_gemm(L.M, L.N, L.K, L.rank, device_cus());
  if (p.ws_bytes > 0 && (!workspace || ws_bytes < p.ws_bytes)) return RQ_ERR_WORKSPACE;
  if (workspace && !aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  float* up = L.rank > 0 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.u_offset) : nullptr;
  int st;
  if (L.rank > 0 && (st = run_lora_u(L, p.u_splits, up, stream)) != RQ_OK) return st;
  const LinearEpi e = make_epi(L, up, p.u_splits);
  if (L.x_dtype == RQ_DTYPE_BF16) return run_gemm<RQ_DTYPE_BF16>(L, p, e, stream);
  return run_gemm<RQ_DTYPE_F16>(L, p, e, stream);
}

}  // namespace rq
