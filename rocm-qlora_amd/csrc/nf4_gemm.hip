// NF4 prefill / training GEMM (M > 16 rows of activations) for gfx950:
//   y[M, N] = RND(RND(x W^T + RND(bias)) + RND(RND(RND(u) RND(B)^T) * scaling))
// with W = RND(T[code] * scale) dequantized exactly as the reference does
// (quant_ops.py:144-148 then .to(x.dtype), quant_linear.py:191-193) and the
// LoRA term of lora_layer.py:67-70 fused into the epilogue (u = xl A^T comes
// from lora_u_kernel, summed and rounded by lora_u_round_kernel).
//
// Workgroup tile BM x BN, BM = 4 waves x 32 MB rows.  Each wave owns 32 MB
// token rows and all BN feature columns as 32x32 blocks of
// v_mfma_f32_32x32x16_{bf16,f16}.  K advances 64 at a time -- one NF4 block
// per weight row, so one scale per row per step:
//   * activations stream from global memory (L2) straight into registers in
//     the MFMA operand layout; every activation row is loaded by exactly one
//     wave, so there is no redundant activation traffic and none of it passes
//     through LDS;
//   * the BN x 64 weight slice is loaded packed (two steps ahead),
//     dequantized once per workgroup through the LDS pair table, rounded to
//     the activation dtype and written to a padded LDS tile (double
//     buffered), from which every wave reads its weight operands.
// Tiles are numbered so that the workgroups of one XCD (workgroup id mod 8)
// share activation row slices, which then stay in that XCD's L2.
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"

namespace rq {

constexpr int kGemmThreads = 256;
constexpr int kGemmBK = 64;
constexpr int kWPitch = kGemmBK + 8;  // operand elements per LDS weight row: the pad spreads rows over banks
constexpr int kLutBytes = kF32PairLutQwords * 8;
constexpr int kWDepth = 4;  // packed-weight prefetch distance in k-steps

template <int BN>
constexpr int gemm_lds_bytes() {
  return kLutBytes + 2 * BN * kWPitch * 2;
}

struct GemmArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* packed;
  int64_t M, N, K;
  int64_t blocks_per_row;  // K / block_size
  int bs_log2;             // log2(block_size)
  int tiles_m, tiles_n;
  bool xcd_map;            // tiles of one row slice on one XCD
};

struct GemmEpi {
  const void* bias;
  int bias_dt;
  int rank, rank16;      // LoRA rank and rank rounded up to 16
  const uint16_t* u;     // RND(u) [M][rank16], zero padded
  const void* lora_b;
  int64_t ld_lora_b;
  int lora_dt;
  float scaling;
  uint16_t* y;
  int64_t ldy;
};

// 16 bytes at element offset `off` of a 16-bit array (unsigned 32-bit offset
// from a wave-uniform base: the SGPR-base + VGPR-offset load form).
__device__ __forceinline__ u32x4 ld16(const uint16_t* base, uint32_t off) {
  const uint32_t byte_off = off * 2u;
  return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + byte_off);
}

// One k-step's packed weights for this thread: BN rows x 32 bytes over 256
// threads -- 16 bytes of one row (BN = 128) or a whole 32-byte row (BN = 256).
template <int BN, class Scale>
struct GemmWLoads {
  static constexpr int kChunks = BN / 128;  // 16-byte chunks per thread
  u32x4 w[kChunks];
  typename Scale::Raw s;
};

template <int BN>
__device__ __forceinline__ int w_row(int tid) { return BN == 128 ? (tid >> 1) : tid; }
template <int BN>
__device__ __forceinline__ int w_chunk(int tid) { return BN == 128 ? (tid & 1) : 0; }

template <int BN, class Scale>
__device__ __forceinline__ void gemm_issue_w(GemmWLoads<BN, Scale>& L, const GemmArgs& a, const Scale& scale,
                                             uint32_t wrow, int64_t n, int64_t kt) {
  constexpr int C = GemmWLoads<BN, Scale>::kChunks;
  const uint32_t off = wrow + uint32_t(kt) * 32u;  // byte offset; the host keeps the weights under 4 GiB
#pragma unroll
  for (int c = 0; c < C; ++c) L.w[c] = *reinterpret_cast<const u32x4*>(a.packed + (off + 16u * c));
  L.s = scale.load(n * a.blocks_per_row + ((kt * kGemmBK) >> a.bs_log2));
}

// Dequantize one k-step into an LDS weight tile (row-major, kWPitch).
template <int XT, int BN, class Scale>
__device__ __forceinline__ void gemm_dequant_w(const GemmWLoads<BN, Scale>& L, const Scale& scale, uint16_t* wt,
                                               const u32x2* lut, uint32_t lane_off, int tid) {
  constexpr int C = GemmWLoads<BN, Scale>::kChunks;
  const float s = scale.value(L.s);
  uint16_t* dst = wt + w_row<BN>(tid) * kWPitch + 32 * w_chunk<BN>(tid);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const u32x4 v = L.w[c];
    *reinterpret_cast<u32x4*>(dst + 32 * c) = expand8_scaled<XT>(lut, v.x, lane_off, s);
    *reinterpret_cast<u32x4*>(dst + 32 * c + 8) = expand8_scaled<XT>(lut, v.y, lane_off, s);
    *reinterpret_cast<u32x4*>(dst + 32 * c + 16) = expand8_scaled<XT>(lut, v.z, lane_off, s);
    *reinterpret_cast<u32x4*>(dst + 32 * c + 24) = expand8_scaled<XT>(lut, v.w, lane_off, s);
  }
}

// Activation operands: lane (i, q) of a wave feeds row i of each 32-row
// block; within a 64-k step, sub-step s of the MFMA chain takes k = 16 s +
// 8 q + e (e = 0..7), so the two lanes of a row load 32 contiguous bytes per
// instruction (one half of a 64-byte sector, not two quarters of two), and
// the four sub-steps cover the row's 128 bytes.  The weight operands read
// from LDS use the same k order (any consistent permutation of k leaves the
// dot product unchanged).
//
// One 64-k step for a wave's (32 MB) x BN tile, software-pipelined by hand
// so that the matrix cores never wait on the other work of the wave: an
// MFMA occupies the core for 32 cycles, in which the wave can issue a few
// VALU, LDS and vector-memory instructions, so that work is spread between
// the MFMAs rather than batched after them (in-order issue would otherwise
// leave the core idle while the batch drains).  Sub-step s (k = 16 s + 8 q +
// e, eight MFMAs in four pairs):
//   head:   the weight-operand reads of sub-step s + 1;
//   pair 0: one activation load (step j + 3, into xf, the register set step
//           j - 1 used; element offset knext), or the packed weights of step
//           j + 4 into wl_fill once the activations are all issued;
//   pair 1: table addresses and lookups for dword s + 1 of this thread's
//           packed weights of the next tile;
//   pair 2, 3: scale-multiply and round dword s's lookups (issued a
//           sub-step earlier), then store the 8 dequantized weights to LDS.
// Scheduling fences pin each group, so every wait on the memory counter
// covers only loads issued at least a step earlier and every wait on the
// LDS counter covers reads issued a pair group or more earlier.
template <int XT, int MB, int NB, int BN, bool DEQ, class Scale>
__device__ __forceinline__ void gemm_step(f32x16 (&acc)[MB][NB], const u32x4 (&xa)[MB][4], u32x4 (&xf)[MB][4],
                                          const uint16_t* wt, int i32, int q, const uint32_t (&xo)[MB],
                                          int64_t knext, const GemmWLoads<BN, Scale>& wq, GemmWLoads<BN, Scale>& wl_fill,
                                          const GemmArgs& a, const Scale& scale, uint32_t wrow, int64_t wn,
                                          int64_t kfill, uint16_t* wdst, const u32x2* lut, uint32_t lane_off) {
  constexpr int C = GemmWLoads<BN, Scale>::kChunks;
  static_assert(NB == 4, "four MFMA pairs per sub-step");
  static_assert(MB * 4 < 16, "activation loads fit in the pair-0 slots");
  float sc = 0.0f;
  if constexpr (DEQ) sc = scale.value(wq.s);
  auto word_of = [&](int c, int s) -> uint32_t {
    return s == 0 ? wq.w[c].x : s == 1 ? wq.w[c].y : s == 2 ? wq.w[c].z : wq.w[c].w;
  };
  auto lookup = [&](u32x2 (&lk)[C][4], int s) {
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t addr = __builtin_amdgcn_perm(word_of(c, s), lane_off, 0x0C0C0000u | (uint32_t(4 + h) << 8));
        lk[c][h] = *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(lut) + addr);
      }
  };
  u32x4 b[NB], bn[NB];
  u32x2 lk[C][4], lkn[C][4];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
    b[nb] = *reinterpret_cast<const u32x4*>(wt + (32 * nb + i32) * kWPitch + 8 * q);
  if constexpr (DEQ) lookup(lk, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s < 3) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bn[nb] = *reinterpret_cast<const u32x4*>(wt + (32 * nb + i32) * kWPitch + 8 * q + 16 * (s + 1));
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t r[C][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma32x32x16<XT>(xa[mb][s], b[nb], acc[mb][nb]);
      if (nb == 0) {
        // activation loads: 4 MB pieces over the 4 sub-steps' pair-0 slots,
        // MB per slot, a row block's pieces in line order
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          xf[mb][s] = ld16(a.x, xo[mb] + uint32_t(knext) + 16u * s);
        if (s == 3) gemm_issue_w<BN>(wl_fill, a, scale, wrow, wn, kfill);
      } else if (nb == 1) {
        if constexpr (DEQ) {
          if (s < 3) lookup(lkn, s + 1);
        }
      } else if constexpr (DEQ) {
        const int h0 = nb == 2 ? 0 : 2;
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int h = h0; h < h0 + 2; ++h)
            r[c][h] = cvt_pk<XT>(__fmul_rn(u2f(lk[c][h].x), sc), __fmul_rn(u2f(lk[c][h].y), sc));
        if (nb == 3) {
#pragma unroll
          for (int c = 0; c < C; ++c)
            *reinterpret_cast<u32x4*>(wdst + 32 * c + 8 * s) = u32x4{r[c][0], r[c][1], r[c][2], r[c][3]};
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (s < 3) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) b[nb] = bn[nb];
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int h = 0; h < 4; ++h) lk[c][h] = lkn[c][h];
    }
  }
}

template <int XT, int BN, int MB, class Scale>
__global__ __launch_bounds__(kGemmThreads) void nf4_gemm_kernel(GemmArgs a, Scale scale, GemmEpi e) {
  constexpr int NB = BN / 32;  // 32-wide column blocks per wave
  constexpr int BM = 4 * 32 * MB;
  // One static LDS block: the pair table at address 0 (lookups fold their
  // base into the instruction offset), then two weight tiles.  The epilogue
  // reuses all of it for RND(lora_B) rows.
  __shared__ __attribute__((aligned(16))) uint8_t lds[gemm_lds_bytes<BN>()];
  u32x2* lut = reinterpret_cast<u32x2*>(lds);
  uint16_t* wt0 = reinterpret_cast<uint16_t*>(lds + kLutBytes);
  uint16_t* wt1 = wt0 + BN * kWPitch;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i32 = lane & 31, q = lane >> 5;

  // tile of this workgroup
  const int64_t T = int64_t(a.tiles_m) * a.tiles_n;
  const int64_t g = blockIdx.x;
  const int64_t t = a.xcd_map ? (g % 8) * (T / 8) + g / 8 : g;
  const int64_t mt = t / a.tiles_n, nt = t % a.tiles_n;
  const int64_t m0 = mt * BM, n0 = nt * BN;
  const int64_t m0w = m0 + 32 * MB * wave;
  const int64_t nk = a.K / kGemmBK;

  // Per-lane element offsets from the activation base (32-bit: the host
  // keeps the activations under 4 GiB), so the loads use the SGPR-base form.
  uint32_t xo[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    int64_t m = m0w + 32 * mb + i32;
    m = m < a.M ? m : a.M - 1;  // rows past M re-read a live row; never stored
    xo[mb] = uint32_t(m * a.ldx + 8 * q);
  }
  int64_t wn = n0 + w_row<BN>(tid);
  wn = wn < a.N ? wn : a.N - 1;  // rows past N re-read a live row; never stored
  const uint32_t wrow = uint32_t(wn * (a.K >> 1) + 16 * w_chunk<BN>(tid));  // byte offset of this thread's row segment

  // Staggered start: workgroups that share an activation row slice begin
  // their k loop at different steps (wrapping around K), so all but the
  // first to reach a step find its activations already in L2 instead of
  // all of them waiting on the same HBM fetch.  Step j covers k-step
  // ks(j) = (j + k_off) mod nk; the fp32 sum order changes, nothing else.
  const int nk32 = __builtin_amdgcn_readfirstlane(int(nk));
  const int k_off = __builtin_amdgcn_readfirstlane(int(((nt & 31) * nk) >> 5));
  auto ks = [&](int64_t j) -> int64_t {
    int v = int(j) + k_off;
    v = v >= nk32 ? v - nk32 : v;
    v = v >= nk32 ? v - nk32 : v;
    return v;
  };

  // Register pipelines: packed weights kWDepth steps ahead (wl[j % 4] holds
  // step j + 4 once step j has issued it), activations three steps ahead
  // (xa[j % 4] holds step j; step j fills xa[(j + 3) % 4]).
  GemmWLoads<BN, Scale> wl[kWDepth];
#pragma unroll
  for (int d = 0; d < kWDepth; ++d) gemm_issue_w<BN>(wl[d], a, scale, wrow, wn, ks(d));
  u32x4 xa[4][MB][4];
#pragma unroll
  for (int h = 0; h < 3; ++h)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int s = 0; s < 4; ++s) xa[h][mb][s] = ld16(a.x, xo[mb] + uint32_t(ks(h) * kGemmBK) + 16u * s);

  fill_f32pair_lut<kGemmThreads * 2>(lut, tid);  // the 512-thread fill pattern, in two halves
  fill_f32pair_lut<kGemmThreads * 2>(lut, tid + kGemmThreads);
  __syncthreads();
  const uint32_t lane_off = uint32_t(lane & 31) * 8u;
  gemm_dequant_w<XT, BN>(wl[0], scale, wt0, lut, lane_off, tid);
  __syncthreads();

  f32x16 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

  // Step j: MFMAs on tile j % 2 and xa[j % 4]; loads of activations j + 3
  // into xa[(j + 3) % 4] and packed weights j + 4 into wl[j % 4]; dequantize
  // step j + 1 from wl[(j + 1) % 4] into tile (j + 1) % 2; barrier.  Four
  // steps per iteration index every register set and tile statically; the
  // loop has a single exit, so the accumulators stay in place.  Steps past
  // the end wrap around K (in bounds; their results are never used).
  uint16_t* wd[2];
  wd[0] = wt0 + w_row<BN>(tid) * kWPitch + 32 * w_chunk<BN>(tid);  // this thread's row segment
  wd[1] = wd[0] + BN * kWPitch;
  const uint16_t* wts[2] = {wt0, wt1};
#define RQ_GEMM_STEP(J, P)                                                                                \
  do {                                                                                                    \
    gemm_step<XT, MB, NB, BN, true>(acc, xa[P], xa[((P) + 3) & 3], wts[(P) & 1], i32, q, xo,               \
                                    ks((J) + 3) * kGemmBK, wl[((P) + 1) & 3], wl[P], a, scale, wrow, wn,   \
                                    ks((J) + kWDepth), wd[((P) + 1) & 1], lut, lane_off);                  \
    __syncthreads();                                                                                      \
  } while (0)
  int64_t j = 0;
  for (; j + 4 <= nk; j += 4) {
    RQ_GEMM_STEP(j, 0);
    RQ_GEMM_STEP(j + 1, 1);
    RQ_GEMM_STEP(j + 2, 2);
    RQ_GEMM_STEP(j + 3, 3);
  }
  const int64_t rem = nk - j;
  if (rem > 0) RQ_GEMM_STEP(j, 0);
  if (rem > 1) RQ_GEMM_STEP(j + 1, 1);
  if (rem > 2) RQ_GEMM_STEP(j + 2, 2);
#undef RQ_GEMM_STEP

  // ---- epilogue.  base = RND(acc + RND(bias)); the LoRA product
  // RND(u) RND(B)^T accumulates per 32-column block by MFMA (u operands from
  // the rounded u rows in global memory, RND(B) rows staged in LDS); then
  // y = RND(base + RND(RND(lora) * scaling)).
  const int rank = e.rank;
  const int r16 = e.rank16;
  const int bpitch = r16 + 8;
  uint16_t* bs = reinterpret_cast<uint16_t*>(lds);  // [BN][bpitch]
  if (rank > 0) {
    __syncthreads();  // every wave is done with the weight tiles and the table
    for (int idx = tid; idx < BN * r16; idx += kGemmThreads) {
      const int r = idx / r16, j = idx - r * r16;
      const int64_t n = n0 + r;
      const float v = (j < rank && n < a.N) ? load_as_f32(e.lora_b, n * e.ld_lora_b + j, e.lora_dt) : 0.0f;
      bs[r * bpitch + j] = uint16_t(to_x16<XT>(v));
    }
    __syncthreads();
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = n0 + 32 * nb + i32;
    const float bias = (e.bias && n < a.N) ? round_x<XT>(load_as_f32(e.bias, n, e.bias_dt)) : 0.0f;
    f32x16 lo[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) lo[mb][r] = 0.0f;
    for (int s = 0; s < r16 / 16; ++s) {
      const u32x4 ub = *reinterpret_cast<const u32x4*>(bs + (32 * nb + i32) * bpitch + 16 * s + 8 * q);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        int64_t m = m0w + 32 * mb + i32;
        m = m < a.M ? m : a.M - 1;
        const u32x4 ua = *reinterpret_cast<const u32x4*>(e.u + m * r16 + 16 * s + 8 * q);
        lo[mb] = mfma32x32x16<XT>(ua, ub, lo[mb]);
      }
    }
    if (n >= a.N) continue;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0w + 32 * mb + 8 * (r >> 2) + 4 * q + (r & 3);
        if (m >= a.M) continue;
        float v = acc[mb][nb][r];
        if (e.bias) v = __fadd_rn(v, bias);
        v = round_x<XT>(v);
        if (rank > 0) v = round_x<XT>(__fadd_rn(v, round_x<XT>(__fmul_rn(round_x<XT>(lo[mb][r]), e.scaling))));
        e.y[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
      }
    }
  }
}

// RND(u) for the epilogue: the sum of the KS fp32 partial products that
// lora_u_kernel wrote ([KS][M][rank]), rounded to the activation dtype, as
// [M][rank16] with zero padding.
template <int XT>
__global__ __launch_bounds__(256) void lora_u_round_kernel(const float* __restrict__ up, int KS, int64_t M,
                                                           int rank, int rank16, uint16_t* __restrict__ u16) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= M * rank16) return;
  const int64_t m = i / rank16;
  const int j = int(i - m * rank16);
  float v = 0.0f;
  if (j < rank)
    for (int k = 0; k < KS; ++k) v = __fadd_rn(v, up[(int64_t(k) * M + m) * rank + j]);
  u16[i] = uint16_t(to_x16<XT>(v));
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct GemmPlan {
  int BN, MB;
  int tiles_m, tiles_n;
  bool xcd_map;
  int u_splits, rank16;
  size_t ws_bytes, u16_offset;
};

static GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t rank) {
  GemmPlan p{};
  p.MB = 2;
  p.BN = 128;
  p.tiles_m = int((M + 4 * 32 * p.MB - 1) / (4 * 32 * p.MB));
  p.tiles_n = int((N + p.BN - 1) / p.BN);
  const int64_t T = int64_t(p.tiles_m) * p.tiles_n;
  p.xcd_map = T % 8 == 0;
  p.rank16 = int((rank + 15) & ~int64_t(15));
  p.u_splits = 0;
  p.ws_bytes = 0;
  if (rank > 0) {
    const int64_t steps_per_wg = 16;  // 32-k steps per lora_u workgroup
    p.u_splits = int((K / 32 + steps_per_wg - 1) / steps_per_wg);
    p.u16_offset = (size_t(p.u_splits) * M * rank * 4 + 255) & ~size_t(255);
    p.ws_bytes = p.u16_offset + size_t(M) * p.rank16 * 2;
  }
  return p;
}

int gemm_workspace(const LinearArgs& L, size_t* bytes) {
  *bytes = plan_gemm(L.M, L.N, L.K, L.rank).ws_bytes;
  return RQ_OK;
}

template <int XT, int BN, int MB, class Scale>
static int launch_gemm_t(const LinearArgs& L, const GemmPlan& p, Scale scale, const GemmEpi& e,
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
  const unsigned grid = unsigned(int64_t(p.tiles_m) * p.tiles_n);
  nf4_gemm_kernel<XT, BN, MB, Scale><<<grid, kGemmThreads, 0, stream>>>(a, scale, e);
  return rq_check_launch();
}

template <int XT, class Scale>
static int launch_gemm_cfg(const LinearArgs& L, const GemmPlan& p, Scale scale, const GemmEpi& e,
                           hipStream_t stream) {
  return launch_gemm_t<XT, 128, 2>(L, p, scale, e, stream);
}

template <int XT>
static int run_gemm(const LinearArgs& L, const GemmPlan& p, const GemmEpi& e, hipStream_t stream) {
  if (L.c2) {
    const int sh = pow2_shift(L.block2);
    switch (L.absmax_dtype) {
      case RQ_DTYPE_F32:
        return launch_gemm_cfg<XT>(L, p, ScaleDQ<RQ_DTYPE_F32>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, stream);
      case RQ_DTYPE_BF16:
        return launch_gemm_cfg<XT>(L, p, ScaleDQ<RQ_DTYPE_BF16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, stream);
      default:
        return launch_gemm_cfg<XT>(L, p, ScaleDQ<RQ_DTYPE_F16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, stream);
    }
  }
  switch (L.absmax_dtype) {
    case RQ_DTYPE_F32: return launch_gemm_cfg<XT>(L, p, ScaleAbsmax<RQ_DTYPE_F32>{L.absmax}, e, stream);
    case RQ_DTYPE_BF16: return launch_gemm_cfg<XT>(L, p, ScaleAbsmax<RQ_DTYPE_BF16>{L.absmax}, e, stream);
    default: return launch_gemm_cfg<XT>(L, p, ScaleAbsmax<RQ_DTYPE_F16>{L.absmax}, e, stream);
  }
}

template <int XT>
static int launch_u_round(const float* up, int ks, int64_t M, int rank, int rank16, uint16_t* u16,
                          hipStream_t stream) {
  const int64_t total = M * rank16;
  lora_u_round_kernel<XT><<<unsigned((total + 255) / 256), 256, 0, stream>>>(up, ks, M, rank, rank16, u16);
  return rq_check_launch();
}

int run_nf4_gemm(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  // the activation operands are loaded 16 bytes at a time
  if (!aligned(L.x, 16) || L.ldx % 8 != 0) return RQ_ERR_BAD_ALIGNMENT;
  // activation and packed-weight loads use 32-bit byte offsets
  if (double(L.M) * double(L.ldx) * 2.0 >= 4294967296.0 || double(L.N) * double(L.K) * 0.5 >= 4294967296.0)
    return RQ_ERR_UNSUPPORTED;
  const GemmPlan p = plan_gemm(L.M, L.N, L.K, L.rank);
  if (p.ws_bytes > 0 && (!workspace || ws_bytes < p.ws_bytes)) return RQ_ERR_WORKSPACE;
  if (workspace && !aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  GemmEpi e{};
  e.bias = L.bias;
  e.bias_dt = L.bias_dtype;
  e.rank = int(L.rank > 0 ? L.rank : 0);
  e.rank16 = p.rank16;
  e.lora_b = L.lora_b;
  e.ld_lora_b = L.ld_lora_b;
  e.lora_dt = L.lora_dtype;
  e.scaling = L.scaling;
  e.y = static_cast<uint16_t*>(L.y);
  e.ldy = L.ldy;
  int st;
  if (e.rank > 0) {
    float* up = static_cast<float*>(workspace);
    uint16_t* u16 = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + p.u16_offset);
    if ((st = run_lora_u(L, p.u_splits, up, stream)) != RQ_OK) return st;
    st = L.x_dtype == RQ_DTYPE_BF16 ? launch_u_round<RQ_DTYPE_BF16>(up, p.u_splits, L.M, e.rank, p.rank16, u16, stream)
                                    : launch_u_round<RQ_DTYPE_F16>(up, p.u_splits, L.M, e.rank, p.rank16, u16, stream);
    if (st != RQ_OK) return st;
    e.u = u16;
  }
  if (L.x_dtype == RQ_DTYPE_BF16) return run_gemm<RQ_DTYPE_BF16>(L, p, e, stream);
  return run_gemm<RQ_DTYPE_F16>(L, p, e, stream);
}

}  // namespace rq
