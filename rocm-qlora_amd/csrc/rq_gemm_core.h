// The NF4/byte-weight MFMA GEMM core for gfx950, shared by the forward
// GEMM, the dX backward and the INT8/FP8 linears: activation rows streamed
// into a swizzled LDS ring by direct-to-LDS loads, a weight operand tile
// produced each step by a producer policy (see the producer interface
// below), 32x32x16 MFMAs, and the bias/LoRA/scale epilogue.  Layout and
// schedule are described at gemm_step and nf4_gemm_kernel.
#pragma once
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"
#include "rq_lora.h"

namespace rq {

constexpr int kGemmThreads = 256;
constexpr int kGemmBM = 256;
constexpr int kGemmBN = 128;
constexpr int kGemmBK = 64;
constexpr int kGemmMB = 2;  // 32-row blocks per wave
constexpr int kGemmNB = 4;  // 32-column blocks per wave
constexpr int kLutBytes = kF32PairLutQwords * 8;     // 64 KiB
constexpr int kXWaveBytes = 64 * 128;                // one wave's rows of one step
constexpr int kXStepBytes = 4 * kXWaveBytes;         // 32 KiB
constexpr int kWTileBytes = kGemmBN * 128;           // 16 KiB
constexpr int kXRingOff = kLutBytes;
constexpr int kWTileOff = kXRingOff + 2 * kXStepBytes;
constexpr int kGemmLds = kWTileOff + 2 * kWTileBytes;  // 160 KiB
constexpr int kWDepth = 4;                           // packed-weight prefetch distance in steps
constexpr int kGemmMaxSplits = 4;                    // K splits of the eight-wave core
static_assert(kGemmLds == 160 * 1024, "LDS plan");

// Core problem: out[M, N] = act[M, K] . op[N, K]^T (+ epilogue).
struct GemmArgs {
  const uint16_t* x;  // activations (x forward, dY for dX), row stride ldx
  int64_t ldx;
  int64_t M, N, K;    // rows, output columns, reduction length
  int tiles_m, tiles_n;
  bool xcd_map;       // tiles of one row slice on one XCD
  // K splits of the last wave's tiles (eight-wave core, xcd_map only).  Of
  // the T / 8 tiles of an XCD, the first lf run whole; the other lt =
  // T / 8 - lf run as `splits` workgroups each, over K ranges of equal
  // length.  Each split stores its fp32 tile to part and counts itself in
  // tile_cnt (zero before the launch); the last one of a tile sums the splits
  // in split order, runs the epilogue and sets the count back to 0.
  int splits;
  int lf;
  float* part;         // [splits][8 lt][64 x 512] fp32
  uint32_t* tile_cnt;  // [8 lt]
};

struct GemmEpi {
  const void* bias;
  int bias_dt;
  int rank, rank16;      // LoRA rank and rank rounded up to 16
  const uint16_t* u;     // RND(u) [M][rank16] (dX: RND(g)), zero padded
  const uint16_t* bl;    // RND(B) [N][rank16] (dX: RND(A^T)), zero padded
  // eight-wave core: the bl operand read as it is -- element (n, j) at
  // braw[n * b_sn + j * b_sj], of b_dt -- and rounded while staged, in place
  // of bl (nullptr: bl)
  const void* braw;
  int b_dt;
  int64_t b_sn, b_sj;
  bool b_vec;            // b_sj == 1 and braw rows 16-byte aligned (fp32 vector loads)
  float scaling;         // 1 for dX
  // FP8: y = RND(RND(acc * (*post_a) * (*post_b)) + RND(bias)) (the scaled
  // product is rounded before the bias is added); nullptr otherwise
  const float* post_a;
  const float* post_b;
  uint16_t* y;
  int64_t ldy;
};

// Byte offset of 16-byte chunk c of row r in a swizzled 128-byte-row tile.
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) { return r * 128u + ((c ^ ((r >> 1) & 7u)) << 4); }

// Waits until at most N vector-memory loads of this wave are outstanding.
// The activation ring is read through LDS, which the compiler's own wait
// insertion does not track, so the kernel places these waits itself.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier for the k loop: this wave's LDS stores are complete and
// at most N of its vector-memory loads are still outstanding, then s_barrier.
// (__syncthreads() would also drain every global load -- including the
// packed-weight prefetch issued just before -- and expose a full memory
// latency on every step.)
template <int N>
__device__ __forceinline__ void step_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// One direct-to-LDS load: 16 bytes per lane from global memory (wave-uniform
// base + 32-bit byte offset) to LDS address lds_addr + 16 * lane.  Written
// as inline assembly so that the compiler's wait insertion does not treat it
// as an outstanding LDS access (it would otherwise drain every LDS read with
// lgkmcnt(0) after each such load); the kernel waits for these loads itself
// (wait_vmcnt / step_barrier).  The static LDS block starts at address 0, so
// LDS addresses are byte offsets into it.
__device__ __forceinline__ void dma16(const void* base, uint32_t byte_off, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(byte_off), "s"(base), "s"(lds_addr)
               : "memory", "m0");
}

// Table address of byte h of a packed dword (v_perm_b32 puts the code byte
// in bits 8..15 next to the lane's copy offset).
__device__ __forceinline__ uint32_t lut_addr(uint32_t word, uint32_t lane_off, int h) {
  return __builtin_amdgcn_perm(word, lane_off, 0x0C0C0000u | (uint32_t(4 + h) << 8));
}
__device__ __forceinline__ u32x2 lut_read(const u32x2* lut, uint32_t addr) {
  return *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(lut) + addr);
}

// ---------------------------------------------------------------------------
// Weight producers.  Interface (all per thread):
//   Regs                     one step's packed weights and scales (registers)
//   kLoads                   vector-memory loads issued by issue()
//   issue(R, kstep)          load step kstep's packed weights and scales
//   Step                     per-step dequantization state
//   prep(S, R)               everything derived from R (scales, table
//                            addresses); called before the step's
//                            direct-to-LDS loads, so that no later
//                            instruction waits on a register load
//   lookup(S, p)             table reads of piece p (p = 0..3)
//   finish(S, p, h, tile)    half h of piece p's scale-multiply and rounding,
//                            and its LDS stores into the operand tile
// ---------------------------------------------------------------------------
struct ProducerParams {
  const uint8_t* packed;
  int64_t row_bytes;        // bytes per packed weight row (layer K / 2)
  int64_t rows;             // layer N (weight rows)
  int64_t blocks_per_row;   // layer K / block_size
  int bs_log2;
};

// One 64-k step for a wave's 64 x 128 tile, software-pipelined by hand so
// that the matrix cores never wait on the rest of the wave's work: an MFMA
// keeps the core busy for 32 cycles, in which the wave can issue a few VALU,
// LDS and vector-memory instructions, so that work is spread between the
// MFMAs (in-order issue would otherwise leave the core idle while a batch of
// it drains).  Sub-step s (k = 16 s + 8 q + e, eight MFMAs in four pairs):
//   head:   activation and weight operand reads of sub-step s + 1;
//   pair 0: (s < 2) four of the eight direct-to-LDS loads of step j + 1;
//   pair 1: table lookups of piece s + 1 of the next step's weights;
//   pair 2, 3: the two halves of piece s's scale-multiply, rounding and
//           LDS stores into the other weight tile; after the last pair, the
//           packed weights of step j + 4 (the last loads of the step, so the
//           next step's activation wait leaves them in flight).
// Scheduling fences pin each group.
template <int XT, class Prod>
__device__ __forceinline__ void gemm_step(f32x16 (&acc)[kGemmMB][kGemmNB], const uint8_t* xr, const uint8_t* wt,
                                          int i32, int q, const GemmArgs& a, const uint32_t (&xo)[8],
                                          int64_t kx, uint32_t xdst, const Prod& prod,
                                          const typename Prod::Regs& wq, typename Prod::Regs& wl_fill,
                                          int64_t kfill, uint8_t* wdst) {
  typename Prod::Step S;
  prod.prep(S, wq);
  auto read_ops = [&](u32x4 (&xa)[kGemmMB], u32x4 (&b)[kGemmNB], int s) {
    const uint32_t c = uint32_t(2 * s + q);
#pragma unroll
    for (int mb = 0; mb < kGemmMB; ++mb)
      xa[mb] = *reinterpret_cast<const u32x4*>(xr + swz(uint32_t(32 * mb + i32), c));
#pragma unroll
    for (int nb = 0; nb < kGemmNB; ++nb)
      b[nb] = *reinterpret_cast<const u32x4*>(wt + swz(uint32_t(32 * nb + i32), c));
  };
  u32x4 xa[kGemmMB], b[kGemmNB], xan[kGemmMB], bn[kGemmNB];
  read_ops(xa, b, 0);
  prod.lookup(S, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s < 3) read_ops(xan, bn, s + 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int nb = 0; nb < kGemmNB; ++nb) {
#pragma unroll
      for (int mb = 0; mb < kGemmMB; ++mb) acc[mb][nb] = mfma32x32x16<XT>(xa[mb], b[nb], acc[mb][nb]);
      if (nb == 0) {
        if (s < 2) {
#pragma unroll
          for (int t = 4 * s; t < 4 * s + 4; ++t) dma16(a.x, (xo[t] + uint32_t(kx) * kGemmBK) * 2u, xdst + t * 1024);
        }
      } else if (nb == 1) {
        if (s < 3) prod.lookup(S, s + 1);
      } else {
        prod.finish(S, s, nb - 2, wdst);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (s < 3) {
#pragma unroll
      for (int mb = 0; mb < kGemmMB; ++mb) xa[mb] = xan[mb];
#pragma unroll
      for (int nb = 0; nb < kGemmNB; ++nb) b[nb] = bn[nb];
    }
  }
  prod.issue(wl_fill, kfill);
  __builtin_amdgcn_sched_barrier(0);
}

template <int XT, class Prod, class Scale>
__global__ __launch_bounds__(kGemmThreads) void nf4_gemm_kernel(GemmArgs a, ProducerParams pp, Scale scale,
                                                                GemmEpi e) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kGemmLds];
  u32x2* lut = reinterpret_cast<u32x2*>(lds);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i32 = lane & 31, q = lane >> 5;

  // tile of this workgroup
  const int64_t T = int64_t(a.tiles_m) * a.tiles_n;
  const int64_t g = blockIdx.x;
  const int64_t t = a.xcd_map ? (g % 8) * (T / 8) + g / 8 : g;
  const int64_t mt = t / a.tiles_n, nt = t % a.tiles_n;
  const int64_t m0 = mt * kGemmBM, n0 = nt * kGemmBN;
  const int64_t m0w = m0 + 64 * wave;
  const int64_t nk = a.K / kGemmBK;

  // Activation DMA lanes: per instruction t, row r = 8t + lane / 8 of the
  // wave, chunk (lane % 8) ^ ((r / 2) & 7); element offsets are 32-bit (the
  // host keeps the activations under 4 GiB).
  uint32_t xo[8];
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) {
    const int r = 8 * tt + (lane >> 3);
    int64_t m = m0w + r;
    m = m < a.M ? m : a.M - 1;  // rows past M re-read a live row; never stored
    xo[tt] = uint32_t(m * a.ldx + 8 * ((lane & 7) ^ ((r >> 1) & 7)));
  }
  uint8_t* xring = lds + kXRingOff + wave * kXWaveBytes;  // + (step & 1) * kXStepBytes
  const uint32_t xring_addr = __builtin_amdgcn_readfirstlane(uint32_t(kXRingOff + wave * kXWaveBytes));
  uint8_t* wtile = lds + kWTileOff;                       // + (step & 1) * kWTileBytes
  Prod prod;
  prod.init(pp, scale, lut, tid, n0);

  // Staggered start: step j covers k-step ks(j) = (j + k_off) mod nk.
  // Workgroups sharing an activation row slice (one XCD) and those sharing a
  // weight tile (one per XCD) start at different steps, so that one of them
  // misses on each line and the rest find it in L2 or the MALL.
  const int nk32 = __builtin_amdgcn_readfirstlane(int(nk));
  const int k_off = __builtin_amdgcn_readfirstlane(int((((nt + 4 * mt) & 31) * nk) >> 5));
  auto ks = [&](int64_t j) -> int64_t {
    int v = int(j) + k_off;
    v = v >= nk32 ? v - nk32 : v;
    v = v >= nk32 ? v - nk32 : v;
    return v;
  };

  // prologue: activations of step 0, packed weights of steps 0..3, the
  // table, and step 0's weight tile
  {
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) dma16(a.x, (xo[tt] + uint32_t(ks(0)) * kGemmBK) * 2u, xring_addr + tt * 1024);
  }
  typename Prod::Regs wl[kWDepth];
#pragma unroll
  for (int d = 0; d < kWDepth; ++d) prod.issue(wl[d], ks(d));
  fill_f32pair_lut<kGemmThreads * 2>(lut, tid);  // the 512-thread fill pattern, in two halves
  fill_f32pair_lut<kGemmThreads * 2>(lut, tid + kGemmThreads);
  __syncthreads();
  {
    typename Prod::Step S;
    prod.prep(S, wl[0]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      prod.lookup(S, p);
      prod.finish(S, p, 0, wtile);
      prod.finish(S, p, 1, wtile);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();

  f32x16 acc[kGemmMB][kGemmNB];
#pragma unroll
  for (int mb = 0; mb < kGemmMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kGemmNB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

  // Step j: MFMAs on weight tile j % 2 and activation ring slot j % 2;
  // direct-to-LDS loads of activations j + 1 into slot (j + 1) % 2;
  // dequantize step j + 1 from wl[(j + 1) % 4] into tile (j + 1) % 2;
  // packed weights j + 4 into wl[j % 4]; then wait for this wave's
  // activation loads (all but the step's kLoads trailing weight loads) and
  // barrier.  Four steps per iteration index every register set statically;
  // the loop has a single exit, so the accumulators stay in place.  Steps
  // past the end wrap around K (in bounds; their results are never used).
  // In the loop, each step's last vector-memory loads are the kLoads weight
  // loads, whose registers later steps consume; the barrier leaves them in
  // flight.  In the tail the weight loads feed nothing, so the compiler drops
  // them, and the barrier must wait for every load (the activations of the
  // next step would otherwise be read before they land).
#define RQ_GEMM_STEP(J, P, WAIT)                                                                               \
  do {                                                                                                         \
    gemm_step<XT, Prod>(acc, xring + ((P) & 1) * kXStepBytes, wtile + ((P) & 1) * kWTileBytes, i32, q, a, xo,  \
                        ks((J) + 1), xring_addr + (((P) + 1) & 1) * kXStepBytes, prod, wl[((P) + 1) & 3], wl[P], \
                        ks((J) + kWDepth), wtile + (((P) + 1) & 1) * kWTileBytes);                             \
    step_barrier<WAIT>();                                                                                      \
  } while (0)
  int64_t j = 0;
  for (; j + 4 <= nk; j += 4) {
    RQ_GEMM_STEP(j, 0, Prod::kLoads);
    RQ_GEMM_STEP(j + 1, 1, Prod::kLoads);
    RQ_GEMM_STEP(j + 2, 2, Prod::kLoads);
    RQ_GEMM_STEP(j + 3, 3, Prod::kLoads);
  }
  const int64_t rem = nk - j;
  if (rem > 0) RQ_GEMM_STEP(j, 0, 0);
  if (rem > 1) RQ_GEMM_STEP(j + 1, 1, 0);
  if (rem > 2) RQ_GEMM_STEP(j + 2, 2, 0);
#undef RQ_GEMM_STEP
  wait_vmcnt<0>();  // nothing may still be landing in LDS when the epilogue reuses it

  // ---- epilogue.  y = RND(RND(acc + RND(bias)) + RND(RND(lora) * scaling))
  // with lora = RND(u) RND(B)^T accumulated by MFMA in chunks of 64 ranks,
  // both operands staged from their pre-rounded 16-bit copies into LDS
  // (u rows of the tile, B rows of the tile, 144-byte pitch).
  const int rank = e.rank;
  f32x16 lo[kGemmMB][kGemmNB];
#pragma unroll
  for (int mb = 0; mb < kGemmMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kGemmNB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) lo[mb][nb][r] = 0.0f;
  if (rank > 0) {
    constexpr int kP = 72;  // staging pitch in elements
    uint16_t* us = reinterpret_cast<uint16_t*>(lds);   // [256][kP]
    uint16_t* bs = us + kGemmBM * kP;                  // [128][kP]
    for (int j0 = 0; j0 < e.rank16; j0 += 64) {
      const int w8 = (e.rank16 - j0 < 64 ? e.rank16 - j0 : 64) / 8;  // 16-byte chunks per row
      __syncthreads();  // the tiles, ring and table (first chunk) or the last chunk's operands are free
      for (int idx = tid; idx < kGemmBM * w8; idx += kGemmThreads) {
        const int r = idx / w8, c = idx - r * w8;
        int64_t m = m0 + r;
        m = m < a.M ? m : a.M - 1;
        *reinterpret_cast<u32x4*>(us + r * kP + 8 * c) =
            *reinterpret_cast<const u32x4*>(e.u + m * e.rank16 + j0 + 8 * c);
      }
      for (int idx = tid; idx < kGemmBN * w8; idx += kGemmThreads) {
        const int r = idx / w8, c = idx - r * w8;
        int64_t n = n0 + r;
        n = n < a.N ? n : a.N - 1;
        *reinterpret_cast<u32x4*>(bs + r * kP + 8 * c) =
            *reinterpret_cast<const u32x4*>(e.bl + n * e.rank16 + j0 + 8 * c);
      }
      __syncthreads();
      for (int s = 0; s < w8 / 2; ++s) {
        u32x4 ua[kGemmMB];
#pragma unroll
        for (int mb = 0; mb < kGemmMB; ++mb)
          ua[mb] = *reinterpret_cast<const u32x4*>(us + (64 * wave + 32 * mb + i32) * kP + 16 * s + 8 * q);
#pragma unroll
        for (int nb = 0; nb < kGemmNB; ++nb) {
          const u32x4 ub = *reinterpret_cast<const u32x4*>(bs + (32 * nb + i32) * kP + 16 * s + 8 * q);
#pragma unroll
          for (int mb = 0; mb < kGemmMB; ++mb) lo[mb][nb] = mfma32x32x16<XT>(ua[mb], ub, lo[mb][nb]);
        }
      }
    }
  }
#pragma unroll
  for (int nb = 0; nb < kGemmNB; ++nb) {
    const int64_t n = n0 + 32 * nb + i32;
    if (n >= a.N) continue;
    const float bias = e.bias ? round_x<XT>(load_as_f32(e.bias, n, e.bias_dt)) : 0.0f;
    const float post = e.post_a ? __fmul_rn(*e.post_a, *e.post_b) : 1.0f;
#pragma unroll
    for (int mb = 0; mb < kGemmMB; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0w + 32 * mb + 8 * (r >> 2) + 4 * q + (r & 3);
        if (m >= a.M) continue;
        float v = acc[mb][nb][r];
        if (e.post_a) {
          v = round_x<XT>(__fmul_rn(v, post));
          if (e.bias) v = round_x<XT>(__fadd_rn(v, bias));
        } else {
          if (e.bias) v = __fadd_rn(v, bias);
          v = round_x<XT>(v);
        }
        if (rank > 0)
          v = round_x<XT>(__fadd_rn(v, round_x<XT>(__fmul_rn(round_x<XT>(lo[mb][nb][r]), e.scaling))));
        e.y[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side planning and launch (shared by the entry points)
// ---------------------------------------------------------------------------
struct GemmPlan {
  int tiles_m, tiles_n;
  bool xcd_map;
  int splits, lf, lt;  // see GemmArgs; lt = split tiles per XCD
  size_t part_offset;
  int rank16;
  LoraRowsPlan lr;
  size_t u16_offset, bl16_offset, ws_bytes;
};

// M activation rows, N output columns, K reduction; the LoRA operands are
// u [M][r16] (product of activations with an [r][K] matrix) and bl
// [N][r16].  Workspace: [lora_rows partials][RND(S) r x K][u16][bl16].
inline GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t rank, int cus, bool split_ok = false) {
  GemmPlan p{};
  p.tiles_m = int((M + kGemmBM - 1) / kGemmBM);
  p.tiles_n = int((N + kGemmBN - 1) / kGemmBN);
  const int64_t T = int64_t(p.tiles_m) * p.tiles_n;
  p.xcd_map = T % 8 == 0;
  // The tiles of an XCD past its last whole wave (cus / 8 workgroups per
  // XCD) run as K splits while the split tiles still fit in one wave (at
  // least 8 steps of 64 k per split).
  p.splits = 1;
  p.lf = int(T / 8);
  p.lt = 0;
  if (split_ok && p.xcd_map) {
    const int64_t L = T / 8, c8 = cus / 8 > 0 ? cus / 8 : 1;
    const int64_t lf = (L / c8) * c8, lt = L - lf;
    int s = 1;
    while (lt > 0 && s < kGemmMaxSplits && lt * s * 2 <= c8 && K / kGemmBK / (s * 2) >= 8) s *= 2;
    if (s > 1) {
      p.splits = s;
      p.lf = int(lf);
      p.lt = int(lt);
    }
  }
  p.rank16 = int((rank + 15) & ~int64_t(15));
  p.ws_bytes = 0;
  if (rank > 0) {
    p.lr = plan_lora_rows(M, K, rank, cus);
    p.u16_offset = p.lr.part_bytes + p.lr.s16_bytes;
    p.bl16_offset = p.u16_offset + ((size_t(M) * p.rank16 * 2 + 255) & ~size_t(255));
    p.ws_bytes = p.bl16_offset + size_t(N) * p.rank16 * 2;
  }
  p.part_offset = (p.ws_bytes + 255) & ~size_t(255);
  if (p.splits > 1) p.ws_bytes = p.part_offset + size_t(p.splits) * 8 * p.lt * kGemmBM * kGemmBN * 4;
  return p;
}


template <int XT, template <int, class> class ProdT, class Scale>
static inline int launch_core(const GemmArgs& a, const ProducerParams& pp, Scale scale, const GemmEpi& e,
                       hipStream_t stream) {
  const unsigned grid = unsigned(int64_t(a.tiles_m) * a.tiles_n);
  nf4_gemm_kernel<XT, ProdT<XT, Scale>, Scale><<<grid, kGemmThreads, 0, stream>>>(a, pp, scale, e);
  return rq_check_launch();
}

// Scale provider by format: absmax of its dtype, or double quantization
// (c2 codes of c2_format with c2_scales of their dtype).
template <int XT, template <int, class> class ProdT>
static inline int run_core(const GemmArgs& a, const ProducerParams& pp, const void* absmax, int absmax_dtype,
                    const uint8_t* c2, int c2_format, int64_t block2, const GemmEpi& e, hipStream_t stream) {
  if (c2) {
    const int sh = pow2_shift(block2);
    switch (absmax_dtype) {
      case RQ_DTYPE_F32:
        return launch_core<XT, ProdT>(a, pp, ScaleDQ<RQ_DTYPE_F32>{c2, absmax, c2_format, sh, block2}, e, stream);
      case RQ_DTYPE_BF16:
        return launch_core<XT, ProdT>(a, pp, ScaleDQ<RQ_DTYPE_BF16>{c2, absmax, c2_format, sh, block2}, e, stream);
      default:
        return launch_core<XT, ProdT>(a, pp, ScaleDQ<RQ_DTYPE_F16>{c2, absmax, c2_format, sh, block2}, e, stream);
    }
  }
  switch (absmax_dtype) {
    case RQ_DTYPE_F32: return launch_core<XT, ProdT>(a, pp, ScaleAbsmax<RQ_DTYPE_F32>{absmax}, e, stream);
    case RQ_DTYPE_BF16: return launch_core<XT, ProdT>(a, pp, ScaleAbsmax<RQ_DTYPE_BF16>{absmax}, e, stream);
    default: return launch_core<XT, ProdT>(a, pp, ScaleAbsmax<RQ_DTYPE_F16>{absmax}, e, stream);
  }
}

inline bool offsets_fit(int64_t M, int64_t ld, int64_t N, int64_t K) {
  // activation and packed-weight loads use 32-bit byte offsets
  return double(M) * double(ld) * 2.0 < 4294967296.0 && double(N) * double(K) * 0.5 < 4294967296.0;
}


}  // namespace rq
