// NF4 prefill / training GEMM (M > 16 rows of activations) for gfx950:
//   y[M, N] = RND(RND(x W^T + RND(bias)) + RND(RND(RND(u) RND(B)^T) * scaling))
// with W = RND(T[code] * scale) dequantized exactly as the reference does
// (quant_ops.py:144-148 then .to(x.dtype), quant_linear.py:191-193) and the
// LoRA term of lora_layer.py:67-70 fused into the epilogue (RND(u) and RND(B)
// come from the LoRA operand kernels of rq_lora.hip).
//
// Workgroup tile 256 tokens x 128 features, 4 waves; wave w owns rows
// 64 w .. 64 w + 63 and all 128 columns as 2 x 4 blocks of
// v_mfma_f32_32x32x16_{bf16,f16}.  K advances 64 per step -- one NF4 block
// per weight row, one scale per row per step.  LDS (160 KiB, all of it):
//   [0, 64K)     the fp32 pair table for exact dequantization (address 0,
//                so lookups fold their base into the instruction offset);
//   [64K, 128K)  activation ring: 2 steps x 4 waves x 64 rows x 128 bytes;
//   [128K, 160K) weight tiles: 2 steps x 128 rows x 128 bytes.
// Both LDS layouts store 16-byte chunk c of row r at slot c ^ ((r / 2) & 7)
// of the row: the LDS serves 16 lanes x 16 bytes (its 64 banks) per cycle,
// and 16 consecutive rows then cover 16 distinct 16-byte bank groups (row
// parity picks the 128-byte half), so the MFMA operand reads and the
// dequantizer's row-segment stores are conflict-free.
//   * Activations go from global memory straight into the ring with
//     global_load_lds_dwordx4: each instruction moves 8 whole 128-byte rows
//     (8 cache lines; loads that spread 32 rows over one instruction cost the
//     vector L1 32 line lookups and stall the MFMA stream).  Each wave loads
//     and reads only its own rows, so the ring needs no workgroup barrier.
//   * Packed weights (16 bytes per thread per step) and their scales sit in
//     registers four steps ahead; each step dequantizes the next step's tile
//     through the pair table into the other weight tile.
// Tiles are numbered so that the workgroups of one XCD (workgroup id mod 8)
// share activation row slices, which then stay in that XCD's L2, and their
// k loops start staggered so that only one of them misses on each slice.
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
static_assert(kGemmLds == 160 * 1024, "LDS plan");

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
  const uint16_t* bl;    // RND(B) [N][rank16], zero padded
  float scaling;
  uint16_t* y;
  int64_t ldy;
};

// Byte offset of 16-byte chunk c of row r in a swizzled 128-byte-row tile.
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) { return r * 128u + ((c ^ ((r >> 1) & 7u)) << 4); }

// One k-step's packed weights for this thread: 16 bytes (32 codes) of row
// tid / 2, half tid % 2 of the step, and the row's scale.
template <class Scale>
struct GemmWLoads {
  u32x4 w;
  typename Scale::Raw s;
};

template <class Scale>
__device__ __forceinline__ void gemm_issue_w(GemmWLoads<Scale>& L, const GemmArgs& a, const Scale& scale,
                                             uint32_t wrow, int64_t n, int64_t kt) {
  const uint32_t off = wrow + uint32_t(kt) * 32u;  // byte offset; the host keeps the weights under 4 GiB
  L.w = *reinterpret_cast<const u32x4*>(a.packed + off);
  L.s = scale.load(n * a.blocks_per_row + ((kt * kGemmBK) >> a.bs_log2));
}

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

// Issue this wave's 8 direct-to-LDS loads of one step's activations
// (instruction t: rows 8t .. 8t + 7 of the wave, lane l -> row r = 8t + l / 8,
// slot l % 8, which holds chunk (l % 8) ^ ((r / 2) & 7)).  xo[t] is the
// lane's element offset at k-step 0.
__device__ __forceinline__ void x_dma(const GemmArgs& a, const uint32_t (&xo)[8], int64_t kstep, uint32_t dst) {
#pragma unroll
  for (int t = 0; t < 8; ++t) dma16(a.x, (xo[t] + uint32_t(kstep) * kGemmBK) * 2u, dst + t * 1024);
}

// One 64-k step for a wave's 64 x 128 tile, software-pipelined by hand so
// that the matrix cores never wait on the rest of the wave's work: an MFMA
// keeps the core busy for 32 cycles, in which the wave can issue a few VALU,
// LDS and vector-memory instructions, so that work is spread between the
// MFMAs (in-order issue would otherwise leave the core idle while a batch of
// it drains).  Sub-step s (k = 16 s + 8 q + e, eight MFMAs in four pairs):
//   head:   activation and weight operand reads of sub-step s + 1;
//   pair 0: (s < 2) four of the eight direct-to-LDS loads of step j + 1;
//   pair 1: table lookups for dword s + 1 of this thread's packed weights
//           of step j + 1;
//   pair 2, 3: scale-multiply and round dword s's lookups, store the eight
//           dequantized weights to the other weight tile; after the last
//           pair, the packed weights of step j + 4 (the last loads of the
//           step, so the next step's activation wait leaves them in flight).
// Scheduling fences pin each group.
template <int XT, bool DEQ, class Scale>
__device__ __forceinline__ void gemm_step(f32x16 (&acc)[kGemmMB][kGemmNB], const uint8_t* xr, const uint8_t* wt,
                                          int i32, int q, const GemmArgs& a, const uint32_t (&xo)[8],
                                          int64_t kx, uint32_t xdst, const GemmWLoads<Scale>& wq,
                                          GemmWLoads<Scale>& wl_fill, const Scale& scale, uint32_t wrow, int64_t wn,
                                          int64_t kfill, uint8_t* wdst, uint32_t wrow_tile, uint32_t whalf,
                                          const u32x2* lut, uint32_t lane_off) {
  // Everything derived from the packed weights (scale, the 16 table
  // addresses) is computed here, before this step's direct-to-LDS loads:
  // those loads are invisible to the compiler's wait counting, so a later
  // use of a loaded register would make it wait on them too.
  float sc = 0.0f;
  uint32_t taddr[4][4];
  if constexpr (DEQ) {
    sc = scale.value(wq.s);
    const uint32_t words[4] = {wq.w.x, wq.w.y, wq.w.z, wq.w.w};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int h = 0; h < 4; ++h)
        taddr[s][h] = __builtin_amdgcn_perm(words[s], lane_off, 0x0C0C0000u | (uint32_t(4 + h) << 8));
  }
  auto lookup = [&](u32x2 (&lk)[4], int s) {
#pragma unroll
    for (int h = 0; h < 4; ++h)
      lk[h] = *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(lut) + taddr[s][h]);
  };
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
  u32x2 lk[4], lkn[4];
  read_ops(xa, b, 0);
  if constexpr (DEQ) lookup(lk, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s < 3) read_ops(xan, bn, s + 1);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t r[4];
#pragma unroll
    for (int nb = 0; nb < kGemmNB; ++nb) {
#pragma unroll
      for (int mb = 0; mb < kGemmMB; ++mb) acc[mb][nb] = mfma32x32x16<XT>(xa[mb], b[nb], acc[mb][nb]);
      if (nb == 0) {
        if (s < 2) {
#pragma unroll
          for (int t = 4 * s; t < 4 * s + 4; ++t) {
            dma16(a.x, (xo[t] + uint32_t(kx) * kGemmBK) * 2u, xdst + t * 1024);
          }
        }
      } else if (nb == 1) {
        if constexpr (DEQ) {
          if (s < 3) lookup(lkn, s + 1);
        }
      } else if constexpr (DEQ) {
        const int h0 = nb == 2 ? 0 : 2;
#pragma unroll
        for (int h = h0; h < h0 + 2; ++h) r[h] = cvt_pk<XT>(__fmul_rn(u2f(lk[h].x), sc), __fmul_rn(u2f(lk[h].y), sc));
        if (nb == 3)
          *reinterpret_cast<u32x4*>(wdst + swz(wrow_tile, 4u * whalf + uint32_t(s))) = u32x4{r[0], r[1], r[2], r[3]};
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (s < 3) {
#pragma unroll
      for (int mb = 0; mb < kGemmMB; ++mb) xa[mb] = xan[mb];
#pragma unroll
      for (int nb = 0; nb < kGemmNB; ++nb) b[nb] = bn[nb];
#pragma unroll
      for (int h = 0; h < 4; ++h) lk[h] = lkn[h];
    }
  }
  gemm_issue_w(wl_fill, a, scale, wrow, wn, kfill);
  __builtin_amdgcn_sched_barrier(0);
}

template <int XT, class Scale>
__global__ __launch_bounds__(kGemmThreads) void nf4_gemm_kernel(GemmArgs a, Scale scale, GemmEpi e) {
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
  const uint32_t wrow_tile = uint32_t(tid >> 1), whalf = uint32_t(tid & 1);
  int64_t wn = n0 + wrow_tile;
  wn = wn < a.N ? wn : a.N - 1;  // rows past N re-read a live row; never stored
  const uint32_t wrow = uint32_t(wn * (a.K >> 1) + 16 * whalf);  // byte offset of this thread's row segment

  // Staggered start: step j covers k-step ks(j) = (j + k_off) mod nk.
  const int nk32 = __builtin_amdgcn_readfirstlane(int(nk));
  // (workgroups sharing a weight tile, one per XCD, are staggered too, so
  // that one of them misses on each weight line and the rest hit the MALL)
  const int k_off = __builtin_amdgcn_readfirstlane(int((((nt + 4 * mt) & 31) * nk) >> 5));
  auto ks = [&](int64_t j) -> int64_t {
    int v = int(j) + k_off;
    v = v >= nk32 ? v - nk32 : v;
    v = v >= nk32 ? v - nk32 : v;
    return v;
  };

  // prologue: activations of step 0, packed weights of steps 0..3, the
  // table, and step 0's weight tile
  x_dma(a, xo, ks(0), xring_addr);
  GemmWLoads<Scale> wl[kWDepth];
#pragma unroll
  for (int d = 0; d < kWDepth; ++d) gemm_issue_w(wl[d], a, scale, wrow, wn, ks(d));
  fill_f32pair_lut<kGemmThreads * 2>(lut, tid);  // the 512-thread fill pattern, in two halves
  fill_f32pair_lut<kGemmThreads * 2>(lut, tid + kGemmThreads);
  __syncthreads();
  const uint32_t lane_off = uint32_t(lane & 31) * 8u;
  {
    const float sc = scale.value(wl[0].s);
    const uint32_t words[4] = {wl[0].w.x, wl[0].w.y, wl[0].w.z, wl[0].w.w};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      *reinterpret_cast<u32x4*>(wtile + swz(wrow_tile, 4u * whalf + uint32_t(s))) =
          expand8_scaled<XT>(lut, words[s], lane_off, sc);
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
  // activation loads (all but the step's kW trailing weight loads) and
  // barrier.  Four steps per iteration index every register set statically;
  // the loop has a single exit, so the accumulators stay in place.  Steps
  // past the end wrap around K (in bounds; their results are never used).
  constexpr int kW = 1 + Scale::kLoads;  // vector-memory loads of one gemm_issue_w
#define RQ_GEMM_STEP(J, P)                                                                                  \
  do {                                                                                                      \
    gemm_step<XT, true>(acc, xring + ((P) & 1) * kXStepBytes, wtile + ((P) & 1) * kWTileBytes, i32, q, a, xo, \
                        ks((J) + 1), xring_addr + (((P) + 1) & 1) * kXStepBytes, wl[((P) + 1) & 3], wl[P], scale, \
                        wrow, wn, ks((J) + kWDepth), wtile + (((P) + 1) & 1) * kWTileBytes, wrow_tile, whalf,  \
                        lut, lane_off);                                                                     \
    step_barrier<kW>();                                                                                     \
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
#pragma unroll
    for (int mb = 0; mb < kGemmMB; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0w + 32 * mb + 8 * (r >> 2) + 4 * q + (r & 3);
        if (m >= a.M) continue;
        float v = acc[mb][nb][r];
        if (e.bias) v = __fadd_rn(v, bias);
        v = round_x<XT>(v);
        if (rank > 0)
          v = round_x<XT>(__fadd_rn(v, round_x<XT>(__fmul_rn(round_x<XT>(lo[mb][nb][r]), e.scaling))));
        e.y[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct GemmPlan {
  int tiles_m, tiles_n;
  bool xcd_map;
  int rank16;
  LoraRowsPlan lr;
  size_t u16_offset, bl16_offset, ws_bytes;
};

static GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t rank, int cus) {
  GemmPlan p{};
  p.tiles_m = int((M + kGemmBM - 1) / kGemmBM);
  p.tiles_n = int((N + kGemmBN - 1) / kGemmBN);
  const int64_t T = int64_t(p.tiles_m) * p.tiles_n;
  p.xcd_map = T % 8 == 0;
  p.rank16 = int((rank + 15) & ~int64_t(15));
  p.ws_bytes = 0;
  if (rank > 0) {
    // [lora_rows partials][RND(A) r x K][RND(u) M x r16][RND(B) N x r16]
    p.lr = plan_lora_rows(M, K, rank, cus);
    p.u16_offset = p.lr.part_bytes + p.lr.s16_bytes;
    p.bl16_offset = p.u16_offset + ((size_t(M) * p.rank16 * 2 + 255) & ~size_t(255));
    p.ws_bytes = p.bl16_offset + size_t(N) * p.rank16 * 2;
  }
  return p;
}

int gemm_workspace(const LinearArgs& L, size_t* bytes) {
  *bytes = plan_gemm(L.M, L.N, L.K, L.rank, device_cus()).ws_bytes;
  return RQ_OK;
}

template <int XT, class Scale>
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
  nf4_gemm_kernel<XT, Scale><<<grid, kGemmThreads, 0, stream>>>(a, scale, e);
  return rq_check_launch();
}

template <int XT, class Scale>
static int launch_gemm_cfg(const LinearArgs& L, const GemmPlan& p, Scale scale, const GemmEpi& e,
                           hipStream_t stream) {
  return launch_gemm_t<XT>(L, p, scale, e, stream);
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

int run_nf4_gemm(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  // the activation operands are loaded 16 bytes at a time
  if (!aligned(L.x, 16) || L.ldx % 8 != 0) return RQ_ERR_BAD_ALIGNMENT;
  // activation and packed-weight loads use 32-bit byte offsets
  if (double(L.M) * double(L.ldx) * 2.0 >= 4294967296.0 || double(L.N) * double(L.K) * 0.5 >= 4294967296.0)
    return RQ_ERR_UNSUPPORTED;
  const GemmPlan p = plan_gemm(L.M, L.N, L.K, L.rank, device_cus());
  if (p.ws_bytes > 0 && (!workspace || ws_bytes < p.ws_bytes)) return RQ_ERR_WORKSPACE;
  if (workspace && !aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  GemmEpi e{};
  e.bias = L.bias;
  e.bias_dt = L.bias_dtype;
  e.rank = int(L.rank > 0 ? L.rank : 0);
  e.rank16 = p.rank16;
  e.scaling = L.scaling;
  e.y = static_cast<uint16_t*>(L.y);
  e.ldy = L.ldy;
  if (e.rank > 0) {
    char* ws = static_cast<char*>(workspace);
    uint16_t* u16 = reinterpret_cast<uint16_t*>(ws + p.u16_offset);
    uint16_t* bl16 = reinterpret_cast<uint16_t*>(ws + p.bl16_offset);
    // u = RND(xl . RND(A)^T), A [r][K] row-major (lora_layer.py:67)
    int st = run_lora_rows(L.x_dtype, static_cast<const uint16_t*>(L.lora_x), L.ld_lora_x, L.M, L.K, L.lora_a,
                           L.lora_dtype, L.K, 1, e.rank, false, 1.0f, p.lr, reinterpret_cast<float*>(ws),
                           reinterpret_cast<uint16_t*>(ws + p.lr.part_bytes), u16, p.rank16, stream);
    if (st != RQ_OK) return st;
    // RND(B), B [N][r] with row stride ld_lora_b
    st = run_lora_round(L.x_dtype, L.lora_b, L.lora_dtype, L.ld_lora_b, 1, L.N, e.rank, p.rank16, bl16, stream);
    if (st != RQ_OK) return st;
    e.u = u16;
    e.bl = bl16;
  }
  if (L.x_dtype == RQ_DTYPE_BF16) return run_gemm<RQ_DTYPE_BF16>(L, p, e, stream);
  return run_gemm<RQ_DTYPE_F16>(L, p, e, stream);
}

}  // namespace rq
