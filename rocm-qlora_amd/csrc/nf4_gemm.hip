// NF4 prefill / training GEMM (M > 16 rows of activations) for gfx950, and
// the training backward dX on the same core:
//   y[M, N]  = RND(RND(x W^T + RND(bias)) + RND(RND(RND(u) RND(B)^T) * scaling))
//   dX[M, K] = RND(RND(dY W) + RND(RND(g) RND(A)))
//              with g = RND(RND(dY * scaling) RND(B)) (dequant_matmul.py:338-351
//              for the base, lora_layer.py:67 differentiated for the adapter)
// with W = RND(T[code] * scale) dequantized exactly as the reference does
// (quant_ops.py:144-148 then .to(x.dtype), quant_linear.py:191-193) and the
// LoRA term of lora_layer.py:67-70 fused into the epilogue (RND(u) and RND(B)
// come from the LoRA operand kernels of rq_lora.hip).
//
// The core multiplies activation rows (x, or dY) by a weight operand tile
// that a producer policy dequantizes into LDS: FwdProducer writes W rows
// (output feature n, reduction k), DxProducer writes W^T rows (output
// feature k, reduction n) by dequantizing a 64 x 128 block of W and storing
// it transposed.  Below, "columns" are output features and "k" is the
// reduction index of the core.
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

// Core problem: out[M, N] = act[M, K] . op[N, K]^T (+ epilogue).
struct GemmArgs {
  const uint16_t* x;  // activations (x forward, dY for dX), row stride ldx
  int64_t ldx;
  int64_t M, N, K;    // rows, output columns, reduction length
  int tiles_m, tiles_n;
  bool xcd_map;       // tiles of one row slice on one XCD
};

struct GemmEpi {
  const void* bias;
  int bias_dt;
  int rank, rank16;      // LoRA rank and rank rounded up to 16
  const uint16_t* u;     // RND(u) [M][rank16] (dX: RND(g)), zero padded
  const uint16_t* bl;    // RND(B) [N][rank16] (dX: RND(A^T)), zero padded
  float scaling;         // 1 for dX
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

// Forward: tile row = output feature n, 64 reduction k per step.  Thread t
// dequantizes row t / 2, codes 32 (t % 2) .. +32 of the step (16 packed
// bytes, 4 pieces of 8 codes).
template <int XT, class Scale>
struct FwdProducer {
  static constexpr int kLoads = 1 + Scale::kLoads;
  struct Regs {
    u32x4 w;
    typename Scale::Raw s;
  };
  struct Step {
    float sc;
    uint32_t taddr[4][4];
    u32x2 lk[2][4];
    uint32_t r[4];
  };
  ProducerParams P;
  Scale scale;
  const u32x2* lut;
  uint32_t lane_off, tile_row, half, wrow;
  int64_t wn;

  __device__ __forceinline__ void init(const ProducerParams& p, const Scale& sc, const u32x2* l, int tid,
                                       int64_t col0) {
    P = p;
    scale = sc;
    lut = l;
    lane_off = uint32_t(tid & 31) * 8u;
    tile_row = uint32_t(tid >> 1);
    half = uint32_t(tid & 1);
    wn = col0 + tile_row;
    wn = wn < P.rows ? wn : P.rows - 1;  // rows past N re-read a live row; never stored
    wrow = uint32_t(wn * P.row_bytes + 16 * half);  // the host keeps the weights under 4 GiB
  }
  __device__ __forceinline__ void issue(Regs& R, int64_t kstep) const {
    R.w = *reinterpret_cast<const u32x4*>(P.packed + (wrow + uint32_t(kstep) * 32u));
    R.s = scale.load(wn * P.blocks_per_row + ((kstep * kGemmBK) >> P.bs_log2));
  }
  __device__ __forceinline__ void prep(Step& S, const Regs& R) const {
    S.sc = scale.value(R.s);
    const uint32_t words[4] = {R.w.x, R.w.y, R.w.z, R.w.w};
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int h = 0; h < 4; ++h) S.taddr[p][h] = lut_addr(words[p], lane_off, h);
  }
  __device__ __forceinline__ void lookup(Step& S, int p) const {
#pragma unroll
    for (int h = 0; h < 4; ++h) S.lk[p & 1][h] = lut_read(lut, S.taddr[p][h]);
  }
  __device__ __forceinline__ void finish(Step& S, int p, int hh, uint8_t* tile) const {
#pragma unroll
    for (int h = 2 * hh; h < 2 * hh + 2; ++h)
      S.r[h] = cvt_pk<XT>(__fmul_rn(u2f(S.lk[p & 1][h].x), S.sc), __fmul_rn(u2f(S.lk[p & 1][h].y), S.sc));
    if (hh == 1)
      *reinterpret_cast<u32x4*>(tile + swz(tile_row, 4u * half + uint32_t(p))) = u32x4{S.r[0], S.r[1], S.r[2], S.r[3]};
  }
};

// dX: tile row = layer input feature k (output column of dX), 64 reduction
// n (layer output features) per step.  Thread t dequantizes rows
// n = 64 kstep + 4 (t % 16) + i (i = 0..3, piece i) at layer columns
// col0 + 8 (t / 16) .. +8 (one packed dword per row) and stores the 4 x 8
// block transposed: for each of its 8 k, the 4 n values as one 8-byte
// store.  16 consecutive lanes cover one k row's 64 n (all 128 bytes);
// odd-numbered column groups store their rows in swapped pair order so that
// the two groups served together hit different row parities (bank halves).
template <int XT, class Scale>
struct DxProducer {
  static constexpr int kLoads = 4 * (1 + Scale::kLoads);
  struct Regs {
    uint32_t w[4];
    typename Scale::Raw s[4];
  };
  struct Step {
    float sc[4];
    uint32_t taddr[4][4];
    u32x2 lk[2][4];
    float v[8];       // piece 0 / 2 products, waiting for their partner
    uint32_t pr[2][8];  // {n, n + 1} pairs of pieces (0, 1) and (2, 3)
  };
  ProducerParams P;
  Scale scale;
  const u32x2* lut;
  uint32_t lane_off, rg, dcol, swap, boff;
  int64_t kcol;

  __device__ __forceinline__ void init(const ProducerParams& p, const Scale& sc, const u32x2* l, int tid,
                                       int64_t col0) {
    P = p;
    scale = sc;
    lut = l;
    lane_off = uint32_t(tid & 31) * 8u;
    rg = uint32_t(tid & 15);
    dcol = uint32_t(tid >> 4);
    swap = dcol & 1u;
    const int64_t layer_k = P.row_bytes * 2;
    kcol = col0 + 8 * dcol;
    kcol = kcol < layer_k ? kcol : layer_k - 8;  // columns past K re-read live codes; never stored
    boff = uint32_t(kcol >> 1);
  }
  __device__ __forceinline__ void issue(Regs& R, int64_t kstep) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = kstep * kGemmBK + 4 * rg + i;
      R.w[i] = *reinterpret_cast<const uint32_t*>(P.packed + (uint32_t(n * P.row_bytes) + boff));
      R.s[i] = scale.load(n * P.blocks_per_row + (kcol >> P.bs_log2));
    }
  }
  __device__ __forceinline__ void prep(Step& S, const Regs& R) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      S.sc[i] = scale.value(R.s[i]);
#pragma unroll
      for (int h = 0; h < 4; ++h) S.taddr[i][h] = lut_addr(R.w[i], lane_off, h);
    }
  }
  __device__ __forceinline__ void lookup(Step& S, int p) const {
#pragma unroll
    for (int h = 0; h < 4; ++h) S.lk[p & 1][h] = lut_read(lut, S.taddr[p][h]);
  }
  __device__ __forceinline__ void finish(Step& S, int p, int hh, uint8_t* tile) const {
#pragma unroll
    for (int h = 2 * hh; h < 2 * hh + 2; ++h) {
      const float a = __fmul_rn(u2f(S.lk[p & 1][h].x), S.sc[p]);  // k = 2h
      const float b = __fmul_rn(u2f(S.lk[p & 1][h].y), S.sc[p]);  // k = 2h + 1
      if ((p & 1) == 0) {
        S.v[2 * h] = a;
        S.v[2 * h + 1] = b;
      } else {
        S.pr[p >> 1][2 * h] = cvt_pk<XT>(S.v[2 * h], a);
        S.pr[p >> 1][2 * h + 1] = cvt_pk<XT>(S.v[2 * h + 1], b);
      }
    }
    if (p == 3 && hh == 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int e0 = e ^ 1;
        const uint32_t lo = swap ? S.pr[0][e0] : S.pr[0][e];
        const uint32_t hi = swap ? S.pr[1][e0] : S.pr[1][e];
        const uint32_t krow = 8u * dcol + (uint32_t(e) ^ swap);
        *reinterpret_cast<u32x2*>(tile + swz(krow, rg >> 1) + ((rg & 1u) << 3)) = u32x2{lo, hi};
      }
    }
  }
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
#define RQ_GEMM_STEP(J, P)                                                                                     \
  do {                                                                                                         \
    gemm_step<XT, Prod>(acc, xring + ((P) & 1) * kXStepBytes, wtile + ((P) & 1) * kWTileBytes, i32, q, a, xo,  \
                        ks((J) + 1), xring_addr + (((P) + 1) & 1) * kXStepBytes, prod, wl[((P) + 1) & 3], wl[P], \
                        ks((J) + kWDepth), wtile + (((P) + 1) & 1) * kWTileBytes);                             \
    step_barrier<Prod::kLoads>();                                                                              \
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

// M activation rows, N output columns, K reduction; the LoRA operands are
// u [M][r16] (product of activations with an [r][K] matrix) and bl
// [N][r16].  Workspace: [lora_rows partials][RND(S) r x K][u16][bl16].
static GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t rank, int cus) {
  GemmPlan p{};
  p.tiles_m = int((M + kGemmBM - 1) / kGemmBM);
  p.tiles_n = int((N + kGemmBN - 1) / kGemmBN);
  const int64_t T = int64_t(p.tiles_m) * p.tiles_n;
  p.xcd_map = T % 8 == 0;
  p.rank16 = int((rank + 15) & ~int64_t(15));
  p.ws_bytes = 0;
  if (rank > 0) {
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

template <int XT, template <int, class> class ProdT, class Scale>
static int launch_core(const GemmArgs& a, const ProducerParams& pp, Scale scale, const GemmEpi& e,
                       hipStream_t stream) {
  const unsigned grid = unsigned(int64_t(a.tiles_m) * a.tiles_n);
  nf4_gemm_kernel<XT, ProdT<XT, Scale>, Scale><<<grid, kGemmThreads, 0, stream>>>(a, pp, scale, e);
  return rq_check_launch();
}

// Scale provider by format: absmax of its dtype, or double quantization
// (c2 codes of c2_format with c2_scales of their dtype).
template <int XT, template <int, class> class ProdT>
static int run_core(const GemmArgs& a, const ProducerParams& pp, const void* absmax, int absmax_dtype,
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

static bool offsets_fit(int64_t M, int64_t ld, int64_t N, int64_t K) {
  // activation and packed-weight loads use 32-bit byte offsets
  return double(M) * double(ld) * 2.0 < 4294967296.0 && double(N) * double(K) * 0.5 < 4294967296.0;
}

int run_nf4_gemm(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  // the activation operands are loaded 16 bytes at a time
  if (!aligned(L.x, 16) || L.ldx % 8 != 0) return RQ_ERR_BAD_ALIGNMENT;
  if (!offsets_fit(L.M, L.ldx, L.N, L.K)) return RQ_ERR_UNSUPPORTED;
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
  GemmArgs a{};
  a.x = static_cast<const uint16_t*>(L.x);
  a.ldx = L.ldx;
  a.M = L.M;
  a.N = L.N;
  a.K = L.K;
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  a.xcd_map = p.xcd_map;
  ProducerParams pp{L.w_packed, L.K / 2, L.N, L.K / L.block_size, pow2_shift(L.block_size)};
  if (L.x_dtype == RQ_DTYPE_BF16)
    return run_core<RQ_DTYPE_BF16, FwdProducer>(a, pp, L.absmax, L.absmax_dtype, L.c2, L.c2_format, L.block2, e,
                                                stream);
  return run_core<RQ_DTYPE_F16, FwdProducer>(a, pp, L.absmax, L.absmax_dtype, L.c2, L.c2_format, L.block2, e,
                                             stream);
}

// ---------------------------------------------------------------------------
// dX = dY . W_deq (+ LoRA): the core with activations dY [M][N], output
// columns k of the layer, reduction over the layer's N.
// ---------------------------------------------------------------------------
int validate_dx(const DxArgs& D) {
  if (!D.dy || !D.w_packed || !D.absmax || !D.dx) return RQ_ERR_NULL_POINTER;
  if (D.dy_dtype != RQ_DTYPE_BF16 && D.dy_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (D.absmax_dtype != RQ_DTYPE_F32 && D.absmax_dtype != RQ_DTYPE_BF16 && D.absmax_dtype != RQ_DTYPE_F16)
    return RQ_ERR_BAD_DTYPE;
  if (D.M < 0 || D.N <= 0 || D.K <= 0) return RQ_ERR_BAD_SHAPE;
  if (D.N % 64 != 0 || D.K % 64 != 0 || D.block_size < 64 || (D.block_size & (D.block_size - 1)) != 0 ||
      D.K % D.block_size != 0)
    return RQ_ERR_BAD_SHAPE;
  if (D.lddy < D.N || D.lddx < D.K) return RQ_ERR_BAD_SHAPE;
  if (D.c2 && (D.block2 <= 0 || (D.c2_format != RQ_C2_FP8_E4M3FNUZ && D.c2_format != RQ_C2_INT8)))
    return RQ_ERR_BAD_SHAPE;
  if (!aligned(D.dy, 16) || D.lddy % 8 != 0 || !aligned(D.w_packed, 4)) return RQ_ERR_BAD_ALIGNMENT;
  if (!offsets_fit(D.M, D.lddy, D.N, D.K)) return RQ_ERR_UNSUPPORTED;
  if (D.rank > 0) {
    if (!D.lora_a || !D.lora_b) return RQ_ERR_NULL_POINTER;
    if (D.rank > 256 || D.ld_lora_b < D.rank) return RQ_ERR_BAD_SHAPE;
    if (D.lora_dtype != RQ_DTYPE_F32 && D.lora_dtype != D.dy_dtype) return RQ_ERR_BAD_DTYPE;
  }
  return RQ_OK;
}

int dx_workspace(const DxArgs& D, size_t* bytes) {
  *bytes = plan_gemm(D.M, D.K, D.N, D.rank > 0 ? D.rank : 0, device_cus()).ws_bytes;
  return RQ_OK;
}

int run_nf4_dx(const DxArgs& D, void* workspace, size_t ws_bytes, hipStream_t stream) {
  int st = validate_dx(D);
  if (st != RQ_OK) return st;
  if (D.M == 0) return RQ_OK;
  const int64_t rank = D.rank > 0 ? D.rank : 0;
  const GemmPlan p = plan_gemm(D.M, D.K, D.N, rank, device_cus());
  if (p.ws_bytes > 0 && (!workspace || ws_bytes < p.ws_bytes)) return RQ_ERR_WORKSPACE;
  if (workspace && !aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  GemmEpi e{};
  e.rank = int(rank);
  e.rank16 = p.rank16;
  e.scaling = 1.0f;
  e.y = static_cast<uint16_t*>(D.dx);
  e.ldy = D.lddx;
  if (rank > 0) {
    char* ws = static_cast<char*>(workspace);
    uint16_t* g16 = reinterpret_cast<uint16_t*>(ws + p.u16_offset);
    uint16_t* at16 = reinterpret_cast<uint16_t*>(ws + p.bl16_offset);
    // g = RND(RND(dY * s) . RND(B)): S[j][n] = B[n][j]
    st = run_lora_rows(D.dy_dtype, static_cast<const uint16_t*>(D.dy), D.lddy, D.M, D.N, D.lora_b, D.lora_dtype, 1,
                       D.ld_lora_b, int(rank), true, D.scaling, p.lr, reinterpret_cast<float*>(ws),
                       reinterpret_cast<uint16_t*>(ws + p.lr.part_bytes), g16, p.rank16, stream);
    if (st != RQ_OK) return st;
    // RND(A^T) [K][r]: element (k, j) = A[j][k], A [r][K] row-major
    st = run_lora_round(D.dy_dtype, D.lora_a, D.lora_dtype, 1, D.K, D.K, int(rank), p.rank16, at16, stream);
    if (st != RQ_OK) return st;
    e.u = g16;
    e.bl = at16;
  }
  GemmArgs a{};
  a.x = static_cast<const uint16_t*>(D.dy);
  a.ldx = D.lddy;
  a.M = D.M;
  a.N = D.K;
  a.K = D.N;
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  a.xcd_map = p.xcd_map;
  ProducerParams pp{D.w_packed, D.K / 2, D.N, D.K / D.block_size, pow2_shift(D.block_size)};
  if (D.dy_dtype == RQ_DTYPE_BF16)
    return run_core<RQ_DTYPE_BF16, DxProducer>(a, pp, D.absmax, D.absmax_dtype, D.c2, D.c2_format, D.block2, e,
                                               stream);
  return run_core<RQ_DTYPE_F16, DxProducer>(a, pp, D.absmax, D.absmax_dtype, D.c2, D.c2_format, D.block2, e,
                                            stream);
}

}  // namespace rq

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
static rq::DxArgs pack_dx_args(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t lddy,
                               const uint8_t* w_packed, int64_t K, int64_t block_size, const void* absmax,
                               int absmax_dtype, const uint8_t* c2, int c2_format, int64_t block2,
                               const void* lora_a, const void* lora_b, int64_t ld_lora_b, int lora_dtype,
                               int64_t rank, float scaling, void* dx, int64_t lddx) {
  rq::DxArgs D;
  D.dy = dy; D.dy_dtype = dy_dtype; D.M = M; D.N = N; D.lddy = lddy;
  D.w_packed = w_packed; D.K = K; D.block_size = block_size;
  D.absmax = absmax; D.absmax_dtype = absmax_dtype; D.c2 = c2; D.c2_format = c2_format; D.block2 = block2;
  D.lora_a = lora_a; D.lora_b = lora_b; D.ld_lora_b = ld_lora_b; D.lora_dtype = lora_dtype;
  D.rank = (lora_a && lora_b) ? rank : 0; D.scaling = scaling;
  D.dx = dx; D.lddx = lddx;
  return D;
}

extern "C" int rq_nf4_linear_dx_workspace_size(int dy_dtype, int64_t M, int64_t N, int64_t K, int64_t rank,
                                               int64_t* bytes) {
  if (!bytes) return RQ_ERR_NULL_POINTER;
  if (dy_dtype != RQ_DTYPE_BF16 && dy_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || N <= 0 || K <= 0 || rank < 0) return RQ_ERR_BAD_SHAPE;
  rq::DxArgs D{};
  D.M = M; D.N = N; D.K = K; D.rank = rank;
  size_t b = 0;
  const int st = rq::dx_workspace(D, &b);
  *bytes = int64_t(b);
  return st;
}

extern "C" int rq_nf4_linear_dx(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t lddy,
                                const uint8_t* w_packed, int64_t K, int64_t block_size, const void* absmax,
                                int absmax_dtype, const uint8_t* c2, int c2_format, int64_t block2,
                                const void* lora_a, const void* lora_b, int64_t ld_lora_b, int lora_dtype,
                                int64_t rank, float scaling, void* dx, int64_t lddx, void* workspace,
                                int64_t workspace_bytes, hipStream_t stream) {
  const rq::DxArgs D = pack_dx_args(dy, dy_dtype, M, N, lddy, w_packed, K, block_size, absmax, absmax_dtype, c2,
                                    c2_format, block2, lora_a, lora_b, ld_lora_b, lora_dtype, rank, scaling, dx,
                                    lddx);
  return rq::run_nf4_dx(D, workspace, workspace_bytes < 0 ? 0 : size_t(workspace_bytes), stream);
}
