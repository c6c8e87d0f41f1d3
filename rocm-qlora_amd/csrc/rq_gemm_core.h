// Shared pieces of the NF4/byte-weight MFMA GEMM for gfx950 (the forward
// GEMM, the dX backward and the INT8/FP8 linears): tile and LDS layout
// constants, kernel arguments, the swizzle, wait and direct-to-LDS helpers,
// the producer interface, and the host-side plan.  The kernel itself is
// nf4_gemm8_kernel (rq_gemm8.h).
#pragma once
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"
#include "rq_lora.h"

namespace rq {

constexpr int kGemmBM = 256;
constexpr int kGemmBN = 128;
constexpr int kGemmBK = 64;
constexpr int kLutBytes = kF32PairLutQwords * 8;     // 64 KiB
constexpr int kXWaveBytes = 64 * 128;                // one 64-row slice of one step
constexpr int kXStepBytes = 4 * kXWaveBytes;         // 32 KiB
constexpr int kWTileBytes = kGemmBN * 128;           // 16 KiB
constexpr int kXRingOff = kLutBytes;
constexpr int kWTileOff = kXRingOff + 2 * kXStepBytes;
constexpr int kGemmLds = kWTileOff + 2 * kWTileBytes;  // 160 KiB
constexpr int kWDepth = 4;                           // packed-weight prefetch distance in steps
constexpr int kGemmMaxSplits = 4;                    // K splits of a tile
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
  float* part;         // [splits][8 lt][16 x 512 x 4] fp32 (chunk, thread, value)
  uint32_t* tile_cnt;  // [8 lt]
};

struct GemmEpi {
  const void* bias;
  int bias_dt;
  int rank, rank16;      // LoRA rank and rank rounded up to 16
  const uint16_t* u;     // RND(u) [M][rank16] (dX: RND(g)), zero padded
  // the other LoRA operand, B [N][rank] (dX: A^T [K][rank]), read as it is --
  // element (n, j) at braw[n * b_sn + j * b_sj], of b_dt -- and rounded to
  // the activation dtype while the epilogue stages it
  const void* braw;
  int b_dt;
  int64_t b_sn, b_sj;
  bool b_vec;            // b_sj == 1 and braw rows 16-byte aligned (fp32 vector loads)
  // rank16 <= 64, rank % 8 == 0, b_sj == 1 and u and braw rows 16-byte
  // aligned: the kernel reads the tile's u and B rows into registers during
  // its prologue, 16 bytes at a time
  bool lora_regs;
  float scaling;         // 1 for dX
  // dX with LoRA dropout: the adapter term is RND(RND(lora) * (mask ? mask_scale
  // : 0)) (dropout's backward, mask [M][N] bytes with row stride ldm);
  // nullptr otherwise
  const uint8_t* mask;
  int64_t ldm;
  float mask_scale;
  uint16_t* y;
  int64_t ldy;
};

// Byte offset of 16-byte chunk c of row r in a swizzled 128-byte-row tile.
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) { return r * 128u + ((c ^ ((r >> 1) & 7u)) << 4); }
// The weight tile's swizzle: also rows 2i and 2i + 1 take different chunk
// permutations.  The producers store a tile row's chunks from four adjacent
// lanes; with swz the stores of rows 2i and 2i + 1 met in the same banks
// (the forward GEMM's only LDS bank conflicts, 14 % of its LDS cycles),
// while the MFMA operand reads (16 consecutive rows of one chunk) stay
// conflict-free with either.
__device__ __forceinline__ uint32_t swzw(uint32_t r, uint32_t c) {
  return r * 128u + ((c ^ (((r >> 1) ^ (r & 1u)) & 7u)) << 4);
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
//   lookup(S, p)             table reads of piece p
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
  size_t u16_offset, ws_bytes;
};

// M activation rows, N output columns, K reduction; the LoRA operand u
// [M][r16] is the product of the activations with an [r][K] matrix.
// Workspace: [lora_rows partials][u16][K-split tiles].
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
    p.u16_offset = p.lr.part_bytes;
    p.ws_bytes = p.u16_offset + size_t(M) * p.rank16 * 2;
  }
  p.part_offset = (p.ws_bytes + 255) & ~size_t(255);
  if (p.splits > 1) p.ws_bytes = p.part_offset + size_t(p.splits) * 8 * p.lt * kGemmBM * kGemmBN * 4;
  return p;
}


inline bool offsets_fit(int64_t M, int64_t ld, int64_t N, int64_t K) {
  // activation and packed-weight loads use 32-bit byte offsets
  return double(M) * double(ld) * 2.0 < 4294967296.0 && double(N) * double(K) * 0.5 < 4294967296.0;
}


}  // namespace rq
