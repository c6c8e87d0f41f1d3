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
#include <algorithm>
#include <atomic>

#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"
#include "rq_generic.h"

namespace rq {

// ---------------------------------------------------------------------------
// Decode GEMV: y[M <= 16, N] = x[M, K] . W^T, W NF4 (block size a power of
// two >= 64 dividing K, K % 64 == 0).
//
// Work units.  A tile is 16 rows of W; a segment is 256 k of a tile (128
// contiguous code bytes per row); a unit (tile, segment) is 8 MFMA steps of
// one wave.  Workgroup (g, s) of 16 waves owns tiles g, g + G, ..., g + (TS -
// 1) G and the segments of K split s.  The host assigns the units to the
// waves (a table in the kernel arguments; at most 4 units per wave) so that
// every wave has work for any K: one segment per wave when K = 4096, several
// tiles per wave for shorter K, several segments of one tile per wave for
// longer K.
//
// HBM access of a unit: two 1 KiB loads, 4 lanes x 16 B per row and load
// (the two loads together read each row's 128-byte line):
//   load A: lane (n = l % 16, q = l / 16) reads row n, chunk q      -> X1
//   load B: lane (n, q)                   reads row n, chunk q + 4  -> X2
// (chunk = 16 B = 32 k): the 16x16x32 MFMA B-operand layout (lane l = row
// l % 16, k group l / 16) straight from the loads, with no lane exchange or
// LDS round trip.  Steps 0-3 take X1's dwords, steps 4-7 X2's; the
// activation operand (A, rows = tokens, zero past M) uses the same k order.
// Each dword of codes becomes RND(T[code] * scale) through the LDS pair
// table.  Every address is a per-lane constant plus a wave-uniform unit
// offset, so a unit's loads cost a few adds.  (Loads of 8 lanes x 16 B per
// row, with the halves exchanged by a select and a DPP row rotate, measured
// 0.4-0.7 us slower per launch at the 14336 x 4096 shapes: the twelve lane
// operations per unit cost more than the wider pieces gain.)
//
// Schedule.  The code is straight-line: the units are unrolled, no load sits
// under a branch and no loaded value is carried around a loop, so the
// compiler's in-order load counting is exact and each unit waits only for
// its own data.
//   1. With the LoRA down-projection in the launch, the state of the
//      partial regions and, in a wave with a job, the job's operands.  The
//      first unit's loads: its activations (M <= 2 and 16-byte aligned
//      rows: the M x 256 values of the unit's segment, one 16-byte load per
//      lane; otherwise the wave's MFMA operands directly, eight
//      16-byte loads, and all of the wave's units share one segment), then its
//      weights and scales.
//   2. The byte table (built from constants, no loads); one barrier; a job
//      wave's MFMAs and its partials' stores.
//   3. The epilogue operands (the tiles' LoRA B rows, bias, RND(u) partials),
//      kept as raw bits until the end.
//   4. Per unit: issue the next unit's loads; put the unit's activations
//      through the wave's own LDS slice into the MFMA layout (no barrier: the
//      wave writes and reads its slice itself); dequantize and multiply; the
//      16 x M partial goes to LDS, indexed by (tile, segment).
//   5. With the down-projection in the launch, the poll of its partials.
//      The epilogue operands into LDS, one barrier; one thread per output sums
//      its tile's segment partials in segment order (deterministic), adds the
//      bias and the LoRA term, rounds and stores -- or writes the fp32 sum of
//      its K split to the workspace for the split-K finisher.  The launch's
//      last job readies the other partial region for the next launch.
// ---------------------------------------------------------------------------
constexpr int kGemvThreads = 1024;
constexpr int kGemvWaves = kGemvThreads / 64;
constexpr int kSegK = 256;
constexpr int kGemvMaxU = 4;           // units per wave
constexpr int kGemvMaxTS = 4;          // tiles per workgroup
constexpr int kGemvMaxFusedRank = 64;  // LoRA rank the in-kernel epilogue stages
// LDS pitches of the staged LoRA operands, padded so that the epilogue's
// reads are free of bank conflicts: the 16 output columns of a wave read 16
// B rows (16-bit, 144 bytes apart: 16 distinct groups of 4 banks) and its
// four output rows read four u rows (fp32, 272 bytes apart).  Unpadded
// (128 / 256 bytes) the reads were 8-way / 4-way conflicted: 10 % of the
// LoRA launch's LDS cycles at M = 16.
constexpr int kGemvBPitch = kGemvMaxFusedRank + 8;
constexpr int kGemvUPitch = kGemvMaxFusedRank + 4;
constexpr int kGemvMaxUSplits = 16;
constexpr int kGemvXSliceMaxM = 2;  // activation rows through the per-wave LDS slice
constexpr int kGemvLutQwords = 256 * 32;  // 64 KiB: code byte -> fp32 (T[lo], T[hi]), 32 copies
constexpr int kGemvLdsBudget = 160 * 1024 - kGemvLutQwords * 8;

struct GemvArgs {
  const uint16_t* x;
  int ldx;                 // activation row stride (elements)
  const uint8_t* packed;
  int M, N, K;
  int bpr;                 // scale blocks per row, K / block_size
  int bs_log2;             // log2(block_size)
  int nseg;                // segments per K split
  int TS;                  // tiles per workgroup
  bool direct;             // one K split: the epilogue in this kernel
  // K splits (gridDim.y > 1): fp32 partials [S][M][N] to ws; with tile_cnt
  // the last split of a workgroup column to count itself (tile_cnt[g],
  // zero between launches) sums the splits' partials in split order and
  // runs the epilogue, else a finisher launch does
  uint32_t* tile_cnt;
  bool xvec;               // x rows 16-byte aligned (vector loads)
  int bvec_log2;           // LoRA B rows read as 16-byte chunks, 2^bvec_log2 per row (-1: by element)
  float* ws;               // [S, M, N] partials when !direct
  // LoRA down-projection inside this launch (jobs > 0): job b computes the
  // fp32 partials of ranks [16 (b / u_splits), +16) over K split
  // b % u_splits, one wave per job (wave b / G of workgroup b % G, G the
  // workgroups of the launch, workgroup (g, s) of K split s counted as
  // s gridDim.x + g; waves counted from the last when the last waves have
  // fewer units, else from wave 1), into region P [u_splits][M][rank] of parts,
  // P = bit 0 of state[0] as read at the launch's start, +0.0 stored as -0.0
  // so that 0 means "not written yet"; after its units every workgroup polls the
  // partials until none is 0.  No workgroup waits on a count at its end:
  // region P is zero at the start of every launch (but for partials the
  // launch itself writes), and the other region holds the previous launch's
  // partials, state[1 + p] words of region p.  Every job counts itself in
  // *jc after its stores; the last job's wave, at its end, clears the other
  // region, records this launch's extent and flips the parity, so the next
  // launch finds its region zero.  Every job has read the state before it
  // counts itself, and the launch fits the device (one workgroup per compute
  // unit), so the other workgroups have read it before that wave ends; one
  // that starts later (the device shared with other work) finds no partials
  // and computes u itself.
  int jobs;
  uint32_t wait_ticks;     // real-time ticks a workgroup waits before it computes u itself
  uint32_t* jc;            // jobs done (zero between launches)
  uint32_t* state;         // parity of the next launch's region, extents of regions 0 and 1
  uint32_t* parts;         // two regions of kGemvPartWords: partials as fp32 bits
  const uint16_t* lora_x;
  int ld_lora_x;
  const void* lora_a;      // [rank, K]
};

__host__ __device__ inline int gemv_part_floats(int TS, int nseg, int M) { return TS * nseg * M * 16; }

// Dynamic LDS of the GEMV (bytes): segment partials [TS][nseg][M][16], the
// waves' scale slices [16][64][16 bytes] (gathered absmax), the waves'
// activation slices [16][M][256] (16-bit), RND(B) of the tiles' rows
// [TS * 16][64] (16-bit), RND(bias) [TS * 16], RND(u) [M][64] (fp32).
constexpr int kGemvScaleSliceBytes = 64 * 16;
__host__ __device__ inline size_t gemv_lds_bytes(int TS, int nseg, int M, bool gather, bool xslice, bool lora) {
  size_t b = size_t(gemv_part_floats(TS, nseg, M)) * 4;
  if (gather) b += size_t(kGemvWaves) * kGemvScaleSliceBytes;
  if (xslice) b += size_t(kGemvWaves) * M * kSegK * 2;
  b += (lora ? size_t(TS) * 16 * kGemvBPitch * 2 : 0) + size_t(TS) * 16 * 4;
  b += lora ? size_t(M) * kGemvUPitch * 4 : 0;
  return b;
}

__device__ __forceinline__ uint32_t buf_load4_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return uint32_t(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kCoherent));
}
__device__ __forceinline__ uint32_t buf_load1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return uint32_t(__builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0));
}
// One element of a runtime float dtype (fp32 or 16-bit) as raw bits: both
// widths are issued, the unused one out of range, so that no load sits under
// a branch; elem_to_f32 picks and converts at the point of use.
struct RawElem {
  uint32_t w4, w2;
};
__device__ __forceinline__ RawElem buf_load_elem(__amdgpu_buffer_rsrc_t r, uint32_t idx, bool live, int dt) {
  const bool f32 = dt == RQ_DTYPE_F32;
  RawElem v;
  v.w4 = buf_load4(r, live && f32 ? idx * 4u : kOobOffset);
  v.w2 = buf_load2(r, live && !f32 ? idx * 2u : kOobOffset);
  return v;
}
__device__ __forceinline__ float elem_to_f32(const RawElem& v, int dt) {
  return dt == RQ_DTYPE_F32 ? u2f(v.w4) : (dt == RQ_DTYPE_BF16 ? bf16_to_f32(uint16_t(v.w2)) : f16_to_f32(uint16_t(v.w2)));
}

// Per-unit scale loads through buffer resources: the scales of the blocks
// holding k1 (steps 0-3) and k2 = k1 + 128 (steps 4-7) of the lane's row,
// given as block indices b1 and b2 (a past-the-end index reads zero).
template <class Scale>
struct GemvScale;

// Absmax scales are gathered once per wave: lane (u, r) = (l / 16, l % 16)
// loads the scales of row r of unit u's tile for unit u's segment (at most
// four blocks: 16 bytes of fp32, 8 of 16-bit values) and the wave puts them
// through its own LDS slice; unit u's lanes then read their two blocks there.
template <int SDT>
struct GemvScale<ScaleAbsmax<SDT>> {
  static constexpr bool kGather = true;
  static constexpr uint32_t kBytes = SDT == RQ_DTYPE_F32 ? 4u : 2u;
  struct Pair {};
  __amdgpu_buffer_rsrc_t r;
  __device__ GemvScale(const ScaleAbsmax<SDT>& s, uint32_t nblocks) { r = buffer_rsrc(s.p, nblocks * kBytes); }
  // the four blocks from block b on (a past-the-end b reads zeros)
  __device__ __forceinline__ u32x4 gather(uint32_t b) const {
    if constexpr (SDT == RQ_DTYPE_F32) return buf_load16(r, b * 4u);
    else {
      const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, b * 2u, 0, 0));
      return u32x4{v.x, v.y, 0u, 0u};
    }
  }
  // block c (0..3) of a gathered row
  __device__ __forceinline__ float value(const uint32_t* row, uint32_t c) const {
    if constexpr (SDT == RQ_DTYPE_F32) return u2f(row[c]);
    else {
      const uint16_t h = reinterpret_cast<const uint16_t*>(row)[c];
      if constexpr (SDT == RQ_DTYPE_BF16) return bf16_to_f32(h);
      else return f16_to_f32(h);
    }
  }
  __device__ __forceinline__ Pair load(uint32_t, uint32_t) const { return Pair{}; }
  __device__ __forceinline__ void hold(const Pair&) const {}
  __device__ __forceinline__ float v1(const Pair&) const { return 0.0f; }
  __device__ __forceinline__ float v2(const Pair&) const { return 0.0f; }
};

template <int SDT>
struct GemvScale<ScaleDQ<SDT>> {
  static constexpr bool kGather = false;
  struct Raw {
    uint32_t code, hi;
  };
  struct Pair {
    Raw s1, s2;
  };
  __amdgpu_buffer_rsrc_t rc, rs;
  int fmt, sh;
  uint32_t bs2;
  __device__ GemvScale(const ScaleDQ<SDT>& s, uint32_t nblocks) {
    rc = buffer_rsrc(s.c2, nblocks);
    const uint32_t ngroups = s.bs2_shift >= 0 ? ((nblocks + (1u << s.bs2_shift) - 1u) >> s.bs2_shift)
                                              : uint32_t((int64_t(nblocks) + s.bs2 - 1) / s.bs2);
    rs = buffer_rsrc(s.c2s, ngroups * (SDT == RQ_DTYPE_F32 ? 4u : 2u));
    fmt = s.fmt;
    sh = s.bs2_shift;
    bs2 = uint32_t(s.bs2);
  }
  __device__ __forceinline__ Raw load1(uint32_t b) const {
    // a missing unit's block (from kDeadBlock on) reads code 0 and scale 0
    const uint32_t g = b >= 0x20000000u ? b : (sh >= 0 ? (b >> sh) : b / bs2);
    Raw v;
    v.code = buf_load1(rc, b);
    if constexpr (SDT == RQ_DTYPE_F32) v.hi = buf_load4(rs, g * 4u);
    else v.hi = buf_load2(rs, g * 2u);
    return v;
  }
  __device__ __forceinline__ Pair load(uint32_t b1, uint32_t b2) const { return Pair{load1(b1), load1(b2)}; }
  __device__ __forceinline__ float value(const Raw& v) const {
    float hi;
    if constexpr (SDT == RQ_DTYPE_F32) hi = u2f(v.hi);
    else if constexpr (SDT == RQ_DTYPE_BF16) hi = bf16_to_f32(uint16_t(v.hi));
    else hi = f16_to_f32(uint16_t(v.hi));
    const uint8_t c = uint8_t(v.code);
    const float lo = fmt == RQ_C2_FP8_E4M3FNUZ ? fnuz_to_f32(c) : __fdiv_rn(float(int8_t(c)), 127.0f);
    return __fmul_rn(lo, hi);
  }
  __device__ __forceinline__ float v1(const Pair& p) const { return value(p.s1); }
  __device__ __forceinline__ float v2(const Pair& p) const { return value(p.s2); }
  __device__ __forceinline__ void hold(const Pair&) const {}
};

// One unit's loads for one lane: loads A and B (raw code bits) and the
// scales of steps 0-3 and 4-7.
template <class Scale>
struct GemvUnit {
  u32x4 xc;  // activation chunk (slice mode)
  u32x4 a, b;
  typename GemvScale<Scale>::Pair sp;
};

// Per-lane constants of the unit loads.
struct GemvLane {
  int n16, q;
  uint32_t offA, offB;   // byte offsets of loads A / B within a tile's rows, segment 0
  uint32_t sb1, sb2;     // scale block offsets of k1 / k2 from the tile's first block row, segment 0
  uint32_t c1, c2;       // block of k1 / k2 among a segment's (gathered) blocks
  uint32_t xoff;         // byte offset of the lane's activation chunk, segment 0 (slice mode)
  uint32_t xk;           // k of that chunk within a segment
};

// Wave-uniform bases that put every lane offset past the end of its buffer,
// so the loads of a missing unit read zeros without a per-lane select: a
// byte offset base (buffers here stay under 2^31 bytes) and a scale block
// index base (times 4 bytes still 2^31, with no wrap; scale arrays stay under
// 2^28 bytes since the packed weights stay under 2^31).
constexpr uint32_t kDeadBase = 0x80000000u;
constexpr uint32_t kDeadBlock = 0x20000000u;

template <int XM, class Scale>
__device__ __forceinline__ void gemv_issue(GemvUnit<Scale>& U, const GemvArgs& a, const GemvScale<Scale>& sc,
                                           __amdgpu_buffer_rsrc_t wres, __amdgpu_buffer_rsrc_t xres,
                                           const GemvLane& ln, uint32_t tile, uint32_t seg, bool live) {
  if constexpr (XM == 1) {
    // lane c: row c / 32, k = seg * 256 + 8 (c % 32); issued first, so that
    // waiting for it never waits for the weights.  A row past M reads past
    // the end of x; a k past K (a last, partial segment) must not read the
    // next row.
    const bool kin = seg * kSegK + ln.xk < uint32_t(a.K);
    const uint32_t xb = live ? seg * (kSegK * 2u) : kDeadBase;
    U.xc = buf_load16(xres, kin ? xb + ln.xoff : kDeadBase);
  }
  const uint32_t half_k = uint32_t(a.K) >> 1;
  const uint32_t wb = live ? tile * 16u * half_k + seg * (kSegK / 2) : kDeadBase;
  U.a = buf_load16(wres, wb + ln.offA);
  U.b = buf_load16(wres, wb + ln.offB);
  // scale block of k = seg * 256 + c (c < 256): (seg * 256 + c) >> bs_log2
  const uint32_t sseg = a.bs_log2 <= 8 ? (seg << (8 - a.bs_log2)) : (seg >> (a.bs_log2 - 8));
  if constexpr (!GemvScale<Scale>::kGather) {
    const uint32_t sb = live ? tile * 16u * uint32_t(a.bpr) + sseg : kDeadBlock;
    U.sp = sc.load(sb + ln.sb1, sb + ln.sb2);
  }
}

template <int XT, class Scale>
__device__ __forceinline__ f32x4 gemv_tile(const GemvUnit<Scale>& U, float s1, float s2, const u32x4 (&xa)[8],
                                           const u32x2* lut, uint32_t lane_off) {
  const u32x4 X1 = U.a, X2 = U.b;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  acc = mfma16x16x32<XT>(xa[0], expand8_scaled<XT>(lut, X1.x, lane_off, s1), acc);
  acc = mfma16x16x32<XT>(xa[1], expand8_scaled<XT>(lut, X1.y, lane_off, s1), acc);
  acc = mfma16x16x32<XT>(xa[2], expand8_scaled<XT>(lut, X1.z, lane_off, s1), acc);
  acc = mfma16x16x32<XT>(xa[3], expand8_scaled<XT>(lut, X1.w, lane_off, s1), acc);
  acc = mfma16x16x32<XT>(xa[4], expand8_scaled<XT>(lut, X2.x, lane_off, s2), acc);
  acc = mfma16x16x32<XT>(xa[5], expand8_scaled<XT>(lut, X2.y, lane_off, s2), acc);
  acc = mfma16x16x32<XT>(xa[6], expand8_scaled<XT>(lut, X2.z, lane_off, s2), acc);
  acc = mfma16x16x32<XT>(xa[7], expand8_scaled<XT>(lut, X2.w, lane_off, s2), acc);
  return acc;
}

// Workgroup barrier for LDS only: this wave's LDS accesses are complete,
// then s_barrier.  (__syncthreads() may also wait for every outstanding
// global load, which would serialize the prefetched units.)
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// How long (microseconds of the device's constant-rate real-time counter,
// s_memrealtime) a workgroup polls for the LoRA partials before it gives up
// waiting for the other workgroups' jobs and computes u itself.  A job runs
// before its wave's units and never waits, so every job ends once its
// workgroup has been dispatched (a few microseconds into the launch); the
// bound keeps the wait finite when the device is shared with other work (a
// workgroup still waiting for a compute unit).  A workgroup thus waits at
// most this long plus one poll's round trip, and then runs every job itself.
constexpr uint32_t kGemvDefaultWaitUs = 40;

// In-launch LoRA down-projection jobs: one wave computes the 16 x 16 fp32
// sums x[m, k] RND(A[16 p + jj, k]) (tokens m < 16, ranks 16 p + jj) over the
// 32-k steps [s0, s1) of its K split with one MFMA accumulation in step
// order, loading kJobChunk steps at once.
constexpr int kJobChunk = 4;
// Partials one thread of the epilogue sums: the 16 splits [16 c, 16 c + 16)
// of one (m, j); the C = 2^i threads of one (m, j) are adjacent lanes.
constexpr int kUPerThread = 16;
constexpr int kJobMaxC = 8;

struct JobChunk {
  u32x4 x[kJobChunk], a0[kJobChunk], a1[kJobChunk];
};

// Rank group and step range of wave job b of `ns` K splits per group.
__device__ __forceinline__ void job_range(int K, int ns, int b, int& p, uint32_t& s0, uint32_t& s1) {
  p = b / ns;
  const uint32_t s = uint32_t(b - p * ns), nsteps = uint32_t(K) / 32u;
  s0 = nsteps * s / uint32_t(ns);
  s1 = nsteps * (s + 1u) / uint32_t(ns);
}

// The operands of steps [b0, b0 + kJobChunk) of rank group p: lane (i16, q)
// takes x[i16, k .. k + 7] and A[16 p + i16, k .. k + 7], k = 32 step + 8 q
// (fp32 A as two 16-byte pieces); steps from s1 on, tokens past M and ranks
// past rank read zeros.
template <int XT>
__device__ __forceinline__ void job_issue(JobChunk& c, const GemvArgs& a, const LinearEpi& e, int p, uint32_t b0,
                                          uint32_t s1, int lane) {
  const int i16 = lane & 15, q = lane >> 4;
  const uint32_t K = uint32_t(a.K);
  const bool f32 = e.lora_dt == RQ_DTYPE_F32;
  const uint32_t ab = f32 ? 4u : 2u;
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.lora_x, uint32_t(a.M - 1) * uint32_t(a.ld_lora_x) * 2u + K * 2u);
  const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(a.lora_a, uint32_t(e.rank) * K * ab);
  const bool mlive = i16 < a.M;
  const uint32_t j = uint32_t(16 * p + i16);
  const bool jlive = j < uint32_t(e.rank);
  const uint32_t xrow = uint32_t(i16) * uint32_t(a.ld_lora_x) * 2u, arow = j * K * ab;
#pragma unroll
  for (int t = 0; t < kJobChunk; ++t) {
    const bool live = b0 + uint32_t(t) < s1;
    const uint32_t k = 32u * (b0 + uint32_t(t)) + 8u * uint32_t(q);
    c.x[t] = buf_load16(xr, live && mlive ? xrow + 2u * k : kOobOffset);
    c.a0[t] = buf_load16(ar, live && jlive ? arow + ab * k : kOobOffset);
    c.a1[t] = buf_load16(ar, live && jlive && f32 ? arow + 4u * k + 16u : kOobOffset);
  }
}

// Steps [b0, min(b0 + kJobChunk, s1)) of a job into acc, in step order; A is
// rounded to the activation dtype first (lora_layer.py:67's
// A.to(x.dtype)).  acc[r] of lane (i16, q) is (m, jj) = (4 q + r, i16).
template <int XT>
__device__ __forceinline__ f32x4 job_mfma(const JobChunk& c, f32x4 acc, uint32_t b0, uint32_t s1, bool f32) {
#pragma unroll
  for (int t = 0; t < kJobChunk; ++t) {
    if (b0 + uint32_t(t) < s1) {
      const u32x4 bop = f32 ? u32x4{cvt_pk<XT>(u2f(c.a0[t].x), u2f(c.a0[t].y)), cvt_pk<XT>(u2f(c.a0[t].z), u2f(c.a0[t].w)),
                                    cvt_pk<XT>(u2f(c.a1[t].x), u2f(c.a1[t].y)), cvt_pk<XT>(u2f(c.a1[t].z), u2f(c.a1[t].w))}
                            : c.a0[t];
      acc = mfma16x16x32<XT>(c.x[t], bop, acc);
    }
  }
  return acc;
}

// A whole job whose first chunk (steps from s0) is already in c.
template <int XT>
__device__ __forceinline__ f32x4 job_finish(JobChunk& c, const GemvArgs& a, const LinearEpi& e, int p, uint32_t s0,
                                            uint32_t s1, int lane) {
  const bool f32 = e.lora_dt == RQ_DTYPE_F32;
  f32x4 acc = job_mfma<XT>(c, f32x4{0.f, 0.f, 0.f, 0.f}, s0, s1, f32);
  for (uint32_t b0 = s0 + kJobChunk; b0 < s1; b0 += kJobChunk) {
    job_issue<XT>(c, a, e, p, b0, s1, lane);
    acc = job_mfma<XT>(c, acc, b0, s1, f32);
  }
  return acc;
}

// One LoRA down-projection job of lora_u_jobs_kernel: the fp32 partial sums
// x[m, k] RND(A[16 p + jj, k]) over the k of split s of `splits` (32-k steps
// [S s / splits, S (s + 1) / splits)), the steps dealt to the 16 waves in
// contiguous runs, four in flight at once, then the wave partials summed in
// wave order through `red` (16 KiB of LDS).  Returns the sum for (m, jj) =
// (tid / 16, tid % 16) in threads tid < 16 M.  Ends with red read: the
// caller synchronizes before red is written again.
template <int XT>
__device__ __forceinline__ float lora_u_job(const GemvArgs& a, const LinearEpi& e, int p, int s, int splits, int tid,
                                            int wave, float* red) {
  const int lane = tid & 63, i16 = lane & 15, q = lane >> 4;
  const int M = a.M, rank = e.rank;
  const uint32_t K = uint32_t(a.K), nsteps = K / 32u;
  const uint32_t j0 = nsteps * uint32_t(s) / uint32_t(splits), j1 = nsteps * uint32_t(s + 1) / uint32_t(splits);
  const uint32_t s0 = j0 + (j1 - j0) * uint32_t(wave) / 16u, s1 = j0 + (j1 - j0) * uint32_t(wave + 1) / 16u;
  const bool mlive = i16 < M;
  const uint32_t j = uint32_t(16 * p + i16);
  const bool jlive = j < uint32_t(rank);
  const bool f32 = e.lora_dt == RQ_DTYPE_F32;
  const uint32_t ab = f32 ? 4u : 2u;
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.lora_x, uint32_t(M - 1) * uint32_t(a.ld_lora_x) * 2u + K * 2u);
  const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(a.lora_a, uint32_t(rank) * K * ab);
  const uint32_t xrow = uint32_t(i16) * uint32_t(a.ld_lora_x) * 2u, arow = j * K * ab;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (uint32_t b0 = s0; b0 < s1; b0 += 4) {
    u32x4 xv[4], a0[4], a1[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const bool live = b0 + uint32_t(t) < s1;
      const uint32_t k = 32u * (b0 + uint32_t(t)) + 8u * uint32_t(q);
      xv[t] = buf_load16(xr, live && mlive ? xrow + 2u * k : kOobOffset);
      // fp32 A: two 16-byte pieces of 4 values; 16-bit A: one piece of 8
      a0[t] = buf_load16(ar, live && jlive ? arow + ab * k : kOobOffset);
      a1[t] = buf_load16(ar, live && jlive && f32 ? arow + 4u * k + 16u : kOobOffset);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // RND(A) in the activation dtype (lora_layer.py:67's A.to(x.dtype))
      const u32x4 bop = f32 ? u32x4{cvt_pk<XT>(u2f(a0[t].x), u2f(a0[t].y)), cvt_pk<XT>(u2f(a0[t].z), u2f(a0[t].w)),
                                    cvt_pk<XT>(u2f(a1[t].x), u2f(a1[t].y)), cvt_pk<XT>(u2f(a1[t].z), u2f(a1[t].w))}
                            : a0[t];
      acc = mfma16x16x32<XT>(xv[t], bop, acc);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * q + r;
    if (m < M) red[(wave * 16 + m) * 16 + i16] = acc[r];
  }
  lds_barrier();
  float v = 0.0f;
  if (tid < M * 16) {
#pragma unroll
    for (int w = 0; w < kGemvWaves; ++w) v = __fadd_rn(v, red[w * 256 + tid]);
  }
  return v;
}

template <int XT, class Scale, int U, int XM>
__global__ __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void nf4_gemv_kernel(GemvArgs a, Scale scale_src, LinearEpi e) {
  // The table is the kernel's only static LDS array, so it sits at address
  // 0 and every lookup's base folds into the instruction's offset field.
  __shared__ u32x2 lut[kGemvLutQwords];
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int M = a.M, TS = a.TS, nseg = a.nseg;
  const bool fused = a.jobs > 0;
  const uint32_t g = blockIdx.x, G = gridDim.x;  // this workgroup, their number
  const bool fold = !a.direct && a.tile_cnt != nullptr;  // K splits finished in this launch
  const bool epi = a.direct || fold;                     // the epilogue runs in this launch
  const int rank = (epi && e.rank > 0) ? e.rank : 0;     // LoRA staging only when fused here
  constexpr int RPB = kGemvBPitch, RPU = kGemvUPitch;      // staging pitches
  constexpr bool kGather = GemvScale<Scale>::kGather;
  float* part = reinterpret_cast<float*>(smem);
  // this wave's scale slice [64][4] (gathered absmax)
  uint32_t* gs = reinterpret_cast<uint32_t*>(part + gemv_part_floats(TS, nseg, M)) + wave * (kGemvScaleSliceBytes / 4);
  uint16_t* xs0 = reinterpret_cast<uint16_t*>(reinterpret_cast<uint32_t*>(part + gemv_part_floats(TS, nseg, M)) +
                                              (kGather ? kGemvWaves * (kGemvScaleSliceBytes / 4) : 0));
  // this wave's activation slice [M][256] (slice mode)
  uint16_t* xs = xs0 + wave * M * kSegK;
  // RND(B) rows of the tiles, as activation-dtype bits (exact: RND is the
  // rounding to that dtype)
  uint16_t* lbs = xs0 + (XM == 1 ? kGemvWaves * M * kSegK : 0);
  float* bss = reinterpret_cast<float*>(lbs + (rank > 0 ? TS * 16 * RPB : 0));
  float* us = bss + TS * 16;
  uint32_t* flag = reinterpret_cast<uint32_t*>(us + M * RPU);  // in-launch LoRA: set when u is computed here

  GemvLane ln;
  ln.n16 = lane & 15;
  ln.q = lane >> 4;
  {
    const uint32_t half_k = uint32_t(a.K) >> 1;
    ln.offA = uint32_t(ln.n16) * half_k + 16u * uint32_t(ln.q);
    ln.offB = uint32_t(ln.n16) * half_k + 16u * (uint32_t(ln.q) + 4u);
    // block offsets of k1 = 32 q and k2 = 128 + 32 q within a segment (zero
    // when a block spans whole segments), from the tile's first row
    const uint32_t rowb = uint32_t(ln.n16) * uint32_t(a.bpr);
    ln.sb1 = rowb + (a.bs_log2 <= 8 ? (32u * uint32_t(ln.q)) >> a.bs_log2 : 0u);
    ln.sb2 = rowb + (a.bs_log2 <= 8 ? (128u + 32u * uint32_t(ln.q)) >> a.bs_log2 : 0u);
    ln.c1 = a.bs_log2 <= 8 ? (32u * uint32_t(ln.q)) >> a.bs_log2 : 0u;
    ln.c2 = a.bs_log2 <= 8 ? (128u + 32u * uint32_t(ln.q)) >> a.bs_log2 : 0u;
    const uint32_t c = uint32_t(lane);
    ln.xk = 8u * (c & 31u);
    ln.xoff = ((c >> 5) * uint32_t(a.ldx) + ln.xk) * 2u;
  }
  const uint32_t seg0 = blockIdx.y * uint32_t(nseg);  // first segment of this K split
  const uint32_t n_tiles = uint32_t((a.N + 15) / 16);
  // tiles g, g + G, ...: at any moment the workgroups' loads are spread over
  // the whole weight matrix
  auto tile_of = [&](int t) -> uint32_t { return g + uint32_t(t) * G; };
  const __amdgpu_buffer_rsrc_t wres = buffer_rsrc(a.packed, uint32_t(a.N) * (uint32_t(a.K) >> 1));
  const GemvScale<Scale> sc(scale_src, uint32_t(a.N) * uint32_t(a.bpr));
  // this wave's units (tile slot, segment), wave-uniform scalars computed
  // here rather than read from a table in the arguments: a wave-indexed
  // argument load is a second round trip to the argument memory before the
  // first weight load can be addressed.  With the activation slices unit u
  // of wave w is unit i = w + 16 u of the workgroup's TS * nseg (tile i /
  // nseg, segment i % nseg); without them the R = 16 / nseg wave groups take
  // the tiles round-robin, wave w segment w % nseg of tiles w / nseg + R u.
  // A missing unit reads tile slot 0, segment 0 (its loads are dead).
  int ut[U], useg[U];
  bool ulive[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if constexpr (XM == 1) {
      const int i = wave + kGemvWaves * u;
      ulive[u] = i < TS * nseg;
      ut[u] = ulive[u] ? i / nseg : 0;
      useg[u] = ulive[u] ? i - ut[u] * nseg : 0;
    } else {
      const int R = kGemvWaves / nseg;
      const int t = wave / nseg + u * R;
      ulive[u] = wave < R * nseg && t < TS;
      ut[u] = ulive[u] ? t : 0;
      useg[u] = ulive[u] ? wave - (wave / nseg) * nseg : 0;
    }
  }
  const __amdgpu_buffer_rsrc_t xres =
      buffer_rsrc(a.x, uint32_t(M - 1) * uint32_t(a.ldx) * 2u + uint32_t(a.K) * 2u);
  // units in flight ahead of the one being computed (two measured slower:
  // the extra bytes in flight only lengthened the loaded latency)
  constexpr int D = 1;
  GemvUnit<Scale> L[U];
  // without the slices (M > 2) the first unit's weights go out before
  // anything else (0.4-1 us faster per launch at M = 4-16 than after the
  // LoRA and scale loads); with them the activations and weights go out
  // after those loads (weights first measured 0.5-0.9 us slower at M = 1)
  if constexpr (XM == 0) {
#pragma unroll
    for (int u = 0; u < D; ++u)
      gemv_issue<XM>(L[u], a, sc, wres, xres, ln, tile_of(ut[u]), seg0 + uint32_t(useg[u]), ulive[u]);
  }

  // 1. the first unit's loads; without the slice, this wave's own
  //    activation operands (its units share one segment): step c covers k =
  //    seg * 256 + 128 (c / 4) + 32 q + 8 (c % 4) of token n16; a token past M
  //    or a k past K reads zeros
  // this wave's LoRA down-projection job, if any: its first chunk's loads go
  // out before the unit loads, so that waiting for them never waits for the
  // weights
  const int ns = e.u_splits;
  // jobs go to the waves with the fewest units: the last waves when some
  // waves have one unit fewer (or none), else from wave 1 on, so that wave
  // 0, which polls the partials, reaches its poll as early as it can (the
  // oldest wave of a SIMD finishes its units first)
  const bool light_top = XM == 1 ? (TS * nseg) % kGemvWaves != 0 : (kGemvWaves / nseg) * nseg < kGemvWaves;
  // (workgroups counted over the K splits too: G columns per split)
  const int job = (light_top ? kGemvWaves - 1 - wave : (wave + kGemvWaves - 1) % kGemvWaves) * int(G * gridDim.y) +
                  int(blockIdx.y * G + g);
  const bool has_job = fused && job < a.jobs;
  // this launch's partial region and the other region's extent, loaded by
  // wave 0 (which passes the parity on through LDS) and the job waves (the
  // state and job loads are a wave's first loads, so waiting for them never
  // waits for another; one state load per workgroup keeps the line cool)
  u32x4 st = u32x4{0u, 0u, 0u, 0u};
  if (fused && (wave == 0 || has_job)) st = buf_load16_coherent(buffer_rsrc(a.state, 16u), 0u);
  const uint32_t par = st.x & 1u;
  JobChunk jch;
  int jp = 0;
  uint32_t js0 = 0u, js1 = 0u;
  if (has_job) {
    job_range(a.K, ns, job, jp, js0, js1);
    job_issue<XT>(jch, a, e, jp, js0, js1, lane);
  }
  // the gathered scales first: lane (u, r) = (lane / 16, lane % 16) takes
  // row r of unit u's tile, from unit u's segment's first block on
  u32x4 gsv = u32x4{0u, 0u, 0u, 0u};
  if constexpr (kGather) {
    const int gu = lane >> 4;
    int gt = ut[0], gseg = useg[0];
    bool glive = ulive[0];
#pragma unroll
    for (int u = 1; u < U; ++u)
      if (gu == u) {
        gt = ut[u];
        gseg = useg[u];
        glive = ulive[u];
      }
    const uint32_t sg = seg0 + uint32_t(gseg);
    const uint32_t first = a.bs_log2 <= 8 ? (sg << (8 - a.bs_log2)) : (sg >> (a.bs_log2 - 8));
    const uint32_t blk = (tile_of(gt) * 16u + uint32_t(ln.n16)) * uint32_t(a.bpr) + first;
    gsv = sc.gather(glive && gu < U ? blk : kDeadBlock);
  }
  if constexpr (XM == 1) {
#pragma unroll
    for (int u = 0; u < D; ++u)
      gemv_issue<XM>(L[u], a, sc, wres, xres, ln, tile_of(ut[u]), seg0 + uint32_t(useg[u]), ulive[u]);
  }
  u32x4 xa[8];
  if constexpr (XM == 0) {
    const uint32_t sg = seg0 + uint32_t(useg[0]);
    const bool mlive = ln.n16 < M && ulive[0];
    if (a.xvec) {
      const uint32_t xrow = uint32_t(ln.n16) * uint32_t(a.ldx) * 2u;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t k = sg * kSegK + 128u * (c >> 2) + 32u * uint32_t(ln.q) + 8u * (c & 3);
        xa[c] = buf_load16(xres, (mlive && k < uint32_t(a.K)) ? xrow + 2u * k : kOobOffset);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t k = sg * kSegK + 128u * (c >> 2) + 32u * uint32_t(ln.q) + 8u * (c & 3);
        const bool live = mlive && k < uint32_t(a.K);
        const uint32_t base = (uint32_t(ln.n16 < M ? ln.n16 : 0) * uint32_t(a.ldx) + (live ? k : 0u)) * 2u;
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 4; ++h)
          w[h] = buf_load2(xres, live ? base + 4u * h : kOobOffset) |
                 (buf_load2(xres, live ? base + 4u * h + 2u : kOobOffset) << 16);
        xa[c] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
  }

  // 2. the table; then this wave's job, if any (its unit loads stay in
  //    flight): partials to the region with device-coherent stores, then the
  //    job counts itself; the last one readies the next launch's region
  fill_f32pair_lut<kGemvThreads>(lut, tid);
  if (fused && tid == 0) flag[1] = par;
  lds_barrier();
  uint32_t jc_old = 0u;
  if (has_job) {
    const f32x4 acc = job_finish<XT>(jch, a, e, jp, js0, js1, lane);
    const int s = job - jp * ns, jj = 16 * jp + ln.n16;
    uint32_t* region = a.parts + par * uint32_t(kGemvPartWords);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * ln.q + r;
      if (m < M && jj < e.rank) {
        const uint32_t bits = f2u(acc[r]);
        __hip_atomic_store(&region[(s * M + m) * e.rank + jj], bits != 0u ? bits : 0x80000000u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // the count, its result awaited at the wave's end (an increment: the
    // compiler's atomic optimizer rewrites fetch_add into a form that waits
    // for the result at once)
    if (lane == 0) jc_old = __builtin_amdgcn_atomic_inc32(a.jc, 0xFFFFFFFFu, __ATOMIC_RELAXED, "agent");
  }
  if (fused && tid == 0) *flag = 0u;

  // 3. epilogue operands, raw: LoRA B values (value t of thread tid is row
  //    tid / 64 of tile slot t, rank tid % 64), the bias, the RND(u)
  //    partials: thread tid < M rank C (C = 2^i >= u_splits / 16) takes
  //    splits [16 c, 16 c + 16) of pr = (m, j) = (pr / rank, pr % rank),
  //    pr = tid / C, c = tid % C
  RawElem br = RawElem{0u, 0u};
  u32x4 bvr = u32x4{0u, 0u, 0u, 0u};
  uint32_t up[kUPerThread];
#pragma unroll
  for (int k = 0; k < kUPerThread; ++k) up[k] = 0u;
  int uC = 1;
  while (kUPerThread * uC < ns) uC <<= 1;
  const int upr = tid / uC, uc = tid - upr * uC;
  const bool u_mine = rank > 0 && upr < M * rank;
  const uint32_t ustride = uint32_t(M) * uint32_t(rank);
  // split 16 c + k of this thread's (m, j), or split 0 when past ns (read,
  // never summed)
  auto u_index = [&](int k) -> uint32_t {
    return (kUPerThread * uc + k < ns ? uint32_t(kUPerThread * uc + k) : 0u) * ustride + uint32_t(upr);
  };
  const uint32_t bbytes = e.lora_dt == RQ_DTYPE_F32 ? 4u : 2u;
  // LoRA B rows as 16-byte chunks (the host fuses LoRA only for such rows):
  // thread et < TS * 16 * 2^cl takes chunk et % 2^cl of row (et >> cl) % 16
  // of tile slot et >> (4 + cl), and the bias loads go to wave ew = 0, where
  // et and ew count threads and waves from the last when every wave has one
  // unit (so that wave 0, which polls the partials, has no epilogue loads
  // ahead of its poll), else from the first
  const int cl = rank > 0 ? a.bvec_log2 : 0;
  const int et = U == 1 ? kGemvThreads - 1 - tid : tid, ew = U == 1 ? kGemvWaves - 1 - wave : wave;
  const int bt = et >> (4 + cl), br_row = (et >> cl) & 15, bc = et & ((1 << cl) - 1);
  const bool bvec_live = rank > 0 && et < (TS * 16 << cl);
  if (rank > 0 && ew * 64 < (TS * 16 << cl)) {
    const __amdgpu_buffer_rsrc_t bres = buffer_rsrc(e.lora_b, uint32_t(a.N) * uint32_t(e.ld_lora_b) * bbytes);
    const uint32_t bn = tile_of(bt) * 16u + uint32_t(br_row);
    const bool live = bvec_live && bn < uint32_t(a.N);
    bvr = buf_load16(bres, live ? bn * uint32_t(e.ld_lora_b) * bbytes + 16u * uint32_t(bc) : kOobOffset);
  }
  const bool has_bias = epi && e.bias != nullptr;
  if (has_bias && ew == 0) {
    const __amdgpu_buffer_rsrc_t bres = buffer_rsrc(e.bias, uint32_t(a.N) * (e.bias_dt == RQ_DTYPE_F32 ? 4u : 2u));
    const int cb = et & (kGemvMaxTS * 16 - 1);
    const uint32_t cn = tile_of(cb >> 4) * 16u + uint32_t(cb & 15);
    br = buf_load_elem(bres, cn, (cb >> 4) < TS && cn < uint32_t(a.N), e.bias_dt);
  }
  if (u_mine && !fused) {
    // the partials of a down-projection launched before this kernel
    const __amdgpu_buffer_rsrc_t ures = buffer_rsrc(e.u, uint32_t(ns) * ustride * 4u);
#pragma unroll
    for (int k = 0; k < kUPerThread; ++k) up[k] = buf_load4(ures, u_index(k) * 4u);
  }

  // 4. the units, each as soon as its loads have landed; partials to LDS
  const uint32_t lane_off = uint32_t(lane & 31) * 8u;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u + D < U)
      gemv_issue<XM>(L[u + D], a, sc, wres, xres, ln, tile_of(ut[u + D]), seg0 + uint32_t(useg[u + D]), ulive[u + D]);
    if constexpr (kGather) {
      if (u == 0) *reinterpret_cast<u32x4*>(gs + 4 * lane) = gsv;
    }
    if (ulive[u]) {
      if constexpr (XM == 1) {
        // the unit's activations through this wave's slice: lane c wrote
        // row c / 32, k 8 (c % 32); token n16 < M reads its MFMA operands.
        // The lanes of rows n16 >= M read row 0 instead of zeros: an MFMA
        // output row depends only on its own operand row, and rows >= M are
        // never stored (no branch, no zero fill).  A unit of the previous
        // unit's segment (every unit of a wave when K is 16 segments) keeps
        // the operands already in registers.
        if (u == 0 || !ulive[u - 1] || useg[u] != useg[u - 1]) {
          if (lane < 32 * M) *reinterpret_cast<u32x4*>(xs + 8 * lane) = L[u].xc;
          const uint16_t* xrow = xs + (ln.n16 < M ? ln.n16 : 0) * kSegK + 32 * ln.q;
#pragma unroll
          for (int c = 0; c < 8; ++c) xa[c] = *reinterpret_cast<const u32x4*>(xrow + 128 * (c >> 2) + 8 * (c & 3));
        }
      }
      float s1, s2;
      if constexpr (kGather) {
        const uint32_t* grow = gs + 4 * (16 * u + ln.n16);
        s1 = sc.value(grow, ln.c1);
        s2 = sc.value(grow, ln.c2);
      } else {
        sc.hold(L[u].sp);
        s1 = sc.v1(L[u].sp);
        s2 = sc.v2(L[u].sp);
      }
      const f32x4 acc = gemv_tile<XT>(L[u], s1, s2, xa, lut, lane_off);
      float* pp = part + (ut[u] * nseg + useg[u]) * M * 16 + ln.n16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * ln.q + r;
        if (m < M) pp[m * 16] = acc[r];
      }
    }
  }

  // 5. with the LoRA down-projection in this launch: the threads that take
  //    partials poll them (device-coherent loads) until none reads 0 -- a
  //    bounded poll -- and thread 0 counts the workgroup past its use of
  //    them.  A workgroup in which a poll gave up runs every job itself, the
  //    same way (the same sums), into the table's LDS, which the unit loop
  //    no longer reads, and takes the partials from there.
  uint32_t self_u = 0u;
  if (fused) {
    const uint32_t* region = a.parts + flag[1] * uint32_t(kGemvPartWords);
    if (u_mine) {
      bool ok = false;
      // device-coherent loads through a buffer resource: 32-bit offsets,
      // one address add per load
      const __amdgpu_buffer_rsrc_t rres = buffer_rsrc(region, uint32_t(kGemvPartBytes));
      auto poll = [&]() {
        // all the loads of a poll in flight together: no branch between
        // them (a split past ns reads the first again and is not checked)
#pragma unroll
        for (int k = 0; k < kUPerThread; ++k) up[k] = buf_load4_coherent(rres, u_index(k) * 4u);
        uint32_t missing = 0u;
#pragma unroll
        for (int k = 0; k < kUPerThread; ++k)
          missing |= uint32_t(up[k] == 0u) & uint32_t(kUPerThread * uc + k < ns);
        ok = missing == 0u;
      };
      if (a.wait_ticks > 0) {
        poll();
        // the clock starts only when the first poll finds a partial missing
        // (the common case, every partial there, reads no clock)
        if (!ok) {
          const uint32_t t0 = uint32_t(__builtin_amdgcn_s_memrealtime());
          do {
            __builtin_amdgcn_s_sleep(2);
            poll();
            // (unsigned difference: the counter's low word may wrap)
          } while (!ok && uint32_t(__builtin_amdgcn_s_memrealtime()) - t0 < a.wait_ticks);
        }
      }
      if (!ok) *flag = 1u;
    }
    lds_barrier();
    self_u = __builtin_amdgcn_readfirstlane(*flag);
    if (self_u) {
      float* pl = reinterpret_cast<float*>(lut);  // [u_splits][M][rank]
      for (int b = wave; b < a.jobs; b += kGemvWaves) {
        int p;
        uint32_t s0, s1;
        job_range(a.K, ns, b, p, s0, s1);
        JobChunk c;
        job_issue<XT>(c, a, e, p, s0, s1, lane);
        const f32x4 acc = job_finish<XT>(c, a, e, p, s0, s1, lane);
        const int sp = b - p * ns, jj = 16 * p + ln.n16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 4 * ln.q + r;
          if (m < M && jj < rank) pl[(sp * M + m) * rank + jj] = acc[r];
        }
      }
      lds_barrier();
      if (u_mine) {
#pragma unroll
        for (int k = 0; k < kUPerThread; ++k) up[k] = f2u(pl[u_index(k)]);
      }
    }
  }

  // 6. epilogue operands into LDS, then one thread per output (tile slot
  //    t = tid / 256, row m, column nn).  The empty asm marks the raw values
  //    as changed here, so that no use of them (which waits for its load)
  //    is scheduled into the unit loop above.
  asm volatile("" : "+v"(br.w4), "+v"(br.w2));
  asm volatile("" : "+v"(bvr));
#pragma unroll
  for (int k = 0; k < kUPerThread; ++k) asm volatile("" : "+v"(up[k]));
  if (bvec_live) {
    uint16_t* dst = lbs + (bt * 16 + br_row) * RPB + bc * int(16u / bbytes);
    if (e.lora_dt == RQ_DTYPE_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = uint16_t(to_x16<XT>(u2f(bvr[i])));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t lo = uint16_t(bvr[i]), hi = uint16_t(bvr[i] >> 16);
        dst[2 * i] = uint16_t(to_x16<XT>(e.lora_dt == RQ_DTYPE_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo)));
        dst[2 * i + 1] = uint16_t(to_x16<XT>(e.lora_dt == RQ_DTYPE_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi)));
      }
    }
  }
  if (epi && et < TS * 16) bss[et] = has_bias ? round_x<XT>(elem_to_f32(br, e.bias_dt)) : 0.0f;
  if (rank > 0) {
    // u[m, j]: each thread sums its 16 splits in order, then lane c = 0 of
    // the (m, j) adds the C threads' sums in c order (adjacent lanes of one
    // wave: C divides 64)
    float l1 = 0.0f;
    if (u_mine) {
#pragma unroll
      for (int k = 0; k < kUPerThread; ++k)
        if (kUPerThread * uc + k < ns) l1 = __fadd_rn(l1, u2f(up[k]));
    }
    float sum = l1;
    for (int c = 1; c < uC; ++c) sum = __fadd_rn(sum, __shfl(l1, lane + c));
    if (u_mine && uc == 0) us[(upr / rank) * RPU + (upr - (upr / rank) * rank)] = round_x<XT>(sum);
  }
  lds_barrier();

  // 7. the outputs (with K splits: this split's partials, and in the last
  //    split of the column to count itself, the outputs), then (in-launch
  //    LoRA) wave 0 learns whether this was the launch's last workgroup to
  //    count itself.  One thread per output: tile slot t = tid / 256, row m,
  //    column nn.
  const int ft = tid >> 8, fm = (tid >> 4) & 15, fnn = tid & 15;
  const uint32_t ftile = tile_of(ft);
  const int64_t fn = int64_t(ftile) * 16 + fnn;
  const bool fout = ft < TS && fm < M && ftile < n_tiles && fn < a.N;
  // bias, RND, the LoRA term, RND, store
  auto epilogue = [&](float v) {
    if (e.bias) v = __fadd_rn(v, bss[ft * 16 + fnn]);
    v = round_x<XT>(v);
    if (rank > 0) {
      const uint16_t* brow = lbs + (ft * 16 + fnn) * RPB;
      const float* urow = us + fm * RPU;
      float l = 0.0f;
      for (int j0 = 0; j0 < rank; j0 += 8) {
        float uu[8], bb[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          uu[jj] = urow[j0 + jj];
          bb[jj] = from_x16<XT>(brow[j0 + jj]);
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          if (j0 + jj < rank) l = __fmaf_rn(uu[jj], bb[jj], l);
      }
      l = round_x<XT>(__fmul_rn(round_x<XT>(l), e.scaling));
      v = round_x<XT>(__fadd_rn(v, l));
    }
    static_cast<uint16_t*>(e.y)[fm * e.ldy + fn] = uint16_t(to_x16<XT>(v));
  };
  if (fout) {
    // this workgroup's segments in order
    const float* pp = part + ft * nseg * M * 16 + fm * 16 + fnn;
    float v = 0.0f;
    int sgi = 0;
    for (; sgi + 8 <= nseg; sgi += 8) {
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = pp[(sgi + j) * M * 16];
#pragma unroll
      for (int j = 0; j < 8; ++j) v = __fadd_rn(v, p[j]);
    }
    for (; sgi < nseg; ++sgi) v = __fadd_rn(v, pp[sgi * M * 16]);
    if (a.direct) {
      epilogue(v);
    } else {
      float* dst = a.ws + (int64_t(blockIdx.y) * a.M + fm) * a.N + fn;
      // device-coherent when another workgroup sums it
      if (fold) __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else *dst = v;
    }
  }
  if (fold) {
    // every thread's partials written (the stores complete, device-wide),
    // then the column counts this split; the last one to count sums every
    // split's partials, in split order (the same sums whichever is last),
    // and resets the count for the next launch
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    uint32_t* last_flag = reinterpret_cast<uint32_t*>(lut);  // the table is no longer read
    if (tid == 0) {
      const uint32_t old = __hip_atomic_fetch_add(&a.tile_cnt[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old == gridDim.y - 1u;
      if (last) __hip_atomic_store(&a.tile_cnt[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *last_flag = last ? 1u : 0u;
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(*last_flag) && fout) {
      const int S = int(gridDim.y);
      const float* src = a.ws + int64_t(fm) * a.N + fn;
      const int64_t sstride = int64_t(a.M) * a.N;
      float v = 0.0f;
      for (int s0 = 0; s0 < S; s0 += 8) {
        // eight splits' partials in flight together (a split past S
        // re-reads the first and is not added)
        float p[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
          p[k] = __hip_atomic_load(src + (s0 + k < S ? s0 + k : 0) * sstride, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (s0 + k < S) v = __fadd_rn(v, p[k]);
      }
      epilogue(v);
    }
  }
  if (has_job && __builtin_amdgcn_readfirstlane(jc_old) == uint32_t(a.jobs) - 1u) {
    // the last job: clear the other region (the previous launch's partials,
    // whose readers have all finished), record this launch's extent in
    // region par, reset the count and flip the parity
    const uint32_t other_ext = par ? st.y : st.z;
    const __amdgpu_buffer_rsrc_t other =
        buffer_rsrc(a.parts + (par ^ 1u) * uint32_t(kGemvPartWords), uint32_t(kGemvPartBytes));
    for (uint32_t i = uint32_t(lane); 4u * i < other_ext; i += 64u)
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, other, 16u * i, 0, kCoherent);
    // the zeros are visible device-wide before the parity flips: a
    // workgroup of this launch that starts late reads the flipped parity
    // and must find the region it then polls cleared, not the previous
    // launch's partials.  The zeros are device-coherent (sc1) stores, which
    // write through the L2 and count as done only once written, so waiting
    // for every lane's stores orders them before the state stores; a
    // release fence would also write back the whole L2 (buffer_wbl2),
    // which no store here needs, for about 0.25 us per launch.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) {
      const uint32_t ext = uint32_t(ns) * uint32_t(M) * uint32_t(e.rank);
      __hip_atomic_store(&a.state[1u + par], ext, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.state[2u - par], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.jc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.state, par ^ 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Split-K finisher (and the LoRA epilogue for any M): y = finish(sum_s
// ws[s]).  One thread per output (row blockIdx.y, column n).  Every load a
// thread needs -- the bias, its splits' partials (up to 8), its LoRA B row
// (up to 16 ranks) and, in threads j < rank, the 16 first u partials of rank
// j -- is requested before any of them is used, so a launch costs about one
// memory round trip.  The sums keep their order: splits ascending, ranks
// ascending.
template <int XT>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(const float* __restrict__ ws, int S, int64_t M,
                                                              int64_t N, LinearEpi e) {
  extern __shared__ float us[];  // RND(u) of this row, [rank]
  const int64_t m = blockIdx.y;
  const int tid = threadIdx.x;
  const int64_t n0 = int64_t(blockIdx.x) * 256 + tid;
  const bool live = n0 < N;
  const int64_t n = live ? n0 : N - 1;  // a thread past N loads (and discards) the last column's operands
  const bool has_bias = e.bias != nullptr;
  const Raw16x2 br = load_raw(has_bias ? e.bias : ws, has_bias ? n : 0, has_bias ? e.bias_dt : RQ_DTYPE_F32);
  float p[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) p[k] = ws[(int64_t(k < S ? k : 0) * M + m) * N + n];
  const int rb = e.rank < 16 ? e.rank : 16;
  Raw16x2 b[16];
  if (rb > 0) {
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) b[jj] = load_raw(e.lora_b, n * e.ld_lora_b + (jj < rb ? jj : 0), e.lora_dt);
  }
  // u[m, j] for j = tid < rank: the u_splits partials in order, 16 requested at once
  if (tid < e.rank) {
    float q[16];
    float sum = 0.0f;
    for (int k0 = 0; k0 < e.u_splits; k0 += 16) {
#pragma unroll
      for (int k = 0; k < 16; ++k) q[k] = e.u[(int64_t(k0 + k < e.u_splits ? k0 + k : k0) * M + m) * e.rank + tid];
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (k0 + k < e.u_splits) sum = __fadd_rn(sum, q[k]);
    }
    us[tid] = round_x<XT>(sum);
  }
  __syncthreads();
  if (!live) return;
  float v = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < S) v = __fadd_rn(v, p[k]);
  for (int s0 = 8; s0 < S; s0 += 8) {
    float p2[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) p2[k] = (s0 + k < S) ? ws[(int64_t(s0 + k) * M + m) * N + n] : 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (s0 + k < S) v = __fadd_rn(v, p2[k]);
  }
  float lsum = 0.0f;
#pragma unroll
  for (int jj = 0; jj < 16; ++jj)
    if (jj < rb) lsum = __fmaf_rn(us[jj], round_x<XT>(raw_to_f32(b[jj], e.lora_dt)), lsum);
  for (int j0 = 16; j0 < e.rank; j0 += 8) {
    Raw16x2 b2[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      b2[jj] = load_raw(e.lora_b, n * e.ld_lora_b + (j0 + jj < e.rank ? j0 + jj : 0), e.lora_dt);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      if (j0 + jj < e.rank) lsum = __fmaf_rn(us[j0 + jj], round_x<XT>(raw_to_f32(b2[jj], e.lora_dt)), lsum);
  }
  if (has_bias) v = __fadd_rn(v, round_x<XT>(raw_to_f32(br, e.bias_dt)));
  v = round_x<XT>(v);
  if (e.rank > 0) {
    const float l = round_x<XT>(__fmul_rn(round_x<XT>(lsum), e.scaling));
    v = round_x<XT>(__fadd_rn(v, l));
  }
  static_cast<uint16_t*>(e.y)[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
}


// ---------------------------------------------------------------------------
// LoRA down-projection partials: up[ks, m, j] = sum_{k in split ks}
// xl[m, k] * RND(A[j, k]).  A (rank x K) is the trainable fp32 (or
// activation-dtype) parameter; it is rounded to the activation dtype on load,
// as lora_layer.py:67's `self.lora_A.to(x.dtype)` does.  Workgroup = (16 rows
// of xl, 16 rows of A, K split of at most 16 steps of 32 k); each of its 4
// waves loads its (at most 4) steps' operands at once, then runs the MFMAs,
// and the waves reduce through LDS.
// ---------------------------------------------------------------------------
constexpr int kLoraUStepsPerWave = 4;

template <int XT>
__global__ __launch_bounds__(256) void lora_u_kernel(const uint16_t* __restrict__ xl, int64_t ldxl, bool xvec,
                                                     const void* __restrict__ A, int a_dt, bool avec, int64_t M,
                                                     int64_t K, int rank, int KS, float* __restrict__ up) {
  __shared__ float red[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i16 = lane & 15, q = lane >> 4;
  const int64_t m = int64_t(blockIdx.x) * 16 + i16;
  const int64_t j = int64_t(blockIdx.y) * 16 + i16;
  const int ks = blockIdx.z;
  const int64_t nsteps = K / 32;
  const int64_t s0 = (nsteps * ks) / KS, s1 = (nsteps * (ks + 1)) / KS;
  const int64_t w0 = s0 + ((s1 - s0) * wave) / 4, w1 = s0 + ((s1 - s0) * (wave + 1)) / 4;
  const bool mlive = m < M, jlive = j < rank;
  f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t b0 = w0; b0 < w1; b0 += kLoraUStepsPerWave) {
    u32x4 av[kLoraUStepsPerWave], bv[kLoraUStepsPerWave];
#pragma unroll
    for (int t = 0; t < kLoraUStepsPerWave; ++t) {
      const int64_t k = 32 * (b0 + t) + 8 * q;
      const bool live = b0 + t < w1;
      if (live && mlive) {
        const uint16_t* p = xl + m * ldxl + k;
        if (xvec) {
          av[t] = *reinterpret_cast<const u32x4*>(p);
        } else {
          uint32_t w[4];
#pragma unroll
          for (int h = 0; h < 4; ++h) w[h] = uint32_t(p[2 * h]) | (uint32_t(p[2 * h + 1]) << 16);
          av[t] = u32x4{w[0], w[1], w[2], w[3]};
        }
      } else {
        av[t] = u32x4{0u, 0u, 0u, 0u};
      }
      bv[t] = load_a8<XT>(A, a_dt, j * K + k, live && jlive, avec);
    }
#pragma unroll
    for (int t = 0; t < kLoraUStepsPerWave; ++t) d = mfma16x16x32<XT>(av[t], bv[t], d);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][(4 * q + r) * 16 + i16] = d[r];
  __syncthreads();
  const int idx = threadIdx.x;  // 256 outputs: (row mm, col jj)
  const int mm = idx >> 4, jj = idx & 15;
  const int64_t om = int64_t(blockIdx.x) * 16 + mm, oj = int64_t(blockIdx.y) * 16 + jj;
  if (om < M && oj < rank) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) v = __fadd_rn(v, red[w][idx]);
    up[(int64_t(ks) * M + om) * rank + oj] = v;
  }
}

// The LoRA down-projection as a launch of its own, before a split-K GEMV or
// one with more workgroups than compute units: workgroup j runs job j of
// lora_u_job (ranks [16 (j / u_splits), +16), K split j % u_splits, its
// steps spread over the 16 waves) and stores its partials in the layout
// lora_u_kernel writes.
template <int XT>
__global__ __launch_bounds__(kGemvThreads) void lora_u_jobs_kernel(GemvArgs a, LinearEpi e, float* __restrict__ up) {
  __shared__ float red[kGemvWaves * 256];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = blockIdx.x, ns = e.u_splits;
  const float v = lora_u_job<XT>(a, e, j / ns, j % ns, ns, tid, wave, red);
  const int jj = 16 * (j / ns) + (tid & 15);
  if (tid < a.M * 16 && jj < e.rank) up[((j % ns) * a.M + (tid >> 4)) * e.rank + jj] = v;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// The wait bound of rq_set_gemv_wait_us (a test hook): an atomic, so that
// setting it from one host thread while another launches is defined.
static std::atomic<uint32_t> gemv_wait_us{kGemvDefaultWaitUs};

uint32_t set_gemv_wait_us(uint32_t us) { return gemv_wait_us.exchange(us, std::memory_order_relaxed); }

// Ticks of s_memrealtime per microsecond on the current device (the
// counter's rate is hipDeviceAttributeWallClockRate, in kHz), cached per
// device index.
static uint32_t realtime_ticks_per_us() {
  constexpr int kMaxDevices = 64;
  static std::atomic<uint32_t> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 100u;
  uint32_t t = cache[dev].load(std::memory_order_relaxed);
  if (t == 0u) {
    int khz = 0;
    t = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess && khz >= 1000
            ? uint32_t(khz / 1000)
            : 100u;
    cache[dev].store(t, std::memory_order_relaxed);
  }
  return t;
}

// Work plan of the GEMV: K splits, tiles per workgroup, units per wave, the
// unit table, the activation stage, and the workspace layout.
GemvPlan plan_gemv(int64_t M, int64_t N, int64_t K, int64_t rank, int cus, bool xvec, bool gather,
                   bool lora_vec, bool lora_prod) {
  GemvPlan p{};
  const int nsegs = int((K + kSegK - 1) / kSegK);
  const int64_t tiles = (N + 15) / 16;
  const int64_t ncu = cus > 0 ? cus : 1;
  p.u_splits = 0;
  // K splits of lora_u_jobs_kernel (the down-projection before a split-K
  // GEMV): about 256 k per workgroup job, so that a job's loads are one round
  // of 16-byte loads per wave
  const int fused_splits = int(std::min<int64_t>((K + 255) / 256, kGemvMaxUSplits));
  if (rank > 0) {
    const int64_t steps_per_wg = 4 * kLoraUStepsPerWave;
    const int64_t ks = (K / 32 + steps_per_wg - 1) / steps_per_wg;
    p.u_splits = lora_prod ? fused_splits : int(ks < kGemvMaxUSplits ? ks : kGemvMaxUSplits);
  }
  const int launched_splits = p.u_splits;  // of the down-projection launched before the GEMV
  const bool lora_fusable = rank <= 0 || (rank <= kGemvMaxFusedRank && lora_vec);
  for (int slice = 1; slice >= 0; --slice) {
    // activations through the waves' LDS slices: any unit to any wave
    const bool xslice = slice != 0;
    if (xslice && !(xvec && M <= kGemvXSliceMaxM)) continue;
    // segments one workgroup covers: 4 per wave with the slices, else one
    const int max_nseg = xslice ? kGemvWaves * kGemvMaxU : kGemvWaves;
    const int S = (nsegs + max_nseg - 1) / max_nseg;
    const int nseg = (nsegs + S - 1) / S;
    const int R = kGemvWaves / nseg;  // tile slots per round without the slices
    const int ts_cap = xslice ? (kGemvWaves * kGemvMaxU) / nseg : kGemvMaxU * R;
    const bool direct = S == 1 && lora_fusable;
    // K splits whose last split runs the epilogue: the LoRA term's operands
    // staged like the direct epilogue's, one counter per workgroup column
    const bool fold = S > 1 && lora_fusable;
    const bool epi_lds = (direct || fold) && rank > 0;
    // LDS of the in-launch down-projection: the wait flag
    bool in_launch = (direct || fold) && rank > 0 && lora_prod;
    const size_t job_lds = in_launch ? 16 : 0;
    // best tile count per workgroup: the fewest tiles a compute unit works
    // through one after another, the largest such count
    int best = 0;
    int64_t best_cost = 0;
    for (int TS = 1; TS <= kGemvMaxTS && TS <= ts_cap; ++TS) {
      const int U = xslice ? (TS * nseg + kGemvWaves - 1) / kGemvWaves : (TS + R - 1) / R;
      if (U != 1 && U != 2 && U != 4) continue;
      if (gemv_lds_bytes(TS, nseg, int(M), gather, xslice, epi_lds) + job_lds > size_t(kGemvLdsBudget))
        continue;
      const int64_t grid = (tiles + TS - 1) / TS;
      const int64_t cost = ((grid * S + ncu - 1) / ncu) * TS;
      if (best == 0 || cost <= best_cost) {
        best = TS;
        best_cost = cost;
      }
    }
    if (best == 0) continue;
    p.jobs = 0;
    // the jobs' handshake assumes every workgroup of the launch is resident
    // at once (one per compute unit)
    if ((tiles + best - 1) / best * S > ncu) in_launch = false;
    if (in_launch) {
      // wave jobs of one chunk each where the limits allow: C threads of
      // 16 splits per (m, j) with M rank C <= 1024 threads (C a power of
      // two, at most kJobMaxC; the partials then fit the synchronization
      // area), at most one job per wave
      const int64_t grid = (tiles + best - 1) / best * S;  // workgroups of the launch
      const int64_t nsteps = K / 32, groups = (rank + 15) / 16, mr = M * rank;
      int64_t cmax = 1;
      while (cmax < kJobMaxC && mr * cmax * 2 <= kGemvThreads) cmax *= 2;
      int64_t ns = (nsteps + kJobChunk - 1) / kJobChunk;
      ns = std::min<int64_t>(ns, kUPerThread * cmax);
      ns = std::min<int64_t>(ns, int64_t(kGemvPartWords) / mr);  // one partial region
      ns = std::min<int64_t>(ns, (kGemvWaves * grid) / groups);
      ns = std::max<int64_t>(ns, 1);
      p.u_splits = int(ns);
      p.jobs = int(groups * ns);
      // with K splits, only jobs of one chunk each: longer jobs end after
      // the splits' units (a 14-step job at M = 16, K = 14336 made the
      // launch 5 us slower than the down-projection launched before it)
      if (fold && ns * kJobChunk < nsteps) {
        p.jobs = 0;
        p.u_splits = launched_splits;
      }
    }
    p.S = S;
    p.nseg = nseg;
    p.TS = best;
    p.xslice = xslice;
    p.U = xslice ? (best * nseg + kGemvWaves - 1) / kGemvWaves : (best + R - 1) / R;
    p.grid = int((tiles + best - 1) / best);
    p.direct = direct;
    p.fold = fold && p.grid <= int(kGemmCountBytes / 4);
    break;
  }
  p.lds_bytes = gemv_lds_bytes(p.TS, p.nseg, int(M), gather, p.xslice, (p.direct || p.fold) && rank > 0);
  if (p.jobs > 0) p.lds_bytes += 16;  // the wait flag after RND(u)
  // workspace: the synchronization area (the in-launch down-projection's
  // count and partials, left zero by every launch), the split-K partials,
  // the partials of lora_u_kernel
  const size_t parts = p.direct ? 0 : size_t(p.S) * M * N * 4;
  const bool in_launch = p.jobs > 0;
  const size_t uparts = (rank > 0 && !in_launch) ? size_t(p.u_splits) * M * rank * 4 : 0;
  p.u_offset = kLinearSyncBytes + ((parts + 255) & ~size_t(255));
  p.ws_bytes = parts + uparts > 0 ? p.u_offset + uparts : (in_launch ? kLinearSyncBytes : 0);
  return p;
}

// x rows 16-byte aligned: the GEMV reads activations with 16-byte loads.
static bool gemv_xvec(const LinearArgs& L) { return aligned(L.x, 16) && L.ldx % 8 == 0; }

// log2 of the 16-byte chunks per LoRA B row when the GEMV epilogue can read
// the rows that way (aligned rows of a power of two of whole chunks), else -1:
// the LoRA term then goes to the split-K finisher.
static int gemv_bvec_log2(const LinearArgs& L) {
  if (L.rank <= 0) return -1;
  const int64_t bb = L.lora_dtype == RQ_DTYPE_F32 ? 4 : 2;
  const int64_t cpr = L.rank * bb / 16;
  if (!aligned(L.lora_b, 16) || (L.ld_lora_b * bb) % 16 != 0 || (L.rank * bb) % 16 != 0 || cpr <= 0 ||
      (cpr & (cpr - 1)) != 0)
    return -1;
  return pow2_shift(cpr);
}

template <int XT>
static int launch_lora_u(const LinearArgs& L, int ks, float* up, hipStream_t stream) {
  dim3 grid(unsigned((L.M + 15) / 16), unsigned((L.rank + 15) / 16), unsigned(ks));
  const bool xvec = aligned(L.lora_x, 16) && L.ld_lora_x % 8 == 0;
  const bool avec = aligned(L.lora_a, 16);
  lora_u_kernel<XT><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(L.lora_x), L.ld_lora_x, xvec,
                                              L.lora_a, L.lora_dtype, avec, L.M, L.K, int(L.rank), ks, up);
  return rq_check_launch();
}

template <int XT>
static int launch_lora_u_jobs(const LinearArgs& L, const LinearEpi& e, float* up, hipStream_t stream) {
  GemvArgs a{};
  a.M = int(L.M);
  a.K = int(L.K);
  a.lora_x = static_cast<const uint16_t*>(L.lora_x);
  a.ld_lora_x = int(L.ld_lora_x);
  a.lora_a = L.lora_a;
  const unsigned grid = unsigned((L.rank + 15) / 16) * unsigned(e.u_splits);
  lora_u_jobs_kernel<XT><<<grid, kGemvThreads, 0, stream>>>(a, e, up);
  return rq_check_launch();
}

// Devices on which an instantiation's dynamic-LDS limit has been raised
// (one bit per device index), one set per instantiation.
template <int XT, class Scale, int U, int XM>
static std::atomic<uint64_t>& attr_devices() {
  static std::atomic<uint64_t> bits{0};
  return bits;
}

template <int XT, class Scale, int U, int XM>
static int launch_gemv_u(const GemvArgs& a, const GemvPlan& p, Scale scale, const LinearEpi& e, hipStream_t stream) {
  auto kern = nf4_gemv_kernel<XT, Scale, U, XM>;
  if (int st = allow_dynamic_lds(reinterpret_cast<const void*>(kern), kGemvLdsBudget, attr_devices<XT, Scale, U, XM>());
      st != RQ_OK)
    return st;
  dim3 grid(unsigned(p.grid), unsigned(p.S));
  kern<<<grid, kGemvThreads, p.lds_bytes, stream>>>(a, scale, e);
  return rq_check_launch();
}

template <int XT, class Scale>
static int launch_gemv_t(const LinearArgs& L, const GemvPlan& p, Scale scale, const LinearEpi& e,
                         float* ws, void* sync, hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(L.x);
  a.ldx = int(L.ldx);
  a.packed = L.w_packed;
  a.M = int(L.M);
  a.N = int(L.N);
  a.K = int(L.K);
  a.bpr = int(L.K / L.block_size);
  a.bs_log2 = pow2_shift(L.block_size);
  a.nseg = p.nseg;
  a.TS = p.TS;
  a.direct = p.direct;
  a.tile_cnt = p.fold ? reinterpret_cast<uint32_t*>(static_cast<char*>(sync) + kLinearCountBytes + 2 * kGemvPartBytes)
                      : nullptr;
  a.xvec = gemv_xvec(L);
  a.bvec_log2 = gemv_bvec_log2(L);
  a.jobs = p.jobs;
  {
    const uint64_t ticks = uint64_t(gemv_wait_us.load(std::memory_order_relaxed)) * realtime_ticks_per_us();
    a.wait_ticks = uint32_t(std::min<uint64_t>(ticks, 0xFFFFFFFFull));
  }
  a.jc = static_cast<uint32_t*>(sync);
  a.state = static_cast<uint32_t*>(sync) + kLinearParityWord;
  a.parts = reinterpret_cast<uint32_t*>(static_cast<char*>(sync) + kLinearCountBytes);
  a.lora_x = static_cast<const uint16_t*>(L.lora_x);
  a.ld_lora_x = int(L.ld_lora_x);
  a.lora_a = L.lora_a;
  a.ws = ws;
  if (p.xslice) {
    switch (p.U) {
      case 1: return launch_gemv_u<XT, Scale, 1, 1>(a, p, scale, e, stream);
      case 2: return launch_gemv_u<XT, Scale, 2, 1>(a, p, scale, e, stream);
      default: return launch_gemv_u<XT, Scale, 4, 1>(a, p, scale, e, stream);
    }
  }
  switch (p.U) {
    case 1: return launch_gemv_u<XT, Scale, 1, 0>(a, p, scale, e, stream);
    case 2: return launch_gemv_u<XT, Scale, 2, 0>(a, p, scale, e, stream);
    default: return launch_gemv_u<XT, Scale, 4, 0>(a, p, scale, e, stream);
  }
}

template <int XT>
static int run_gemv(const LinearArgs& L, const GemvPlan& p, const LinearEpi& e, float* ws, void* sync,
                    hipStream_t stream) {
  if (L.c2) {
    const int sh = pow2_shift(L.block2);
    switch (L.absmax_dtype) {
      case RQ_DTYPE_F32:
        return launch_gemv_t<XT>(L, p, ScaleDQ<RQ_DTYPE_F32>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, ws, sync, stream);
      case RQ_DTYPE_BF16:
        return launch_gemv_t<XT>(L, p, ScaleDQ<RQ_DTYPE_BF16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, ws, sync, stream);
      default:
        return launch_gemv_t<XT>(L, p, ScaleDQ<RQ_DTYPE_F16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, ws, sync, stream);
    }
  }
  switch (L.absmax_dtype) {
    case RQ_DTYPE_F32: return launch_gemv_t<XT>(L, p, ScaleAbsmax<RQ_DTYPE_F32>{L.absmax}, e, ws, sync, stream);
    case RQ_DTYPE_BF16: return launch_gemv_t<XT>(L, p, ScaleAbsmax<RQ_DTYPE_BF16>{L.absmax}, e, ws, sync, stream);
    default: return launch_gemv_t<XT>(L, p, ScaleAbsmax<RQ_DTYPE_F16>{L.absmax}, e, ws, sync, stream);
  }
}

template <int XT>
static int launch_splitk_epilogue(const LinearArgs& L, const GemvPlan& p, const LinearEpi& e, const float* ws,
                                  hipStream_t stream) {
  dim3 grid(unsigned((L.N + 255) / 256), unsigned(L.M));
  const size_t lds = size_t(L.rank > 0 ? L.rank : 1) * 4;
  splitk_epilogue_kernel<XT><<<grid, 256, lds, stream>>>(ws, p.S, L.M, L.N, e);
  return rq_check_launch();
}

int validate_linear(const LinearArgs& L) {
  if (!valid_float_dtype(L.x_dtype)) return RQ_ERR_BAD_DTYPE;
  if (!valid_float_dtype(L.absmax_dtype)) return RQ_ERR_BAD_DTYPE;
  if (L.bias && !valid_float_dtype(L.bias_dtype)) return RQ_ERR_BAD_DTYPE;
  // LoRA A/B: fp32 (the trainable parameters) or the activation dtype; with
  // fp32 activations any float dtype (widened exactly, as A.to(x.dtype) does)
  if (L.rank > 0 && L.lora_dtype != RQ_DTYPE_F32 && L.lora_dtype != L.x_dtype &&
      !(L.x_dtype == RQ_DTYPE_F32 && valid_float_dtype(L.lora_dtype)))
    return RQ_ERR_BAD_DTYPE;
  if (L.c2 && L.c2_format != RQ_C2_FP8_E4M3FNUZ && L.c2_format != RQ_C2_INT8) return RQ_ERR_BAD_DTYPE;
  if (L.M < 0 || L.N < 1 || L.K < 1 || L.block_size < 1) return RQ_ERR_BAD_SHAPE;
  if (L.c2 && L.block2 < 1) return RQ_ERR_BAD_SHAPE;
  if (L.ldx < L.K || L.ldy < L.N) return RQ_ERR_BAD_SHAPE;
  if (L.rank < 0 || L.rank > 256) return RQ_ERR_BAD_SHAPE;
  if (L.rank > 0 && (L.ld_lora_x < L.K || L.ld_lora_b < L.rank)) return RQ_ERR_BAD_SHAPE;
  if (L.M == 0) return RQ_OK;
  if (!L.x || !L.w_packed || !L.absmax || !L.y) return RQ_ERR_NULL_POINTER;
  if (L.rank > 0 && (!L.lora_x || !L.lora_a || !L.lora_b)) return RQ_ERR_NULL_POINTER;
  if (!aligned(L.x, dtype_size(L.x_dtype)) || !aligned(L.y, dtype_size(L.x_dtype))) return RQ_ERR_BAD_ALIGNMENT;
  if (L.rank > 0 && !aligned(L.lora_x, dtype_size(L.x_dtype))) return RQ_ERR_BAD_ALIGNMENT;
  return RQ_OK;
}

// Whether the specialized kernels take the call (the decode GEMV, the MFMA
// GEMM, the fp32 path): K a multiple of 64, a power-of-two block size of at
// least 64 dividing K, the operands they read 16 bytes at a time aligned,
// offsets within their 32-bit addressing.  Every other valid call runs on
// the generic kernels.
bool linear_fast_ok(const LinearArgs& L) {
  if (L.K % 64 != 0 || L.block_size < 64 || (L.block_size & (L.block_size - 1)) != 0 || L.K % L.block_size != 0)
    return false;
  if (!aligned(L.w_packed, 8)) return false;
  if (L.x_dtype == RQ_DTYPE_F32)
    return L.rank <= 64 && aligned(L.x, 16) && L.ldx % 4 == 0 && aligned(L.w_packed, 16) &&
           (L.rank == 0 || (aligned(L.lora_x, 16) && L.ld_lora_x % 4 == 0 && aligned(L.lora_a, 16)));
  if (L.M <= kGemvMaxM)
    return L.N * (L.K / 2) <= int64_t(INT32_MAX) - 256 && L.K < (int64_t(1) << 27) &&
           (L.M - 1) * L.ldx + L.K <= (int64_t(1) << 29) && (L.rank == 0 || L.N * L.ld_lora_b <= (int64_t(1) << 29));
  return aligned(L.x, 16) && L.ldx % 8 == 0 && double(L.M) * double(L.ldx) * 2.0 < 4294967296.0 &&
         double(L.N) * double(L.K) * 0.5 < 4294967296.0 &&
         (L.rank == 0 || (aligned(L.lora_x, 16) && L.ld_lora_x % 8 == 0));
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
  // the plan depends on the activations' alignment, unknown here: the larger
  // of the two
  size_t b = 0;
  for (int c = 0; c < 8; ++c) {
    const GemvPlan p = plan_gemv(L.M, L.N, L.K, L.rank, device_cus(), c & 1, false, c & 2, c & 4);
    b = std::max(b, p.ws_bytes);
  }
  *bytes = b;
  return RQ_OK;
}

int run_nf4_gemv(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  // the GEMV addresses the packed weights with 32-bit byte offsets
  if (L.N * (L.K / 2) > int64_t(INT32_MAX) - 256 || L.K >= (int64_t(1) << 27)) return RQ_ERR_UNSUPPORTED;
  // ... and the activations, LoRA B and bias with 32-bit offsets too
  if ((L.M - 1) * L.ldx + L.K > (int64_t(1) << 29)) return RQ_ERR_UNSUPPORTED;
  if (L.rank > 0 && L.N * L.ld_lora_b > (int64_t(1) << 29)) return RQ_ERR_UNSUPPORTED;
  // the down-projection runs inside the GEMV launch when the x rows and A
  // are 16-byte aligned (its jobs read both 16 bytes at a time) and both
  // are addressed with 32-bit offsets
  const bool lora_prod = L.rank > 0 && aligned(L.lora_x, 16) && L.ld_lora_x % 8 == 0 && aligned(L.lora_a, 16) &&
                         (L.M - 1) * L.ld_lora_x + L.K <= (int64_t(1) << 29) && L.rank * L.K <= (int64_t(1) << 28);
  const GemvPlan p = plan_gemv(L.M, L.N, L.K, L.rank, device_cus(), gemv_xvec(L), L.c2 == nullptr,
                               gemv_bvec_log2(L) >= 0, lora_prod);
  if (p.ws_bytes > 0 && (!workspace || ws_bytes < p.ws_bytes)) return RQ_ERR_WORKSPACE;
  if (workspace && !aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  char* wsb = static_cast<char*>(workspace);
  float* ws = p.direct ? nullptr : reinterpret_cast<float*>(wsb + kLinearSyncBytes);
  float* up = L.rank > 0 ? reinterpret_cast<float*>(wsb + p.u_offset) : nullptr;
  int st;
  const LinearEpi e = make_epi(L, up, p.u_splits);
  if (L.rank > 0 && p.jobs == 0) {
    if (lora_prod) {
      st = L.x_dtype == RQ_DTYPE_BF16 ? launch_lora_u_jobs<RQ_DTYPE_BF16>(L, e, up, stream)
                                      : launch_lora_u_jobs<RQ_DTYPE_F16>(L, e, up, stream);
    } else {
      st = run_lora_u(L, p.u_splits, up, stream);
    }
    if (st != RQ_OK) return st;
  }
  if (L.x_dtype == RQ_DTYPE_BF16) st = run_gemv<RQ_DTYPE_BF16>(L, p, e, ws, workspace, stream);
  else st = run_gemv<RQ_DTYPE_F16>(L, p, e, ws, workspace, stream);
  if (st != RQ_OK || p.direct || p.fold) return st;
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

extern "C" uint32_t rq_set_gemv_wait_us(uint32_t us) { return set_gemv_wait_us(us); }

extern "C" int rq_nf4_linear_workspace_size(int x_dtype, int64_t M, int64_t K, int64_t N, int64_t rank,
                                            int64_t* bytes) {
  if (!bytes) return RQ_ERR_NULL_POINTER;
  if (!valid_float_dtype(x_dtype)) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || N < 1 || K < 1 || rank < 0 || rank > 256) return RQ_ERR_BAD_SHAPE;
  // the larger of what the specialized kernels need (when K % 64 == 0; the
  // block size and the operands' alignment, unknown here, decide whether
  // they run) and what the generic kernels need
  size_t b = rank > 0 ? kLinearSyncBytes + generic_lora_bytes(x_dtype, M, rank) : 0;
  if (K % 64 != 0) {
    *bytes = int64_t(b);
    return RQ_OK;
  }
  size_t f = 0;
  LinearArgs L{};
  L.x_dtype = x_dtype; L.M = M; L.K = K; L.N = N; L.rank = rank;
  int st = RQ_OK;
  if (x_dtype == RQ_DTYPE_F32) {
    f32_linear_workspace(L, &f);
  } else {
    st = M <= kGemvMaxM ? gemv_workspace(L, &f) : gemm_workspace(L, &f);
    if (M > kGemvMaxM && f > 0) f += kLinearSyncBytes;
  }
  *bytes = int64_t(std::max(b, f));
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
  if (!linear_fast_ok(L)) return run_generic_nf4_linear(L, workspace, size_t(workspace_bytes), stream);
  if (x_dtype == RQ_DTYPE_F32) return run_nf4_linear_f32(L, workspace, size_t(workspace_bytes), stream);
  if (M <= kGemvMaxM) return run_nf4_gemv(L, workspace, size_t(workspace_bytes), stream);
  // the GEMM's workspace follows the synchronization area, whose last
  // kGemmCountBytes serve as its K splits' tile counters
  const bool area = workspace && size_t(workspace_bytes) >= kLinearSyncBytes;
  return run_nf4_gemm(L, area ? static_cast<char*>(workspace) + kLinearSyncBytes : nullptr,
                      area ? size_t(workspace_bytes) - kLinearSyncBytes : 0,
                      area ? reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + kLinearSyncBytes -
                                                         kGemmCountBytes)
                           : nullptr,
                      kGemmCountBytes / 4, stream);
}

// ===========================================================================
// Allocation-free variant of rq_nf4_linear (no counterpart in the reference):
// its workspace is a file-scope device array, so the call allocates nothing.
// ===========================================================================
namespace rq {

// The workspace of rq_nf4_linear_noalloc on every device the library runs on
// (each device holds its own copy until the process ends).  Host code never
// uses this name as an address: the per-device address comes from
// hipGetSymbolAddress.  Zero at load; its synchronization area is cleared
// once more on a device's first call and left zero by every call.
static __device__ __align__(256) uint8_t scratch[RQ_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
// per device: the array's device address (nullptr until the first call)
static std::atomic<void*> scratch_ptr[kMaxScratchDevices];

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The current device's scratch address; on the device's first call, looks it
// up and clears the synchronization area with a fill kernel on `stream` (a
// kernel, not a memset, so that a graph capture records a kernel node).
static int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return RQ_ERR_HIP;
  if (dev < 0 || dev >= kMaxScratchDevices) return RQ_ERR_UNSUPPORTED;
  void* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    void* q = nullptr;
    if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return RQ_ERR_HIP;
    constexpr int64_t words = int64_t(kLinearSyncBytes) / 4;
    zero_words_kernel<<<unsigned((words + 255) / 256), 256, 0, stream>>>(static_cast<uint32_t*>(q), words);
    if (int st = rq_check_launch(); st != RQ_OK) return st;
    void* expected = nullptr;
    // racing first calls on one device look up the same address
    scratch_ptr[dev].compare_exchange_strong(expected, q, std::memory_order_acq_rel);
    p = q;
  }
  *out = p;
  return RQ_OK;
}

}  // namespace rq

extern "C" int rq_nf4_linear_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                                     const uint8_t* w_packed, int64_t N, int64_t block_size, const void* absmax,
                                     int absmax_dtype, const uint8_t* c2, int c2_format, int64_t block2,
                                     const void* bias, int bias_dtype, const void* lora_x, int64_t ld_lora_x,
                                     const void* lora_a, const void* lora_b, int64_t ld_lora_b, int lora_dtype,
                                     int64_t rank, float scaling, void* y, int64_t ldy, hipStream_t stream) {
  const LinearArgs L = pack_linear_args(x, x_dtype, M, K, ldx, w_packed, N, block_size, absmax, absmax_dtype,
                                        c2, c2_format, block2, bias, bias_dtype, lora_x, ld_lora_x, lora_a,
                                        lora_b, ld_lora_b, lora_dtype, rank, scaling, y, ldy);
  int st = validate_linear(L);
  if (st != RQ_OK || M == 0) return st;
  // the smallest workspace the call runs with (the GEMM drops its K splits
  // when their partial tiles do not fit)
  int64_t need = 0;
  if (!linear_fast_ok(L)) {
    need = L.rank > 0 ? int64_t(kLinearSyncBytes + generic_lora_bytes(x_dtype, M, L.rank)) : 0;
  } else if (x_dtype != RQ_DTYPE_F32 && M > kGemvMaxM) {
    const size_t b = gemm_min_workspace(L);
    need = b > 0 ? int64_t(b + kLinearSyncBytes) : 0;
  } else {
    st = rq_nf4_linear_workspace_size(x_dtype, M, K, N, L.rank, &need);
    if (st != RQ_OK) return st;
  }
  if (need > int64_t(RQ_NOALLOC_SCRATCH_BYTES)) return RQ_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  st = noalloc_scratch(stream, &ws);
  if (st != RQ_OK) return st;
  return rq_nf4_linear(x, x_dtype, M, K, ldx, w_packed, N, block_size, absmax, absmax_dtype, c2, c2_format, block2,
                       bias, bias_dtype, lora_x, ld_lora_x, lora_a, lora_b, ld_lora_b, lora_dtype, rank, scaling,
                       y, ldy, ws, int64_t(RQ_NOALLOC_SCRATCH_BYTES), stream);
}
