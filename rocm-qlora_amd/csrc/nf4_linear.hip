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
#include "rq_mfma.h"
#include "rq_launch.h"
#include "rq_linear.h"
#include "rq_linear_dev.h"

namespace rq {

// ---------------------------------------------------------------------------
// Decode GEMV: y[M <= 16, N] = x[M, K] . W^T, W NF4 (block size a power of
// two >= 64 dividing K, K % 64 == 0).
//
// HBM access: a "segment" is 256 k of a 16-row tile, 128 contiguous bytes per
// row.  A wave reads it with two 1 KiB loads, 8 lanes x 16 B per row (full
// 128-byte lines; narrower per-row pieces cost HBM efficiency):
//   load A: lane (n = l % 16, q = l / 16) reads row n % 8,     chunk q + 4 [n >= 8]
//   load B: lane (n, q)                   reads row 8 + n % 8, chunk q + 4 [n < 8]
// (chunk = 16 B = 32 k).  Then X1 = n < 8 ? A : B holds row n, chunk q in
// every lane, and X2 = row_ror8(n >= 8 ? A : B) (a DPP rotate by 8 within
// each 16-lane row) holds row n, chunk q + 4: the 16x16x32 MFMA B-operand
// layout (lane l = row l % 16, k group l / 16) with no LDS round trip.
// Steps 0-3 take X1's dwords, steps 4-7 X2's; the activation operand (A,
// rows = tokens, zero past M) uses the same k order.  Each dword of codes
// becomes RND(T[code] * scale) through the LDS pair table.
//
// Grid (G, S), 1024 threads: workgroup (g, s) owns K split s (at most 16
// segments; S > 1 only when K > 4096) and the NT <= 4 tiles g, g + G, ...,
// g + (NT - 1) G.  The kernel is straight-line: every wave issues the loads
// of all its tiles before it computes any (NT x 2 KiB per wave), and no
// loaded value is carried around a loop, so the compiler's in-order load
// counting is exact and each tile's math waits only for that tile's data.
// Epilogue operands (the tiles' LoRA B rows, bias, RND(u)) are fetched before
// the weights and staged in LDS once.  One barrier publishes the 16 wave
// partials of every tile; they are summed in a fixed order (deterministic
// results) and finished by one thread per output.
// ---------------------------------------------------------------------------
constexpr int kGemvThreads = 1024;
constexpr int kGemvWaves = kGemvThreads / 64;
constexpr int kSegK = 256;
constexpr int kGemvMaxNT = 4;          // tiles per workgroup
constexpr int kGemvMaxFusedRank = 64;  // LoRA rank the in-kernel epilogue stages
constexpr int kGemvMaxUSplits = 16;
constexpr int kGemvLutQwords = 256 * 32;  // 64 KiB: code byte -> fp32 (T[lo], T[hi]), 32 copies
// Word 3 of a raw (stride 0) buffer resource on gfx9-family GPUs, gfx950
// included: 32-bit data, bounds checked against num_records.
constexpr int kBufferRsrcWord3 = 0x00020000;

struct GemvArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* packed;
  int64_t M, N, K;
  int64_t blocks_per_row;  // K / block_size
  int bs_log2;             // log2(block_size)
  int S;                   // K splits (gridDim.y)
  bool direct;             // epilogue in this kernel (else fp32 partials to ws)
  bool xvec;
  float* ws;               // [S, M, N] partials when !direct
};

// One tile's loads for one lane: loads A and B (raw code bits) and the
// scales of chunks q and q + 4 of row n.
template <class Scale>
struct GemvTileLoads {
  u32x4 a, b;
  typename Scale::Raw s1, s2;
};

struct GemvLane {
  int n16, q;
  int64_t seg;  // this wave's segment
  bool live;    // the wave has a segment of this split
};

// Loads of one tile for one lane.  The packed weights are read through a
// buffer resource whose range is the weight matrix, so rows past N (a tile
// past the end, or the rows of a last, partial tile) read as zero codes
// without a bounds test, and chunks past K in a last, partial segment read
// codes of the next row (or zeros) that meet zero activations.  Offsets are
// 32-bit (the host keeps the packed weights under 2 GiB).  The loads are
// issued on every path, branch-free, so each wave issues the same loads in
// the same order and the compiler's in-order load counting stays exact.
template <class Scale>
__device__ __forceinline__ void gemv_issue_tile(GemvTileLoads<Scale>& L, const GemvArgs& a, const Scale& scale,
                                                __amdgpu_buffer_rsrc_t wres, uint32_t tile, const GemvLane& w) {
  const uint32_t half_k = uint32_t(a.K >> 1);
  const uint32_t r0 = tile * 16u, n7 = uint32_t(w.n16 & 7);
  const uint32_t cA = uint32_t(w.q) + (w.n16 >= 8 ? 4u : 0u), cB = uint32_t(w.q) + (w.n16 < 8 ? 4u : 0u);
  const uint32_t sb = uint32_t(w.seg) * (kSegK / 2);
  L.a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, (r0 + n7) * half_k + sb + 16u * cA, 0, 0));
  L.b = __builtin_bit_cast(u32x4,
                           __builtin_amdgcn_raw_buffer_load_b128(wres, (r0 + 8u + n7) * half_k + sb + 16u * cB, 0, 0));
  uint32_t srow = r0 + uint32_t(w.n16);
  srow = srow < uint32_t(a.N) ? srow : uint32_t(a.N) - 1u;
  const uint32_t kmax = uint32_t(a.K) - 1u;
  uint32_t k1 = uint32_t(w.seg) * kSegK + 32u * uint32_t(w.q), k2 = k1 + 128u;
  k1 = k1 < kmax ? k1 : kmax;
  k2 = k2 < kmax ? k2 : kmax;
  const uint32_t sr = srow * uint32_t(a.blocks_per_row);
  L.s1 = scale.load(int64_t(sr + (k1 >> a.bs_log2)));
  L.s2 = scale.load(int64_t(sr + (k2 >> a.bs_log2)));
}

__device__ __forceinline__ uint32_t row_ror8(uint32_t v) {
  return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x128, 0xF, 0xF, false));
}

template <int XT, class Scale>
__device__ __forceinline__ f32x4 gemv_tile(const GemvTileLoads<Scale>& L, const Scale& scale, const u32x4 (&xa)[8],
                                           const u32x2* lut, uint32_t lane_off, int n16) {
  const bool lo = n16 < 8;
  const u32x4 X1 = lo ? L.a : L.b;
  const u32x4 Y = lo ? L.b : L.a;
  const u32x4 X2 = u32x4{row_ror8(Y.x), row_ror8(Y.y), row_ror8(Y.z), row_ror8(Y.w)};
  const float s1 = scale.value(L.s1), s2 = scale.value(L.s2);
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

// The code book as fp32 bits (for the table fill).
__device__ const uint32_t kNF4BitsDev[16] = {
    kNF4Bits[0], kNF4Bits[1], kNF4Bits[2],  kNF4Bits[3],  kNF4Bits[4],  kNF4Bits[5],  kNF4Bits[6],  kNF4Bits[7],
    kNF4Bits[8], kNF4Bits[9], kNF4Bits[10], kNF4Bits[11], kNF4Bits[12], kNF4Bits[13], kNF4Bits[14], kNF4Bits[15]};

// Fill of the fp32 pair table by 1024 threads: entry e (a code byte) holds
// (T[e & 15], T[e >> 4]); copy c at qword e * 32 + c (lane l reads copy
// l % 32: a ds_read_b64 serves 32 lanes per cycle, which hit 32 distinct
// bank pairs).  Thread t writes copies 8 (t % 4) .. + 7 of entry t / 4.
__device__ __forceinline__ void fill_gemv_lut(u32x2* lut, uint32_t t_even, uint32_t t_odd, int tid) {
  u32x4* dst = reinterpret_cast<u32x4*>(lut + (tid >> 2) * 32 + 8 * (tid & 3));
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = u32x4{t_even, t_odd, t_even, t_odd};
}

// Workgroup barrier for LDS only: this wave's LDS accesses are complete,
// then s_barrier.  (__syncthreads() may also wait for every outstanding
// global load, which would serialize the prefetched tiles.)
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Dynamic LDS of the GEMV: wave partials [NT][16 waves][M][16], RND(B) of the
// tiles' rows [NT * 16][64], RND(bias) [NT * 16], RND(u) [M][64] (fp32).
__host__ __device__ inline size_t gemv_lds_floats(int nt, int64_t M, bool lora) {
  return size_t(nt) * kGemvWaves * M * 16 + (lora ? size_t(nt) * 16 * kGemvMaxFusedRank : 0) + size_t(nt) * 16 +
         (lora ? size_t(M) * kGemvMaxFusedRank : 0);
}

template <int XT, class Scale, int NT>
__global__ __launch_bounds__(kGemvThreads) void nf4_gemv_kernel(GemvArgs a, Scale scale, LinearEpi e) {
  // The table is the kernel's only static LDS array, so it sits at address
  // 0 and every lookup's base folds into the instruction's offset field.
  __shared__ u32x2 lut[kGemvLutQwords];
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int M = int(a.M);
  const int rank = (a.direct && e.rank > 0) ? e.rank : 0;  // LoRA staging only when fused here
  constexpr int RP = kGemvMaxFusedRank;                    // staging pitch
  float* part = reinterpret_cast<float*>(smem);
  float* lbs = part + NT * kGemvWaves * M * 16;
  float* bss = lbs + (rank > 0 ? NT * 16 * RP : 0);
  float* us = bss + NT * 16;

  GemvLane w;
  w.n16 = lane & 15;
  w.q = lane >> 4;
  const int s = blockIdx.y;
  const int64_t nsegs = (a.K + kSegK - 1) / kSegK;
  const int64_t sg0 = (nsegs * s) / a.S, sg1 = (nsegs * (s + 1)) / a.S;
  w.live = sg0 + wave < sg1;
  w.seg = w.live ? sg0 + wave : sg0;  // a wave without a segment re-reads one; its activations are zero
  const uint32_t n_tiles = uint32_t((a.N + 15) / 16);
  // tiles g, g + G, g + 2G, ...: at any moment the workgroups' loads are
  // spread over the whole weight matrix
  auto tile_idx = [&](int t) -> uint32_t { return blockIdx.x + uint32_t(t) * gridDim.x; };
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.packed), 0, int(uint32_t(a.N) * uint32_t(a.K >> 1)), kBufferRsrcWord3);

  // 1. Loads the weights do not depend on, issued first so that staging them
  //    waits only for them: the table entry this thread writes, the tiles'
  //    LoRA B values (value i of thread t is row t / 64 + 16 i, rank t % 64
  //    of the [NT * 16][64] staging block), the bias, the RND(u) partials
  //    (waves m < M) and the activation operands.
  const uint32_t t_even = kNF4BitsDev[(tid >> 2) & 15], t_odd = kNF4BitsDev[tid >> 6];
  Raw16x2 lbr[NT];
  const int lj = tid & (RP - 1);
  if (rank > 0) {
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int rr = (tid >> 6) + 16 * i;
      uint32_t bn = tile_idx(rr >> 4) * 16u + uint32_t(rr & 15);
      bn = bn < uint32_t(a.N) ? bn : uint32_t(a.N) - 1u;
      const int j = lj < rank ? lj : 0;
      lbr[i] = load_raw(e.lora_b, int64_t(bn) * e.ld_lora_b + j, e.lora_dt);
    }
  }
  const bool has_bias = a.direct && e.bias != nullptr;
  Raw16x2 br;
  if (has_bias) {
    const int cb = tid & (NT * 16 - 1);
    uint32_t cn = tile_idx(cb >> 4) * 16u + uint32_t(cb & 15);
    cn = cn < uint32_t(a.N) ? cn : uint32_t(a.N) - 1u;
    br = load_raw(e.bias, int64_t(cn), e.bias_dt);
  }
  float up[kGemvMaxUSplits];
  const int um = wave;  // RND(u) row m is staged by wave m
  const bool stage_u = rank > 0 && um < M;
  if (stage_u) {
    const uint32_t u_idx = uint32_t(um * rank + (lj < rank ? lj : 0));
    const uint32_t u_stride = uint32_t(M * rank);
    const int ns = e.u_splits;
#pragma unroll
    for (int k = 0; k < kGemvMaxUSplits; ++k) up[k] = e.u[(k < ns ? uint32_t(k) : 0u) * u_stride + u_idx];
  }
  // activations: step c covers x[token][seg * 256 + 128 (c / 4) + 32 q + 8
  // (c % 4) ...]; a token past M, a k past K and a wave without a segment
  // read zeros
  u32x4 xa[8];
  const bool mlive = w.n16 < M && w.live;
  if (a.xvec) {
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.x), 0, int(uint32_t(M - 1) * uint32_t(a.ldx) * 2u + uint32_t(a.K) * 2u),
        kBufferRsrcWord3);
    const uint32_t xrow = uint32_t(w.n16) * uint32_t(a.ldx) * 2u;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t k = uint32_t(w.seg) * kSegK + 128u * (c >> 2) + 32u * uint32_t(w.q) + 8u * (c & 3);
      const uint32_t off = (mlive && k < uint32_t(a.K)) ? xrow + 2u * k : 0xFFFFFFF0u;
      xa[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 0, 0));
    }
  } else {
    const uint16_t* xrow = a.x + (w.n16 < M ? w.n16 : 0) * a.ldx;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      int64_t k = w.seg * kSegK + 128 * (c >> 2) + 32 * w.q + 8 * (c & 3);
      const bool live = mlive && k < a.K;
      k = k < a.K ? k : 0;
      const u32x4 v = load_x8(xrow + k, false);
      xa[c] = live ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }

  // 2. every tile's weights and scales
  GemvTileLoads<Scale> buf[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) gemv_issue_tile(buf[t], a, scale, wres, tile_idx(t), w);

  // 3. the table and the epilogue operands into LDS (these wait for the
  //    loads of step 1 only)
  fill_gemv_lut(lut, t_even, t_odd, tid);
  if (rank > 0) {
#pragma unroll
    for (int i = 0; i < NT; ++i)
      lbs[tid + 1024 * i] = lj < rank ? round_x<XT>(raw_to_f32(lbr[i], e.lora_dt)) : 0.0f;
  }
  if (a.direct && tid < NT * 16) bss[tid] = has_bias ? round_x<XT>(raw_to_f32(br, e.bias_dt)) : 0.0f;
  if (stage_u) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kGemvMaxUSplits; ++k)
      if (k < e.u_splits) sum = __fadd_rn(sum, up[k]);
    us[tid] = lj < rank ? round_x<XT>(sum) : 0.0f;
  }
  lds_barrier();

  // 4. the tiles, each as soon as its loads have landed; partials to LDS
  const uint32_t lane_off = uint32_t(lane & 31) * 8u;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const f32x4 acc = gemv_tile<XT>(buf[t], scale, xa, lut, lane_off, w.n16);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * w.q + r;
      if (m < M) part[((t * kGemvWaves + wave) * M + m) * 16 + w.n16] = acc[r];
    }
  }
  lds_barrier();

  // 5. one thread per output (tile t = tid / 256, row m, column nn): the 16 wave
  //    partials in wave order, then bias, LoRA, rounding -- or the fp32 sum
  //    to the split-K workspace
  const int t = tid >> 8, m = (tid >> 4) & 15, nn = tid & 15;
  if (t >= NT || m >= M) return;
  const uint32_t tile = tile_idx(t);
  const int64_t n = int64_t(tile) * 16 + nn;
  if (tile >= n_tiles || n >= a.N) return;
  float p[kGemvWaves];
#pragma unroll
  for (int ww = 0; ww < kGemvWaves; ++ww) p[ww] = part[((t * kGemvWaves + ww) * M + m) * 16 + nn];
  float v = 0.0f;
#pragma unroll
  for (int ww = 0; ww < kGemvWaves; ++ww) v = __fadd_rn(v, p[ww]);
  if (!a.direct) {
    a.ws[(int64_t(s) * a.M + m) * a.N + n] = v;
    return;
  }
  if (e.bias) v = __fadd_rn(v, bss[t * 16 + nn]);
  v = round_x<XT>(v);
  if (rank > 0) {
    const float* brow = lbs + (t * 16 + nn) * RP;
    const float* urow = us + m * RP;
    float l = 0.0f;
    for (int j0 = 0; j0 < rank; j0 += 8) {
      float uu[8], bb[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        uu[jj] = urow[j0 + jj];  // zero past rank
        bb[jj] = brow[j0 + jj];
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) l = __fmaf_rn(uu[jj], bb[jj], l);
    }
    l = round_x<XT>(__fmul_rn(round_x<XT>(l), e.scaling));
    v = round_x<XT>(__fadd_rn(v, l));
  }
  static_cast<uint16_t*>(e.y)[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
}

// Split-K finisher (and the LoRA epilogue for any M): y = finish(sum_s
// ws[s]).  Workgroup = 256 columns x 16 activation rows; B values are read 8
// at a time, all in flight together, and reused for the 16 rows.
template <int XT>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(const float* __restrict__ ws, int S, int64_t M,
                                                              int64_t N, LinearEpi e) {
  extern __shared__ float us[];
  const int64_t m0 = int64_t(blockIdx.y) * 16;
  stage_u<XT>(e, M, m0, 16, us, threadIdx.x, blockDim.x);
  __syncthreads();
  const int64_t n = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (n >= N) return;
  const int rows = int(M - m0 < 16 ? M - m0 : 16);
  float lsum[16];
#pragma unroll
  for (int mm = 0; mm < 16; ++mm) lsum[mm] = 0.0f;
  for (int j0 = 0; j0 < e.rank; j0 += 8) {
    float b[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      b[jj] = (j0 + jj < e.rank) ? round_x<XT>(load_as_f32(e.lora_b, n * e.ld_lora_b + j0 + jj, e.lora_dt)) : 0.0f;
#pragma unroll
    for (int mm = 0; mm < 16; ++mm)
      if (mm < rows)
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          if (j0 + jj < e.rank) lsum[mm] = __fmaf_rn(us[mm * e.rank + j0 + jj], b[jj], lsum[mm]);
  }
#pragma unroll
  for (int mm = 0; mm < 16; ++mm) {
    if (mm >= rows) break;
    const int64_t m = m0 + mm;
    float p[8];
    float v = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 8) {
#pragma unroll
      for (int k = 0; k < 8; ++k) p[k] = (s0 + k < S) ? ws[(int64_t(s0 + k) * M + m) * N + n] : 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (s0 + k < S) v = __fadd_rn(v, p[k]);
    }
    v = finish_value<XT>(e, n, v, lsum[mm]);
    static_cast<uint16_t*>(e.y)[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
  }
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

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
GemvPlan plan_gemv(int64_t M, int64_t N, int64_t K, int64_t rank, int cus) {
  GemvPlan p{};
  const int64_t nsegs = (K + kSegK - 1) / kSegK;
  const int64_t tiles = (N + 15) / 16;
  p.nw = kGemvWaves;
  p.RT = 1;
  // one segment per wave: K splits only past 16 segments (K > 4096)
  const int S = int((nsegs + kGemvWaves - 1) / kGemvWaves);
  p.S = S;
  // tiles per workgroup: enough that one round of workgroups covers the
  // chip's compute units, at most kGemvMaxNT
  int64_t nt = (tiles * S + cus - 1) / (cus > 0 ? cus : 1);
  nt = nt < 1 ? 1 : (nt > kGemvMaxNT ? kGemvMaxNT : nt);
  p.NT = nt > 2 ? 4 : int(nt);
  p.grid = int((tiles + p.NT - 1) / p.NT);
  p.u_splits = 0;
  if (rank > 0) {
    const int64_t steps_per_wg = 4 * kLoraUStepsPerWave;
    p.u_splits = int((K / 32 + steps_per_wg - 1) / steps_per_wg);
  }
  // the fused epilogue stages the tiles' B rows (rank <= 64), <= 16 u splits
  p.direct = S == 1 && rank <= kGemvMaxFusedRank && p.u_splits <= kGemvMaxUSplits;
  p.lds_bytes = gemv_lds_floats(p.NT, M, p.direct && rank > 0) * 4;  // dynamic part (the 64 KiB table is static)
  p.ws_bytes = p.direct ? 0 : size_t(S) * M * N * 4;
  p.u_offset = (p.ws_bytes + 255) & ~size_t(255);
  if (rank > 0) p.ws_bytes = p.u_offset + size_t(p.u_splits) * M * rank * 4;
  return p;
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

template <int XT, class Scale, int NT>
static int launch_gemv_nt(const GemvArgs& a, GemvPlan p, Scale scale, const LinearEpi& e, hipStream_t stream) {
  p.grid = int(((a.N + 15) / 16 + NT - 1) / NT);
  auto kern = nf4_gemv_kernel<XT, Scale, NT>;
  static bool attr_set = false;  // one flag per instantiation
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024 - kGemvLutQwords * 8) != hipSuccess)
      return RQ_ERR_HIP;
    attr_set = true;
  }
  dim3 grid(unsigned(p.grid), unsigned(p.S));
  kern<<<grid, kGemvThreads, p.lds_bytes, stream>>>(a, scale, e);
  return rq_check_launch();
}

template <int XT, class Scale>
static int launch_gemv_t(const LinearArgs& L, const GemvPlan& p, Scale scale, const LinearEpi& e,
                         float* ws, hipStream_t stream) {
  GemvArgs a;
  a.x = static_cast<const uint16_t*>(L.x);
  a.ldx = L.ldx;
  a.packed = L.w_packed;
  a.M = L.M;
  a.N = L.N;
  a.K = L.K;
  a.blocks_per_row = L.K / L.block_size;
  a.bs_log2 = pow2_shift(L.block_size);
  a.S = p.S;
  a.direct = p.direct;
  a.xvec = aligned(L.x, 16) && (L.ldx % 8 == 0);
  a.ws = ws;
  // double quantization keeps two loads per scale: at most 2 tiles per
  // workgroup stay within the registers
  if (p.NT == 1) return launch_gemv_nt<XT, Scale, 1>(a, p, scale, e, stream);
  if constexpr (Scale::kLoads > 1) {
    return launch_gemv_nt<XT, Scale, 2>(a, p, scale, e, stream);
  } else {
    if (p.NT == 2) return launch_gemv_nt<XT, Scale, 2>(a, p, scale, e, stream);
    return launch_gemv_nt<XT, Scale, 4>(a, p, scale, e, stream);
  }
}

template <int XT>
static int run_gemv(const LinearArgs& L, const GemvPlan& p, const LinearEpi& e, float* ws, hipStream_t stream) {
  if (L.c2) {
    const int sh = pow2_shift(L.block2);
    switch (L.absmax_dtype) {
      case RQ_DTYPE_F32:
        return launch_gemv_t<XT>(L, p, ScaleDQ<RQ_DTYPE_F32>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, ws, stream);
      case RQ_DTYPE_BF16:
        return launch_gemv_t<XT>(L, p, ScaleDQ<RQ_DTYPE_BF16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, ws, stream);
      default:
        return launch_gemv_t<XT>(L, p, ScaleDQ<RQ_DTYPE_F16>{L.c2, L.absmax, L.c2_format, sh, L.block2}, e, ws, stream);
    }
  }
  switch (L.absmax_dtype) {
    case RQ_DTYPE_F32: return launch_gemv_t<XT>(L, p, ScaleAbsmax<RQ_DTYPE_F32>{L.absmax}, e, ws, stream);
    case RQ_DTYPE_BF16: return launch_gemv_t<XT>(L, p, ScaleAbsmax<RQ_DTYPE_BF16>{L.absmax}, e, ws, stream);
    default: return launch_gemv_t<XT>(L, p, ScaleAbsmax<RQ_DTYPE_F16>{L.absmax}, e, ws, stream);
  }
}

template <int XT>
static int launch_splitk_epilogue(const LinearArgs& L, const GemvPlan& p, const LinearEpi& e, const float* ws,
                                  hipStream_t stream) {
  dim3 grid(unsigned((L.N + 255) / 256), unsigned((L.M + 15) / 16));
  const size_t lds = size_t(16) * (L.rank > 0 ? L.rank : 1) * 4;
  splitk_epilogue_kernel<XT><<<grid, 256, lds, stream>>>(ws, p.S, L.M, L.N, e);
  return rq_check_launch();
}

int validate_linear(const LinearArgs& L) {
  if (L.x_dtype != RQ_DTYPE_BF16 && L.x_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (!valid_float_dtype(L.absmax_dtype)) return RQ_ERR_BAD_DTYPE;
  if (L.bias && !valid_float_dtype(L.bias_dtype)) return RQ_ERR_BAD_DTYPE;
  // LoRA A/B: fp32 (the trainable parameters) or the activation dtype
  if (L.rank > 0 && L.lora_dtype != RQ_DTYPE_F32 && L.lora_dtype != L.x_dtype) return RQ_ERR_BAD_DTYPE;
  if (L.c2 && L.c2_format != RQ_C2_FP8_E4M3FNUZ && L.c2_format != RQ_C2_INT8) return RQ_ERR_BAD_DTYPE;
  if (L.M < 0 || L.N < 1 || L.K < 64 || L.K % 64 != 0) return RQ_ERR_BAD_SHAPE;
  if (L.block_size < 64 || L.block_size % 64 != 0 || L.K % L.block_size != 0) return RQ_ERR_BAD_SHAPE;
  if ((L.block_size & (L.block_size - 1)) != 0) return RQ_ERR_BAD_SHAPE;
  if (L.c2 && L.block2 < 1) return RQ_ERR_BAD_SHAPE;
  if (L.ldx < L.K || L.ldy < L.N) return RQ_ERR_BAD_SHAPE;
  if (L.rank < 0 || L.rank > 256) return RQ_ERR_BAD_SHAPE;
  if (L.rank > 0 && (L.ld_lora_x < L.K || L.ld_lora_b < L.rank)) return RQ_ERR_BAD_SHAPE;
  if (L.M == 0) return RQ_OK;
  if (!L.x || !L.w_packed || !L.absmax || !L.y) return RQ_ERR_NULL_POINTER;
  if (L.rank > 0 && (!L.lora_x || !L.lora_a || !L.lora_b)) return RQ_ERR_NULL_POINTER;
  if (!aligned(L.w_packed, 8)) return RQ_ERR_BAD_ALIGNMENT;
  if (!aligned(L.x, 2) || !aligned(L.y, 2)) return RQ_ERR_BAD_ALIGNMENT;
  return RQ_OK;
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
  GemvPlan p = plan_gemv(L.M, L.N, L.K, L.rank, device_cus());
  *bytes = p.ws_bytes;
  return RQ_OK;
}

int run_nf4_gemv(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream) {
  // the GEMV addresses the packed weights with 32-bit byte offsets
  if (L.N * (L.K / 2) > int64_t(INT32_MAX) - 256) return RQ_ERR_UNSUPPORTED;
  const GemvPlan p = plan_gemv(L.M, L.N, L.K, L.rank, device_cus());
  if (p.ws_bytes > 0 && (!workspace || ws_bytes < p.ws_bytes)) return RQ_ERR_WORKSPACE;
  if (workspace && !aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  float* ws = static_cast<float*>(workspace);
  float* up = L.rank > 0 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.u_offset) : nullptr;
  int st;
  if (L.rank > 0 && (st = run_lora_u(L, p.u_splits, up, stream)) != RQ_OK) return st;
  const LinearEpi e = make_epi(L, up, p.u_splits);
  if (L.x_dtype == RQ_DTYPE_BF16) st = run_gemv<RQ_DTYPE_BF16>(L, p, e, ws, stream);
  else st = run_gemv<RQ_DTYPE_F16>(L, p, e, ws, stream);
  if (st != RQ_OK || p.direct) return st;
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

extern "C" int rq_nf4_linear_workspace_size(int x_dtype, int64_t M, int64_t K, int64_t N, int64_t rank,
                                            int64_t* bytes) {
  if (!bytes) return RQ_ERR_NULL_POINTER;
  if (x_dtype != RQ_DTYPE_BF16 && x_dtype != RQ_DTYPE_F16) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || N < 1 || K < 64 || K % 64 || rank < 0 || rank > 256) return RQ_ERR_BAD_SHAPE;
  size_t b = 0;
  LinearArgs L{};
  L.x_dtype = x_dtype; L.M = M; L.K = K; L.N = N; L.rank = rank;
  int st = M <= kGemvMaxM ? gemv_workspace(L, &b) : gemm_workspace(L, &b);
  *bytes = int64_t(b);
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
  if (M <= kGemvMaxM) return run_nf4_gemv(L, workspace, size_t(workspace_bytes), stream);
  return run_nf4_gemm(L, workspace, size_t(workspace_bytes), stream);
}
