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
// segments) and visits 16-row tiles g, g + G, ...  Wave w always covers
// segment w of the split, so its activation operands stay in registers.
// Every load goes out as raw bits and is converted only where it is used,
// and every prefetch is unconditional (past the workgroup's last tile it
// reads one shared address), so the in-order load counter stays exact and
// the math of tile j runs while the next tile's loads are in flight.  Each
// tile ends with one barrier: the 16 partial tiles are summed in a fixed
// order through LDS (so results are deterministic) and finished from LDS --
// the tile's LoRA B rows and bias were fetched with its weights, one value
// per thread.
// ---------------------------------------------------------------------------
constexpr int kGemvThreads = 1024;
constexpr int kGemvWaves = kGemvThreads / 64;
constexpr int kSegK = 256;
constexpr int kGemvMaxFusedRank = kGemvThreads / 16;  // B values of a tile, one per thread
constexpr int kGemvMaxUSplits = 16;
constexpr int kGemvDepth = 2;  // tiles whose loads are in flight per wave

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

// tile < 0 marks a prefetch past the workgroup's last tile: every lane then
// reads one shared 16-byte address (and scale 0), which keeps the number of
// loads static -- so the in-order load counter stays exact across the loop --
// at the cost of a single cache line.
template <class Scale>
__device__ __forceinline__ void gemv_issue_tile(GemvTileLoads<Scale>& L, const GemvArgs& a, const Scale& scale,
                                                int64_t tile, const GemvLane& w) {
  if (tile < 0) {
    L.a = *reinterpret_cast<const u32x4*>(a.packed);
    L.b = L.a;
    L.s1 = scale.load(0);
    L.s2 = L.s1;
    return;
  }
  const int64_t half_k = a.K >> 1;
  const int64_t r0 = tile * 16;
  int64_t rowA = r0 + (w.n16 & 7), rowB = r0 + 8 + (w.n16 & 7), rowS = r0 + w.n16;
  rowA = rowA < a.N ? rowA : a.N - 1;  // dead rows re-read a live row; never stored
  rowB = rowB < a.N ? rowB : a.N - 1;
  rowS = rowS < a.N ? rowS : a.N - 1;
  const int cA = w.q + (w.n16 >= 8 ? 4 : 0), cB = w.q + (w.n16 < 8 ? 4 : 0);
  const int64_t sk = w.seg * kSegK;
  // chunks past K (a last, partial segment) re-read the row's last chunk
  int64_t kA = sk + 32 * cA, kB = sk + 32 * cB;
  kA = kA < a.K ? kA : a.K - 32;
  kB = kB < a.K ? kB : a.K - 32;
  L.a = *reinterpret_cast<const u32x4*>(a.packed + rowA * half_k + (kA >> 1));
  L.b = *reinterpret_cast<const u32x4*>(a.packed + rowB * half_k + (kB >> 1));
  int64_t k1 = sk + 32 * w.q, k2 = k1 + 128;
  k1 = k1 < a.K ? k1 : a.K - 1;
  k2 = k2 < a.K ? k2 : a.K - 1;
  L.s1 = scale.load(rowS * a.blocks_per_row + (k1 >> a.bs_log2));
  L.s2 = scale.load(rowS * a.blocks_per_row + (k2 >> a.bs_log2));
}

// LoRA B and bias of one tile as raw bits: thread t holds B[tile row t / 64,
// t % 64] (rank <= 64) and, for t < 16, bias[tile row t].
struct GemvEpiLoads {
  Raw16x2 lb, bias;
};

__device__ __forceinline__ void gemv_issue_epi(GemvEpiLoads& E, const GemvArgs& a, const LinearEpi& e,
                                               int64_t tile, int tid) {
  // always the same loads: without LoRA or bias, or past the last tile, they
  // read x[0] instead
  const bool past = tile < 0;
  tile = past ? 0 : tile;
  int64_t bn = tile * 16 + (tid >> 6);
  bn = bn < a.N ? bn : a.N - 1;
  const int j = tid & 63;
  const bool has_b = e.rank > 0 && !past;
  E.lb = load_raw(has_b ? e.lora_b : static_cast<const void*>(a.x),
                  has_b ? bn * e.ld_lora_b + (j < e.rank ? j : 0) : 0, has_b ? e.lora_dt : RQ_DTYPE_BF16);
  int64_t cn = tile * 16 + (tid & 15);
  cn = cn < a.N ? cn : a.N - 1;
  const bool has_bias = e.bias != nullptr && !past;
  E.bias = load_raw(has_bias ? e.bias : static_cast<const void*>(a.x), has_bias ? cn : 0,
                    has_bias ? e.bias_dt : RQ_DTYPE_BF16);
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

// LDS staging of one tile: 16 wave partials [16][16 m][16 n], RND(B)
// [16][rank], RND(bias) [16].
struct GemvStage {
  float* part;
  float* lb;
  float* bias;
};

template <int XT>
__device__ __forceinline__ void gemv_publish(const f32x4& acc, const GemvEpiLoads& E, const GemvStage& st,
                                             const GemvArgs& a, const LinearEpi& e, int wave, int q, int n16,
                                             int tid) {
#pragma unroll
  for (int r = 0; r < 4; ++r) st.part[(wave * 16 + 4 * q + r) * 16 + n16] = acc[r];
  if (a.direct) {
    const int j = tid & 63;
    if (j < e.rank) st.lb[(tid >> 6) * e.rank + j] = round_x<XT>(raw_to_f32(E.lb, e.lora_dt));
    if (tid < 16) st.bias[tid] = e.bias ? round_x<XT>(raw_to_f32(E.bias, e.bias_dt)) : 0.0f;
  }
}

template <int XT>
__device__ __forceinline__ void gemv_finish(const GemvArgs& a, const LinearEpi& e, const GemvStage& st,
                                            const float* us, int64_t tile, int s, int tid) {
  if (tid >= 256) return;
  const int m = tid >> 4, nn = tid & 15;
  const int64_t n = tile * 16 + nn;
  if (m >= a.M || n >= a.N) return;
  float p[kGemvWaves];
#pragma unroll
  for (int w = 0; w < kGemvWaves; ++w) p[w] = st.part[(w * 16 + m) * 16 + nn];
  float v = 0.0f;
#pragma unroll
  for (int w = 0; w < kGemvWaves; ++w) v = __fadd_rn(v, p[w]);
  if (!a.direct) {
    a.ws[(int64_t(s) * a.M + m) * a.N + n] = v;
    return;
  }
  if (e.bias) v = __fadd_rn(v, st.bias[nn]);
  v = round_x<XT>(v);
  if (e.rank > 0) {
    float l = 0.0f;
    for (int j0 = 0; j0 < e.rank; j0 += 8) {
      float uu[8], bb[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const bool ok = j0 + jj < e.rank;
        uu[jj] = ok ? us[m * e.rank + j0 + jj] : 0.0f;
        bb[jj] = ok ? st.lb[nn * e.rank + j0 + jj] : 0.0f;
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) l = __fmaf_rn(uu[jj], bb[jj], l);
    }
    l = round_x<XT>(__fmul_rn(round_x<XT>(l), e.scaling));
    v = round_x<XT>(__fadd_rn(v, l));
  }
  static_cast<uint16_t*>(e.y)[m * e.ldy + n] = uint16_t(to_x16<XT>(v));
}

template <int XT, class Scale>
__global__ __launch_bounds__(kGemvThreads) void nf4_gemv_kernel(GemvArgs a, Scale scale, LinearEpi e) {
  // The table is the kernel's only static LDS array, so it sits at address
  // 0 and every lookup's base folds into the instruction's offset field.
  __shared__ u32x2 lut[kF32PairLutQwords];
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int rank = (a.direct && e.rank > 0) ? e.rank : 0;  // LoRA staging only when fused here
  // dynamic LDS: 2 tile stages, then RND(u)
  const int stage_floats = kGemvWaves * 256 + 16 * rank + 16;
  GemvStage st[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float* base = reinterpret_cast<float*>(smem) + i * stage_floats;
    st[i] = GemvStage{base, base + kGemvWaves * 256, base + kGemvWaves * 256 + 16 * rank};
  }
  float* us = reinterpret_cast<float*>(smem) + 2 * stage_floats;  // [16][rank]

  GemvLane w;
  w.n16 = lane & 15;
  w.q = lane >> 4;
  const int s = blockIdx.y;
  const int64_t nsegs = (a.K + kSegK - 1) / kSegK;
  const int64_t sg0 = (nsegs * s) / a.S, sg1 = (nsegs * (s + 1)) / a.S;
  w.live = sg0 + wave < sg1;
  w.seg = w.live ? sg0 + wave : sg0;  // a wave without a segment re-reads one; its activations are zero
  const int64_t n_tiles = (a.N + 15) / 16;
  const int64_t step = gridDim.x;
  const int64_t first = blockIdx.x;
  const int64_t n_mine = first < n_tiles ? (n_tiles - 1 - first) / step + 1 : 0;
  auto tile_at = [&](int64_t j) -> int64_t { return j < n_mine ? first + j * step : -1; };
  if (n_mine == 0) return;

  // 1. activation operands (stationary): step st -> k = seg * 256 + 128
  //    (st / 4) + 32 q + 8 (st % 4); zero past M, past K and for a wave
  //    without a segment.  2. the RND(u) partials.  3. the first two tiles.
  u32x4 xraw[8];
  const bool mlive = w.n16 < a.M && w.live;
  {
    const uint16_t* xrow = a.x + (w.n16 < a.M ? w.n16 : 0) * a.ldx;
#pragma unroll
    for (int stp = 0; stp < 8; ++stp) {
      int64_t k = w.seg * kSegK + 128 * (stp >> 2) + 32 * w.q + 8 * (stp & 3);
      k = k < a.K ? k : 0;
      xraw[stp] = load_x8(xrow + k, a.xvec);
    }
  }
  // RND(u) partials: thread t < 16 rank sums u[split][t / rank][t % rank]
  // (every address clamped into the buffer, so the loads are unconditional)
  float up[kGemvMaxUSplits];
  const bool has_u = a.direct && rank > 0;
  {
    const int u_idx = (has_u && tid < 16 * rank) ? tid : 0;
    const int64_t u_m0 = has_u ? u_idx / rank : 0;
    const int64_t u_m = u_m0 < a.M ? u_m0 : a.M - 1;
    const int u_j = has_u ? u_idx % rank : 0;
#pragma unroll
    for (int k = 0; k < kGemvMaxUSplits; ++k) up[k] = 0.0f;
    if (has_u) {
#pragma unroll
      for (int k = 0; k < kGemvMaxUSplits; ++k) {
        const int kk = k < e.u_splits ? k : 0;
        up[k] = e.u[(int64_t(kk) * a.M + u_m) * rank + u_j];
      }
    }
  }
  constexpr int D = kGemvDepth;
  GemvTileLoads<Scale> buf[D];
  GemvEpiLoads ebuf[2];  // the epilogue values run two tiles ahead
#pragma unroll
  for (int i = 0; i < D; ++i) gemv_issue_tile(buf[i], a, scale, tile_at(i), w);
  gemv_issue_epi(ebuf[0], a, e, tile_at(0), tid);
  gemv_issue_epi(ebuf[1], a, e, tile_at(1), tid);

  u32x4 xa[8];
#pragma unroll
  for (int stp = 0; stp < 8; ++stp) {
    const int64_t k = w.seg * kSegK + 128 * (stp >> 2) + 32 * w.q + 8 * (stp & 3);
    xa[stp] = (mlive && k < a.K) ? xraw[stp] : u32x4{0u, 0u, 0u, 0u};
  }
  fill_f32pair_lut<kGemvThreads>(lut, tid);
  if (has_u && tid < 16 * rank) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kGemvMaxUSplits; ++k)
      if (k < e.u_splits) sum = __fadd_rn(sum, up[k]);
    us[tid] = (tid / rank) < a.M ? round_x<XT>(sum) : 0.0f;
  }
  __syncthreads();

  const uint32_t lane_off = uint32_t(lane & 31) * 8u;
  // D tiles per iteration so the ring index is static; the refill D tiles
  // ahead is unconditional
  for (int64_t j = 0; j < n_mine; j += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      if (j + i >= n_mine) break;
      const f32x4 acc = gemv_tile<XT>(buf[i], scale, xa, lut, lane_off, w.n16);
      gemv_issue_tile(buf[i], a, scale, tile_at(j + i + D), w);
      // consecutive tiles alternate LDS stages and epilogue buffers
      const GemvStage& sg = ((j + i) & 1) ? st[1] : st[0];
      GemvEpiLoads& eb = ((j + i) & 1) ? ebuf[1] : ebuf[0];
      gemv_publish<XT>(acc, eb, sg, a, e, wave, w.q, w.n16, tid);
      gemv_issue_epi(eb, a, e, tile_at(j + i + 2), tid);
      __syncthreads();
      gemv_finish<XT>(a, e, sg, us, tile_at(j + i), s, tid);
    }
  }
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
  int S = int((nsegs + kGemvWaves - 1) / kGemvWaves);
  while (S < 8 && tiles * S < cus && nsegs >= 2 * S * (kGemvWaves / 2)) S *= 2;
  p.S = S;
  p.u_splits = 0;
  if (rank > 0) {
    const int64_t steps_per_wg = 4 * kLoraUStepsPerWave;
    p.u_splits = int((K / 32 + steps_per_wg - 1) / steps_per_wg);
  }
  // the fused epilogue stages one B value per thread and sums <= 16 u splits
  p.direct = S == 1 && rank <= kGemvMaxFusedRank && p.u_splits <= kGemvMaxUSplits;
  const int64_t r = p.direct && rank > 0 ? rank : 0;
  // dynamic part only (the 64 KiB table is static): 2 tile stages + RND(u)
  p.lds_bytes = (size_t(2) * (kGemvWaves * 256 + 16 * r + 16) + 16 * r) * 4;
  int per_cu = int((160 * 1024) / (p.lds_bytes + size_t(kF32PairLutQwords) * 8));
  per_cu = per_cu < 1 ? 1 : per_cu;
  const int64_t slots = int64_t(cus) * per_cu / S;
  p.grid = int(tiles < slots ? tiles : (slots > 0 ? slots : 1));
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
  auto kern = nf4_gemv_kernel<XT, Scale>;
  static bool attr_set = false;  // one flag per instantiation
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024 - kF32PairLutQwords * 8) != hipSuccess)
      return RQ_ERR_HIP;
    attr_set = true;
  }
  dim3 grid(unsigned(p.grid), unsigned(p.S));
  kern<<<grid, kGemvThreads, p.lds_bytes, stream>>>(a, scale, e);
  return rq_check_launch();
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
