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
// that a producer policy dequantizes into LDS: Fwd8Producer writes W rows
// (output feature n, reduction k), Dx8Producer writes W^T rows (output
// feature k, reduction n) by dequantizing a 64 x 128 block of W and storing
// it transposed.  Below, "columns" are output features and "k" is the
// reduction index of the core.
//
// Workgroup tile 256 tokens x 128 features, 8 waves (two per SIMD); wave w
// owns rows 64 (w % 4) .. +63 and columns 64 (w / 4) .. +63 as 2 x 2 blocks
// of v_mfma_f32_32x32x16_{bf16,f16} (rq_gemm8.h).  K advances 64 per step --
// one NF4 block per weight row, one scale per row per step.  LDS (160 KiB,
// all of it):
//   [0, 64K)     the fp32 pair table for exact dequantization (address 0,
//                so lookups fold their base into the instruction offset);
//   [64K, 128K)  activation ring: 2 steps x 4 row slices x 64 rows x 128 bytes;
//   [128K, 160K) weight tiles: 2 steps x 128 rows x 128 bytes.
// The activation ring stores 16-byte chunk c of row r at slot c ^ ((r / 2) &
// 7) of the row, the weight tiles at slot c ^ (((r / 2) ^ r) & 7): for the
// MFMA operand reads (16 consecutive rows of one chunk) both put the rows on
// 16 distinct 16-byte bank groups (row parity picks the 128-byte half); the
// weight tile's also separates rows 2i and 2i + 1, whose chunks the
// dequantizer stores from adjacent lanes (with the first swizzle those
// stores met in the same banks).
//   * Activations go from global memory straight into the ring with
//     global_load_lds_dwordx4: each instruction moves 8 whole 128-byte rows
//     (8 cache lines; loads that spread 32 rows over one instruction cost the
//     vector L1 32 line lookups and stall the MFMA stream).  The two waves of
//     a row slice each load half of its rows.
//   * Packed weights and their scales sit in registers four steps ahead;
//     each step dequantizes the next step's tile through the pair table into
//     the other weight tile.
// Tiles are numbered so that the workgroups of one XCD (workgroup id mod 8)
// share activation row slices, which then stay in that XCD's L2, and their
// k loops start staggered so that only one of them misses on each slice.
#include "rq_gemm_core.h"
#include "rq_gemm8.h"
#include "rq_generic.h"

namespace rq {

// dX on the eight-wave core (512 threads): thread t dequantizes rows n = 64
// kstep + 2 (t % 32) + i (i = 0, 1: piece i) at layer columns col0 + 8 (t /
// 32) .. +8, and stores the 2 x 8 block transposed: for each of its 8 k, the
// pair {n, n + 1} as one 4-byte store.  32 consecutive lanes cover one k
// row's 64 n (128 bytes); the other 32 lanes of the wave (the next column
// group) store their rows in swapped pair order, so the two halves of a
// wave hit different row parities (bank halves).
template <int XT, class Scale>
struct Dx8Producer {
  // vector-memory loads issue() makes (the core's waits count them): two
  // weight words, and per row its scale loads -- or, transposed, rows n and
  // n + 1's scales as one 8-byte load (adjacent words, which the compiler
  // would merge into one load anyway)
  static constexpr int kLoads = Scale::kTransposed ? 3 : 2 * (1 + Scale::kLoads);
  // the epilogue's LoRA operands in registers (e.lora_regs): only beside the
  // transposed scales, which is where the host sets it
  static constexpr bool kLoraRegs = Scale::kTransposed;
  struct Regs {
    uint32_t w[2];
    typename Scale::Raw s[2];
  };
  struct Step {
    float sc[2];
    uint32_t taddr[2][4];
    u32x2 lk[2][4];
    float v[8];       // piece 0 products (row n), waiting for their partner
    uint32_t pr[8];   // {n, n + 1} pairs by k
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
    rg = uint32_t(tid & 31);
    dcol = uint32_t(tid >> 5);
    swap = dcol & 1u;
    const int64_t layer_k = P.row_bytes * 2;
    kcol = col0 + 8 * dcol;
    kcol = kcol < layer_k ? kcol : layer_k - 8;  // columns past K re-read live codes; never stored
    boff = uint32_t(kcol >> 1);
  }
  __device__ __forceinline__ void issue(Regs& R, int64_t kstep) const {
    const int64_t blk = kcol >> P.bs_log2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t n = kstep * kGemmBK + 2 * rg + i;
      R.w[i] = *reinterpret_cast<const uint32_t*>(P.packed + (uint32_t(n * P.row_bytes) + boff));
      if constexpr (!Scale::kTransposed) {
        R.s[i] = scale.load(n * P.blocks_per_row + blk);
        // one load per row's scale, as kLoads counts: with one block per row
        // (K == block size) the two rows' scales are adjacent words, which the
        // compiler would otherwise merge into one load
        asm volatile("" ::: "memory");
      }
    }
    if constexpr (Scale::kTransposed) {
      // rows n, n + 1 (n even, rows a multiple of 64): 8-byte aligned
      const u32x2 s2 = *reinterpret_cast<const u32x2*>(static_cast<const uint32_t*>(scale.p) + blk * P.rows +
                                                       kstep * kGemmBK + 2 * rg);
      R.s[0] = s2.x;
      R.s[1] = s2.y;
    }
  }
  __device__ __forceinline__ void prep(Step& S, const Regs& R) const {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      S.sc[i] = scale.value(R.s[i]);
#pragma unroll
      for (int h = 0; h < 4; ++h) S.taddr[i][h] = lut_addr(R.w[i], lane_off, h);
    }
  }
  __device__ __forceinline__ void lookup(Step& S, int p) const {
#pragma unroll
    for (int h = 0; h < 4; ++h) S.lk[p][h] = lut_read(lut, S.taddr[p][h]);
  }
  __device__ __forceinline__ void finish(Step& S, int p, int hh, uint8_t* tile) const {
#pragma unroll
    for (int h = 2 * hh; h < 2 * hh + 2; ++h) {
      const float a = __fmul_rn(u2f(S.lk[p][h].x), S.sc[p]);  // k = 2h
      const float b = __fmul_rn(u2f(S.lk[p][h].y), S.sc[p]);  // k = 2h + 1
      if (p == 0) {
        S.v[2 * h] = a;
        S.v[2 * h + 1] = b;
      } else {
        S.pr[2 * h] = cvt_pk<XT>(S.v[2 * h], a);
        S.pr[2 * h + 1] = cvt_pk<XT>(S.v[2 * h + 1], b);
      }
    }
    if (p == 1 && hh == 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // the values as rvalues: a conditional on the array elements would
        // select an address, and the array would live in scratch memory
        const uint32_t ke = uint32_t(e) ^ swap;
        const uint32_t own = S.pr[e], partner = S.pr[e ^ 1];
        const uint32_t val = swap ? partner : own;
        *reinterpret_cast<uint32_t*>(tile + swzw(8u * dcol + ke, rg >> 2) + ((rg & 3u) << 2)) = val;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
template <int XT, template <int, class> class ProdT, class Scale>
static int launch_core8(const GemmArgs& a, const ProducerParams& pp, Scale scale, const GemmEpi& e,
                        hipStream_t stream) {
  const int64_t T = int64_t(a.tiles_m) * a.tiles_n;
  const unsigned grid = unsigned(a.xcd_map ? 8 * (a.lf + (T / 8 - a.lf) * a.splits) : T);
  nf4_gemm8_kernel<XT, ProdT<XT, Scale>, Scale><<<grid, kGemm8Threads, 0, stream>>>(a, pp, scale, e);
  return rq_check_launch();
}

// The eight-wave core with producer ProdT, by scale format: absmax of its
// dtype, or double quantization (c2 codes of c2_format with c2_scales).
template <int XT, template <int, class> class ProdT>
static int run_core8(const GemmArgs& a, const ProducerParams& pp, const void* absmax, int absmax_dtype,
                     const uint8_t* c2, int c2_format, int64_t block2, const GemmEpi& e, hipStream_t stream) {
  if (c2) {
    const int sh = pow2_shift(block2);
    switch (absmax_dtype) {
      case RQ_DTYPE_F32:
        return launch_core8<XT, ProdT>(a, pp, ScaleDQ<RQ_DTYPE_F32>{c2, absmax, c2_format, sh, block2}, e, stream);
      case RQ_DTYPE_BF16:
        return launch_core8<XT, ProdT>(a, pp, ScaleDQ<RQ_DTYPE_BF16>{c2, absmax, c2_format, sh, block2}, e, stream);
      default:
        return launch_core8<XT, ProdT>(a, pp, ScaleDQ<RQ_DTYPE_F16>{c2, absmax, c2_format, sh, block2}, e, stream);
    }
  }
  switch (absmax_dtype) {
    case RQ_DTYPE_F32: return launch_core8<XT, ProdT>(a, pp, ScaleAbsmax<RQ_DTYPE_F32>{absmax}, e, stream);
    case RQ_DTYPE_BF16: return launch_core8<XT, ProdT>(a, pp, ScaleAbsmax<RQ_DTYPE_BF16>{absmax}, e, stream);
    default: return launch_core8<XT, ProdT>(a, pp, ScaleAbsmax<RQ_DTYPE_F16>{absmax}, e, stream);
  }
}

// The dX operands prepared by one launch before the GEMM, through 64 x 64
// LDS tiles (read along one index, written along the other):
//   st[b][n] = scale(n, b) as fp32, the value the producer computes from the
//     absmax (or from the c2 code and its super-block scale), so that a dX
//     step's scales are contiguous;
//   at[k][j] = RND(A[j][k]) in the activation dtype, rank16 columns (zeros
//     past the rank), when at != nullptr: the epilogue's LoRA operand A^T as
//     rows it reads 16 bytes at a time (A [rank][K] read directly is one
//     strided element per load).
// Workgroups [0, st_tiles) take scale tiles, the rest A tiles.
template <class Scale, int XT>
__global__ __launch_bounds__(1024) void dx_prep_kernel(Scale sc, int64_t rows, int64_t bpr, float* __restrict__ st,
                                                       const void* a, int a_dt, int64_t K, int rank, int rank16,
                                                       uint16_t* __restrict__ at) {
  __shared__ float tile[64][65];
  const int t = threadIdx.x, c = t & 63;
  const int64_t st_x = (rows + 63) / 64, st_tiles = st_x * ((bpr + 63) / 64);
  const int64_t g = blockIdx.x;
  if (g < st_tiles) {
    const int64_t n0 = (g % st_x) * 64, b0 = (g / st_x) * 64;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = n0 + (t >> 6) + 16 * i, b = b0 + c;
      v[i] = (n < rows && b < bpr) ? sc(n * bpr + b) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) tile[(t >> 6) + 16 * i][c] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (t >> 6) + 16 * i;
      const int64_t b = b0 + r, n = n0 + c;
      if (b < bpr && n < rows) st[b * rows + n] = tile[c][r];
    }
    return;
  }
  const int64_t at_x = (K + 63) / 64, ga = g - st_tiles;
  const int64_t k0 = (ga % at_x) * 64, j0 = (ga / at_x) * 64;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t j = j0 + (t >> 6) + 16 * i, k = k0 + c;
    v[i] = (j < rank && k < K) ? load_as_f32(a, j * K + k, a_dt) : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) tile[(t >> 6) + 16 * i][c] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (t >> 6) + 16 * i;
    const int64_t k = k0 + r, j = j0 + c;
    if (k < K && j < rank16) at[k * rank16 + j] = uint16_t(to_x16<XT>(tile[c][r]));
  }
}

template <class Scale>
static int launch_dx_prep(const DxArgs& D, Scale sc, int64_t bpr, float* st, int rank16, uint16_t* at,
                          hipStream_t stream) {
  const int64_t tiles = ((D.N + 63) / 64) * ((bpr + 63) / 64) + (at ? ((D.K + 63) / 64) * ((rank16 + 63) / 64) : 0);
  const int r = at ? int(D.rank) : 0;
  if (D.dy_dtype == RQ_DTYPE_BF16)
    dx_prep_kernel<Scale, RQ_DTYPE_BF16><<<unsigned(tiles), 1024, 0, stream>>>(sc, D.N, bpr, st, D.lora_a,
                                                                              D.lora_dtype, D.K, r, rank16, at);
  else
    dx_prep_kernel<Scale, RQ_DTYPE_F16><<<unsigned(tiles), 1024, 0, stream>>>(sc, D.N, bpr, st, D.lora_a,
                                                                             D.lora_dtype, D.K, r, rank16, at);
  return rq_check_launch();
}

// The transposed scales of a dX call, by scale format (and RND(A)^T when at
// is given).
static int run_dx_prep(const DxArgs& D, float* st, int rank16, uint16_t* at, hipStream_t stream) {
  const int64_t bpr = D.K / D.block_size;
  if (D.c2) {
    const int sh = pow2_shift(D.block2);
    switch (D.absmax_dtype) {
      case RQ_DTYPE_F32:
        return launch_dx_prep(D, ScaleDQ<RQ_DTYPE_F32>{D.c2, D.absmax, D.c2_format, sh, D.block2}, bpr, st, rank16, at,
                              stream);
      case RQ_DTYPE_BF16:
        return launch_dx_prep(D, ScaleDQ<RQ_DTYPE_BF16>{D.c2, D.absmax, D.c2_format, sh, D.block2}, bpr, st, rank16,
                              at, stream);
      default:
        return launch_dx_prep(D, ScaleDQ<RQ_DTYPE_F16>{D.c2, D.absmax, D.c2_format, sh, D.block2}, bpr, st, rank16, at,
                              stream);
    }
  }
  switch (D.absmax_dtype) {
    case RQ_DTYPE_F32: return launch_dx_prep(D, ScaleAbsmax<RQ_DTYPE_F32>{D.absmax}, bpr, st, rank16, at, stream);
    case RQ_DTYPE_BF16: return launch_dx_prep(D, ScaleAbsmax<RQ_DTYPE_BF16>{D.absmax}, bpr, st, rank16, at, stream);
    default: return launch_dx_prep(D, ScaleAbsmax<RQ_DTYPE_F16>{D.absmax}, bpr, st, rank16, at, stream);
  }
}

// Bytes of the transposed scales (at most K / 64 blocks per row: the MFMA dX
// kernel takes block sizes of at least 64), 256-byte padded.
static size_t dx_scale_t_bytes(int64_t N, int64_t K, int64_t block_size) {
  return (size_t(N) * size_t(K / block_size) * 4 + 255) & ~size_t(255);
}
// Bytes of RND(A)^T [K][rank16] in a 16-bit dtype, 256-byte padded.
static size_t dx_at_bytes(int64_t K, int64_t rank16) { return (size_t(K) * size_t(rank16) * 2 + 255) & ~size_t(255); }

int gemm_workspace(const LinearArgs& L, size_t* bytes) {
  *bytes = plan_gemm(L.M, L.N, L.K, L.rank, device_cus(), true).ws_bytes;
  return RQ_OK;
}

size_t gemm_min_workspace(const LinearArgs& L) {
  return plan_gemm(L.M, L.N, L.K, L.rank, device_cus(), false).ws_bytes;
}

int run_nf4_gemm(const LinearArgs& L, void* workspace, size_t ws_bytes, uint32_t* tile_cnt, size_t n_cnt,
                 hipStream_t stream) {
  // the activation operands are loaded 16 bytes at a time
  if (!aligned(L.x, 16) || L.ldx % 8 != 0) return RQ_ERR_BAD_ALIGNMENT;
  if (!offsets_fit(L.M, L.ldx, L.N, L.K)) return RQ_ERR_UNSUPPORTED;
  // K splits need the zeroed tile counts and room for their partial tiles;
  // without them the GEMM runs unsplit
  GemmPlan p = plan_gemm(L.M, L.N, L.K, L.rank, device_cus(), true);
  if (p.splits > 1 && (!tile_cnt || size_t(8) * p.lt > n_cnt || !workspace || ws_bytes < p.ws_bytes))
    p = plan_gemm(L.M, L.N, L.K, L.rank, device_cus(), false);
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
    // u = RND(xl . RND(A)^T), A [r][K] row-major (lora_layer.py:67)
    int st = run_lora_rows(L.x_dtype, static_cast<const uint16_t*>(L.lora_x), L.ld_lora_x, L.M, L.K, L.lora_a,
                           L.lora_dtype, L.K, 1, e.rank, false, 1.0f, p.lr, reinterpret_cast<float*>(ws), u16,
                           p.rank16, stream);
    if (st != RQ_OK) return st;
    // RND(B), B [N][r] with row stride ld_lora_b, rounded as the epilogue stages it
    e.u = u16;
    e.braw = L.lora_b;
    e.b_dt = L.lora_dtype;
    e.b_sn = L.ld_lora_b;
    e.b_sj = 1;
    e.b_vec = aligned(L.lora_b, 16) && (L.lora_dtype != RQ_DTYPE_F32 || L.ld_lora_b % 4 == 0);
    e.lora_regs = p.rank16 <= 64 && e.rank % 8 == 0 && aligned(L.lora_b, 16) &&
                  L.ld_lora_b % (L.lora_dtype == RQ_DTYPE_F32 ? 4 : 8) == 0;
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
  a.splits = p.splits;
  a.lf = p.lf;
  a.part = p.splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.part_offset) : nullptr;
  a.tile_cnt = tile_cnt;
  ProducerParams pp{L.w_packed, L.K / 2, L.N, L.K / L.block_size, pow2_shift(L.block_size)};
  if (L.x_dtype == RQ_DTYPE_BF16)
    return run_core8<RQ_DTYPE_BF16, Fwd8Producer>(a, pp, L.absmax, L.absmax_dtype, L.c2, L.c2_format, L.block2, e,
                                                  stream);
  return run_core8<RQ_DTYPE_F16, Fwd8Producer>(a, pp, L.absmax, L.absmax_dtype, L.c2, L.c2_format, L.block2, e,
                                               stream);
}

// ---------------------------------------------------------------------------
// dX = dY . W_deq (+ LoRA): the core with activations dY [M][N], output
// columns k of the layer, reduction over the layer's N.
// ---------------------------------------------------------------------------
int validate_dx(const DxArgs& D) {
  if (!D.dy || !D.w_packed || !D.absmax || !D.dx) return RQ_ERR_NULL_POINTER;
  if (!valid_float_dtype(D.dy_dtype)) return RQ_ERR_BAD_DTYPE;
  if (D.absmax_dtype != RQ_DTYPE_F32 && D.absmax_dtype != RQ_DTYPE_BF16 && D.absmax_dtype != RQ_DTYPE_F16)
    return RQ_ERR_BAD_DTYPE;
  if (D.M < 0 || D.N <= 0 || D.K <= 0 || D.block_size < 1) return RQ_ERR_BAD_SHAPE;
  if (D.lddy < D.N || D.lddx < D.K) return RQ_ERR_BAD_SHAPE;
  if (D.c2 && (D.block2 <= 0 || (D.c2_format != RQ_C2_FP8_E4M3FNUZ && D.c2_format != RQ_C2_INT8)))
    return RQ_ERR_BAD_SHAPE;
  if (!aligned(D.dy, dtype_size(D.dy_dtype)) || !aligned(D.dx, dtype_size(D.dy_dtype))) return RQ_ERR_BAD_ALIGNMENT;
  if (D.rank > 0) {
    if (!D.lora_a || !D.lora_b) return RQ_ERR_NULL_POINTER;
    if (D.rank > 256 || D.ld_lora_b < D.rank) return RQ_ERR_BAD_SHAPE;
    // fp32 (the trainable parameters) or dY's dtype; with fp32 dY any float
    // dtype (widened exactly, as B.to(dy.dtype) does)
    if (D.lora_dtype != RQ_DTYPE_F32 && D.lora_dtype != D.dy_dtype &&
        !(D.dy_dtype == RQ_DTYPE_F32 && valid_float_dtype(D.lora_dtype)))
      return RQ_ERR_BAD_DTYPE;
    if (D.lora_mask && D.ld_lora_mask < D.K) return RQ_ERR_BAD_SHAPE;
  }
  return RQ_OK;
}

// Whether the MFMA dX kernel takes the call: 16-bit dY read 16 bytes at a
// time, N and K multiples of 64, a power-of-two block size of at least 64
// dividing K, 32-bit offsets; every other valid call runs on the generic
// kernels.
bool dx_fast_ok(const DxArgs& D) {
  if (D.dy_dtype != RQ_DTYPE_BF16 && D.dy_dtype != RQ_DTYPE_F16) return false;
  if (D.N % 64 != 0 || D.K % 64 != 0 || D.block_size < 64 || (D.block_size & (D.block_size - 1)) != 0 ||
      D.K % D.block_size != 0)
    return false;
  if (!aligned(D.dy, 16) || D.lddy % 8 != 0 || !aligned(D.w_packed, 4)) return false;
  return offsets_fit(D.M, D.lddy, D.N, D.K);
}

int dx_workspace(const DxArgs& D, size_t* bytes) {
  // the larger of the MFMA kernel's and the generic kernels' (the operands'
  // alignment and the block size, unknown here, decide which runs)
  const size_t g = generic_lora_bytes(D.dy_dtype, D.M, D.rank);
  const bool fast = D.dy_dtype != RQ_DTYPE_F32 && D.N % 64 == 0 && D.K % 64 == 0;
  const size_t core = (plan_gemm(D.M, D.K, D.N, D.rank > 0 ? D.rank : 0, device_cus()).ws_bytes + 255) & ~size_t(255);
  const int64_t r16 = D.rank > 0 ? (D.rank + 15) & ~int64_t(15) : 0;
  *bytes = std::max(g, fast ? core + dx_scale_t_bytes(D.N, D.K, 64) + (r16 ? dx_at_bytes(D.K, r16) : 0) : size_t(0));
  return RQ_OK;
}

int run_nf4_dx(const DxArgs& D, void* workspace, size_t ws_bytes, hipStream_t stream) {
  int st = validate_dx(D);
  if (st != RQ_OK) return st;
  if (D.M == 0) return RQ_OK;
  if (!dx_fast_ok(D)) return run_generic_nf4_dx(D, workspace, ws_bytes, stream);
  const int64_t rank = D.rank > 0 ? D.rank : 0;
  const GemmPlan p = plan_gemm(D.M, D.K, D.N, rank, device_cus());
  if (p.ws_bytes > 0 && (!workspace || ws_bytes < p.ws_bytes)) return RQ_ERR_WORKSPACE;
  if (workspace && !aligned(workspace, 256)) return RQ_ERR_BAD_ALIGNMENT;
  GemmEpi e{};
  e.rank = int(rank);
  e.rank16 = p.rank16;
  e.scaling = 1.0f;
  e.mask = rank > 0 ? D.lora_mask : nullptr;
  e.ldm = D.ld_lora_mask;
  e.mask_scale = D.mask_scale;
  e.y = static_cast<uint16_t*>(D.dx);
  e.ldy = D.lddx;
  if (rank > 0) {
    char* ws = static_cast<char*>(workspace);
    uint16_t* g16 = reinterpret_cast<uint16_t*>(ws + p.u16_offset);
    // g = RND(RND(dY * s) . RND(B)): S[j][n] = B[n][j]
    st = run_lora_rows(D.dy_dtype, static_cast<const uint16_t*>(D.dy), D.lddy, D.M, D.N, D.lora_b, D.lora_dtype, 1,
                       D.ld_lora_b, int(rank), true, D.scaling, p.lr, reinterpret_cast<float*>(ws), g16, p.rank16,
                       stream);
    if (st != RQ_OK) return st;
    // RND(A^T) [K][r]: element (k, j) = A[j][k], A [r][K] row-major, rounded
    // as the epilogue stages it
    e.u = g16;
    e.braw = D.lora_a;
    e.b_dt = D.lora_dtype;
    e.b_sn = 1;
    e.b_sj = D.K;
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
  a.splits = 1;
  a.lf = p.tiles_m * p.tiles_n / 8;
  ProducerParams pp{D.w_packed, D.K / 2, D.N, D.K / D.block_size, pow2_shift(D.block_size)};
  // With room in the workspace, the scales are decoded and transposed first
  // (one small launch), so that a step's scales are contiguous: at the
  // Llama-3-8B gate shape the scattered per-row scale reads kept the
  // texture addresser 65 % busy and made the dX 12-17 % slower.  The same
  // launch writes RND(A)^T in the activation dtype when there is room for it
  // too, the epilogue's LoRA operand as 16-byte rows.
  const size_t st_off = (p.ws_bytes + 255) & ~size_t(255);
  const size_t st_bytes = dx_scale_t_bytes(D.N, D.K, D.block_size);
  if (workspace && ws_bytes >= st_off + st_bytes) {
    char* ws = static_cast<char*>(workspace);
    float* st = reinterpret_cast<float*>(ws + st_off);
    uint16_t* at = nullptr;
    if (rank > 0 && ws_bytes >= st_off + st_bytes + dx_at_bytes(D.K, p.rank16)) {
      at = reinterpret_cast<uint16_t*>(ws + st_off + st_bytes);
      e.braw = at;
      e.b_dt = D.dy_dtype;
      e.b_sn = p.rank16;
      e.b_sj = 1;
      e.b_vec = true;
      e.lora_regs = p.rank16 <= 64 && rank % 8 == 0;
    }
    if (const int s2 = run_dx_prep(D, st, p.rank16, at, stream); s2 != RQ_OK) return s2;
    const ScaleT sct{st};
    if (D.dy_dtype == RQ_DTYPE_BF16) return launch_core8<RQ_DTYPE_BF16, Dx8Producer>(a, pp, sct, e, stream);
    return launch_core8<RQ_DTYPE_F16, Dx8Producer>(a, pp, sct, e, stream);
  }
  if (D.dy_dtype == RQ_DTYPE_BF16)
    return run_core8<RQ_DTYPE_BF16, Dx8Producer>(a, pp, D.absmax, D.absmax_dtype, D.c2, D.c2_format, D.block2, e,
                                                 stream);
  return run_core8<RQ_DTYPE_F16, Dx8Producer>(a, pp, D.absmax, D.absmax_dtype, D.c2, D.c2_format, D.block2, e,
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
                               int64_t rank, float scaling, const uint8_t* lora_mask, int64_t ld_lora_mask,
                               float mask_scale, void* dx, int64_t lddx) {
  rq::DxArgs D;
  D.dy = dy; D.dy_dtype = dy_dtype; D.M = M; D.N = N; D.lddy = lddy;
  D.w_packed = w_packed; D.K = K; D.block_size = block_size;
  D.absmax = absmax; D.absmax_dtype = absmax_dtype; D.c2 = c2; D.c2_format = c2_format; D.block2 = block2;
  D.lora_a = lora_a; D.lora_b = lora_b; D.ld_lora_b = ld_lora_b; D.lora_dtype = lora_dtype;
  D.rank = (lora_a && lora_b) ? rank : 0; D.scaling = scaling;
  D.lora_mask = lora_mask; D.ld_lora_mask = ld_lora_mask; D.mask_scale = mask_scale;
  D.dx = dx; D.lddx = lddx;
  return D;
}

extern "C" int rq_nf4_linear_dx_workspace_size(int dy_dtype, int64_t M, int64_t N, int64_t K, int64_t rank,
                                               int64_t* bytes) {
  if (!bytes) return RQ_ERR_NULL_POINTER;
  if (!rq::valid_float_dtype(dy_dtype)) return RQ_ERR_BAD_DTYPE;
  if (M < 0 || N <= 0 || K <= 0 || rank < 0) return RQ_ERR_BAD_SHAPE;
  rq::DxArgs D{};
  D.dy_dtype = dy_dtype; D.M = M; D.N = N; D.K = K; D.rank = rank;
  size_t b = 0;
  const int st = rq::dx_workspace(D, &b);
  *bytes = int64_t(b);
  return st;
}

extern "C" int rq_nf4_linear_dx(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t lddy,
                                const uint8_t* w_packed, int64_t K, int64_t block_size, const void* absmax,
                                int absmax_dtype, const uint8_t* c2, int c2_format, int64_t block2,
                                const void* lora_a, const void* lora_b, int64_t ld_lora_b, int lora_dtype,
                                int64_t rank, float scaling, const uint8_t* lora_mask, int64_t ld_lora_mask,
                                float mask_scale, void* dx, int64_t lddx, void* workspace,
                                int64_t workspace_bytes, hipStream_t stream) {
  const rq::DxArgs D = pack_dx_args(dy, dy_dtype, M, N, lddy, w_packed, K, block_size, absmax, absmax_dtype, c2,
                                    c2_format, block2, lora_a, lora_b, ld_lora_b, lora_dtype, rank, scaling,
                                    lora_mask, ld_lora_mask, mask_scale, dx, lddx);
  return rq::run_nf4_dx(D, workspace, workspace_bytes < 0 ? 0 : size_t(workspace_bytes), stream);
}

extern "C" int rq_gemm_tile_config(int32_t* out) {
  if (!out) return RQ_ERR_NULL_POINTER;
  out[0] = rq::kGemmBM;
  out[1] = rq::kGemmBN;
  out[2] = rq::kGemmBK;
  out[3] = rq::kGemm8Threads / 64;  // wavefronts per workgroup
  out[4] = 2;                       // weight / activation tiles in flight in LDS (double buffered)
  return RQ_OK;
}
