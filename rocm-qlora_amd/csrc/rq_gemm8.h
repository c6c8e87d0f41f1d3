// The NF4/byte-weight MFMA GEMM kernel for gfx950 (forward GEMM, dX, INT8 /
// FP8 linears, by producer policy): 256 x 128 workgroup tiles, 64-k steps,
// 512 threads, two waves per SIMD.  Wave w owns rows 64 (w % 4) .. +63 and
// columns 64 (w / 4) .. +63 of the tile as 2 x 2 blocks of
// v_mfma_f32_32x32x16_{bf16,f16} (weights as the A operand, activations as
// B, so that a lane's results lie along an output row).  With one wave per
// SIMD (a 64 x 128 block each) the matrix core waited whenever that wave
// waited (LDS reads, table lookups, barrier); a second wave per SIMD issues
// its MFMAs in those gaps.
//
// The two waves of a row slice (w and w + 4) each bring half of the slice's
// activation rows into the ring; the step barrier, which already waits for
// every wave's activation loads, makes both halves visible to both.
#pragma once

#include "rq_gemm_core.h"

namespace rq {

constexpr int kGemm8Threads = 512;
constexpr int kGemm8MB = 2;  // 32-row blocks per wave
constexpr int kGemm8NB = 2;  // 32-column blocks per wave

// Forward producer for 512 threads: thread t dequantizes tile row t / 4,
// codes 16 (t % 4) .. +16 of the step (8 packed bytes, 2 pieces of 8 codes).
// A wave's 16-byte stores cover 16 rows, 4 chunks each; with the tile
// swizzle any 16 consecutive lanes hit 16 distinct 16-byte bank groups.
template <int XT, class Scale>
struct Fwd8Producer {
  static constexpr int kLoads = 1 + Scale::kLoads;
  static constexpr bool kLoraRegs = true;  // takes e.lora_regs (see GemmEpi)
  struct Regs {
    u32x2 w;
    typename Scale::Raw s;
  };
  struct Step {
    float sc;
    uint32_t taddr[2][4];
    u32x2 lk[2][4];
    uint32_t r[4];
  };
  ProducerParams P;
  Scale scale;
  const u32x2* lut;
  uint32_t lane_off, tile_row, quarter, wrow;
  int64_t wn;

  __device__ __forceinline__ void init(const ProducerParams& p, const Scale& sc, const u32x2* l, int tid,
                                       int64_t col0) {
    P = p;
    scale = sc;
    lut = l;
    lane_off = uint32_t(tid & 31) * 8u;
    tile_row = uint32_t(tid >> 2);
    quarter = uint32_t(tid & 3);
    wn = col0 + tile_row;
    wn = wn < P.rows ? wn : P.rows - 1;  // rows past N re-read a live row; never stored
    wrow = uint32_t(wn * P.row_bytes + 8 * quarter);  // the host keeps the weights under 4 GiB
  }
  __device__ __forceinline__ void issue(Regs& R, int64_t kstep) const {
    R.w = *reinterpret_cast<const u32x2*>(P.packed + (wrow + uint32_t(kstep) * 32u));
    R.s = scale.load(wn * P.blocks_per_row + ((kstep * kGemmBK) >> P.bs_log2));
  }
  __device__ __forceinline__ void prep(Step& S, const Regs& R) const {
    S.sc = scale.value(R.s);
    const uint32_t words[2] = {R.w.x, R.w.y};
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int h = 0; h < 4; ++h) S.taddr[p][h] = lut_addr(words[p], lane_off, h);
  }
  __device__ __forceinline__ void lookup(Step& S, int p) const {
#pragma unroll
    for (int h = 0; h < 4; ++h) S.lk[p][h] = lut_read(lut, S.taddr[p][h]);
  }
  __device__ __forceinline__ void finish(Step& S, int p, int hh, uint8_t* tile) const {
#pragma unroll
    for (int h = 2 * hh; h < 2 * hh + 2; ++h)
      S.r[h] = cvt_pk<XT>(__fmul_rn(u2f(S.lk[p][h].x), S.sc), __fmul_rn(u2f(S.lk[p][h].y), S.sc));
    if (hh == 1)
      *reinterpret_cast<u32x4*>(tile + swzw(tile_row, 2u * quarter + uint32_t(p))) =
          u32x4{S.r[0], S.r[1], S.r[2], S.r[3]};
  }
};

// One 64-k step of a wave's 64 x 64 block.  Sub-step s (k = 16 s + 8 q + e)
// runs four MFMAs; between them: the operand reads of sub-step s + 1, this
// wave's four direct-to-LDS activation loads of step j + 1 (s = 0, 1), the
// table lookups of the next weight tile's two pieces (s = 0, 1) and their
// scale-multiply, rounding and stores (s = 1, 2); after the last sub-step,
// the packed weights of step j + 4.
template <int XT, class Prod>
__device__ __forceinline__ void gemm8_step(f32x16 (&acc)[kGemm8MB][kGemm8NB], const uint8_t* xr,
                                           const uint8_t* wt, int i32, int q, uint32_t col_base,
                                           const GemmArgs& a, const uint32_t (&xo)[4], int64_t kx, uint32_t xdst,
                                           const Prod& prod, const typename Prod::Regs& wq,
                                           typename Prod::Regs& wl_fill, int64_t kfill, uint8_t* wdst) {
  typename Prod::Step S;
  prod.prep(S, wq);
  auto read_ops = [&](u32x4 (&xa)[kGemm8MB], u32x4 (&b)[kGemm8NB], int s) {
    const uint32_t c = uint32_t(2 * s + q);
#pragma unroll
    for (int mb = 0; mb < kGemm8MB; ++mb)
      xa[mb] = *reinterpret_cast<const u32x4*>(xr + swz(uint32_t(32 * mb + i32), c));
#pragma unroll
    for (int nb = 0; nb < kGemm8NB; ++nb)
      b[nb] = *reinterpret_cast<const u32x4*>(wt + swzw(col_base + uint32_t(32 * nb + i32), c));
  };
  u32x4 xa[kGemm8MB], b[kGemm8NB], xan[kGemm8MB], bn[kGemm8NB];
  read_ops(xa, b, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s < 3) read_ops(xan, bn, s + 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kGemm8MB * kGemm8NB; ++i) {
      const int nb = i / kGemm8MB, mb = i % kGemm8MB;
      acc[mb][nb] = mfma32x32x16<XT>(b[nb], xa[mb], acc[mb][nb]);
      if (i == 0 && s < 2) {
#pragma unroll
        for (int t = 2 * s; t < 2 * s + 2; ++t) dma16(a.x, (xo[t] + uint32_t(kx) * kGemmBK) * 2u, xdst + t * 1024);
      } else if (i == 1 && s < 2) {
        prod.lookup(S, s);
      } else if (i >= 2 && (s == 1 || s == 2)) {
        prod.finish(S, s - 1, i - 2, wdst);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (s < 3) {
#pragma unroll
      for (int mb = 0; mb < kGemm8MB; ++mb) xa[mb] = xan[mb];
#pragma unroll
      for (int nb = 0; nb < kGemm8NB; ++nb) b[nb] = bn[nb];
    }
  }
  prod.issue(wl_fill, kfill);
  __builtin_amdgcn_sched_barrier(0);
}

// The output values of a wave's 64 x 64 block, rounded to the operand
// dtype and packed two per dword (pk[mb][nb][h] = columns 8 h + 4 q .. + 3 of
// row m of block (mb, nb)): y = RND(RND(acc + RND(bias)) + RND(RND(lo) * s))
// with s the LoRA scaling (kMode 1), or mask ? mask_scale : 0 for dX with
// LoRA dropout (kMode 2); kMode 0 has no LoRA term.  bias is -0.0 where
// there is none (x + -0.0 == x for every x).  The flags are template
// parameters so the 64 values per lane run without a branch.
template <int XT, int kMode>
__device__ __forceinline__ void gemm8_outputs(const f32x16 (&acc)[kGemm8MB][kGemm8NB],
                                              const f32x16 (&lo)[kGemm8MB][kGemm8NB],
                                              const float (&bias)[kGemm8NB][4][4], const GemmEpi& e,
                                              const GemmArgs& a, int64_t m_lane, int64_t n_lane,
                                              uint32_t (&pk)[kGemm8MB][kGemm8NB][4][2]) {
#pragma unroll
  for (int mb = 0; mb < kGemm8MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kGemm8NB; ++nb)
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = __fadd_rn(acc[mb][nb][4 * h + c], bias[nb][h][c]);
        if constexpr (kMode > 0) {
          round2<XT>(v[0], v[1]);
          round2<XT>(v[2], v[3]);
          float l[4], s[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            l[c] = lo[mb][nb][4 * h + c];
            s[c] = e.scaling;
          }
          if constexpr (kMode == 2) {
            const int64_t m = m_lane + 32 * mb, n = n_lane + 32 * nb + 8 * h;
#pragma unroll
            for (int c = 0; c < 4; ++c)
              s[c] = m < a.M && n + c < a.N && e.mask[m * e.ldm + n + c] ? e.mask_scale : 0.0f;
          }
          round2<XT>(l[0], l[1]);
          round2<XT>(l[2], l[3]);
#pragma unroll
          for (int c = 0; c < 4; ++c) l[c] = __fmul_rn(l[c], s[c]);
          round2<XT>(l[0], l[1]);
          round2<XT>(l[2], l[3]);
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] = __fadd_rn(v[c], l[c]);
        }
        pk[mb][nb][h][0] = cvt_pk<XT>(v[0], v[1]);
        pk[mb][nb][h][1] = cvt_pk<XT>(v[2], v[3]);
      }
}

// Per-wave output staging of the epilogue: a 64 x 64 block of 16-bit values,
// 144-byte rows, in the LDS the activation ring and weight tiles use.
constexpr int kGemm8EpiPitch = 144;
constexpr int kGemm8EpiWaveBytes = 64 * kGemm8EpiPitch;
constexpr int kGemm8EpiOff = kXRingOff;
static_assert(kGemm8EpiOff + 8 * kGemm8EpiWaveBytes <= kGemmLds, "epilogue staging");

template <int XT, class Prod, class Scale>
__global__ __launch_bounds__(kGemm8Threads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void nf4_gemm8_kernel(GemmArgs a, ProducerParams pp, Scale scale, GemmEpi e) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kGemmLds];
  u32x2* lut = reinterpret_cast<u32x2*>(lds);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rb = wave & 3, ch = wave >> 2;  // row slice, column half
  const int i32 = lane & 31, q = lane >> 5;

  // tile and K split of this workgroup: with xcd_map, XCD x = g % 8 takes
  // tiles x T/8 .. +T/8 (row slices whose activations stay in its L2), its first lf
  // tiles whole, the rest as `splits` workgroups each (split tile ti of the
  // launch); every split of a tile sits on the tile's XCD
  const int64_t T = int64_t(a.tiles_m) * a.tiles_n;
  const int64_t g = blockIdx.x;
  int64_t t, ti = 0;
  int split = 0, nsplit = 1;
  if (a.xcd_map) {
    const int64_t x = g % 8, jw = g / 8, L = T / 8;
    if (jw < a.lf) {
      t = x * L + jw;
    } else {
      const int64_t lt = L - a.lf, jj = jw - a.lf;
      split = int(jj / lt);
      nsplit = a.splits;
      t = x * L + a.lf + jj % lt;
      ti = x * lt + jj % lt;
    }
  } else {
    t = g;
  }
  const int64_t mt = t / a.tiles_n, nt = t % a.tiles_n;
  const int64_t m0 = mt * kGemmBM, n0 = nt * kGemmBN;
  const int64_t m0w = m0 + 64 * rb;
  const int64_t nk_all = a.K / kGemmBK;
  const int64_t kbeg = nk_all * split / nsplit;
  const int64_t nk = nk_all * (split + 1) / nsplit - kbeg;  // steps of this split

  // Activation DMA lanes: this wave loads rows 32 ch .. +31 of its slice;
  // instruction tt covers rows 32 ch + 8 tt + lane / 8, chunk (lane % 8) ^
  // ((r / 2) & 7) of each.
  uint32_t xo[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int r = 32 * ch + 8 * tt + (lane >> 3);
    int64_t m = m0w + r;
    m = m < a.M ? m : a.M - 1;  // rows past M re-read a live row; never stored
    xo[tt] = uint32_t(m * a.ldx + 8 * ((lane & 7) ^ ((r >> 1) & 7)));
  }
  uint8_t* xring = lds + kXRingOff + rb * kXWaveBytes;  // + (step & 1) * kXStepBytes
  const uint32_t xring_addr = __builtin_amdgcn_readfirstlane(uint32_t(kXRingOff + rb * kXWaveBytes + ch * 4096));
  uint8_t* wtile = lds + kWTileOff;  // + (step & 1) * kWTileBytes
  const uint32_t col_base = uint32_t(64 * ch);
  Prod prod;
  prod.init(pp, scale, lut, tid, n0);

  // Step j covers k-step ks(j) = kbeg + j mod nk (the prefetches past the
  // end wrap around the split's K range: in bounds, never used).  The
  // workgroups of an XCD walk K together, so the activation (dY) rows they
  // share are fetched once into its L2.  (Starting them at staggered steps,
  // to spread the misses, measured 3 % slower forward and 7 % slower dX: with
  // activation tiles larger than the L2 every workgroup then missed on its
  // own lines.)
  const int nk32 = __builtin_amdgcn_readfirstlane(int(nk));
  const int kb32 = __builtin_amdgcn_readfirstlane(int(kbeg));
  auto ks = [&](int64_t j) -> int64_t {
    int v = int(j);  // j < nk + kWDepth
    if (v >= nk32) {
      v -= nk32;
      if (v >= nk32) v %= nk32;  // only when nk < kWDepth
    }
    return kb32 + v;
  };

  // prologue: activations of step 0, packed weights of steps 0..3, the
  // table, and step 0's weight tile
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) dma16(a.x, (xo[tt] + uint32_t(ks(0)) * kGemmBK) * 2u, xring_addr + tt * 1024);
  typename Prod::Regs wl[kWDepth];
#pragma unroll
  for (int d = 0; d < kWDepth; ++d) prod.issue(wl[d], ks(d));
  // The epilogue's LoRA operands (e.lora_regs: one staging chunk), read raw
  // now so that their latency hides under the prologue's: slot i of thread
  // t is 16-byte chunk c = (t + 512 i) % 8 of row (t + 512 i) / 8 of the u
  // rows (4 slots) and of the B rows (2 slots, two 16-byte halves for fp32);
  // chunks past rank16 / 8 re-read chunk 0 and are not staged.
  u32x4 lu[4], lb[2][2];
  if (Prod::kLoraRegs && e.lora_regs) {
    const int w8 = e.rank16 >> 3, bsh = e.b_dt == RQ_DTYPE_F32 ? 2 : 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + kGemm8Threads * i, c = idx & 7;
      int64_t m = m0 + (idx >> 3);
      m = m < a.M ? m : a.M - 1;
      lu[i] = *reinterpret_cast<const u32x4*>(e.u + m * e.rank16 + 8 * (c < w8 ? c : 0));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + kGemm8Threads * i, c = idx & 7;
      int64_t n = n0 + (idx >> 3);
      n = n < a.N ? n : a.N - 1;
      const uint8_t* row = static_cast<const uint8_t*>(e.braw) + ((n * e.b_sn + 8 * (c < w8 ? c : 0)) << bsh);
      lb[i][0] = *reinterpret_cast<const u32x4*>(row);
      lb[i][1] = *reinterpret_cast<const u32x4*>(row + (bsh == 2 ? 16 : 0));
    }
  }
  fill_f32pair_lut<kGemm8Threads>(lut, tid);
  __syncthreads();
  {
    typename Prod::Step S;
    prod.prep(S, wl[0]);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      prod.lookup(S, p);
      prod.finish(S, p, 0, wtile);
      prod.finish(S, p, 1, wtile);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();

  f32x16 acc[kGemm8MB][kGemm8NB];
#pragma unroll
  for (int mb = 0; mb < kGemm8MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kGemm8NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

  // Step j: MFMAs on weight tile j % 2 and activation ring slot j % 2;
  // direct-to-LDS loads of activations j + 1 into the other slot; step j + 1
  // dequantized from wl[(j + 1) % 4] into the other weight tile; packed
  // weights of step j + 4 into wl[j % 4]; then a barrier that waits for
  // this wave's activation loads (all but the step's kLoads trailing weight
  // loads).  Four steps per iteration index every register set statically;
  // the loop has a single exit, so the accumulators stay in place.  Steps
  // past the end wrap around the split's K range (in bounds; their results
  // are never used).  In the tail the weight loads feed nothing, so the
  // compiler drops them, and the barrier waits for every load.
#define RQ_GEMM8_STEP(J, P, WAIT)                                                                              \
  do {                                                                                                         \
    gemm8_step<XT, Prod>(acc, xring + ((P) & 1) * kXStepBytes, wtile + ((P) & 1) * kWTileBytes, i32, q,       \
                         col_base, a, xo, ks((J) + 1), xring_addr + (((P) + 1) & 1) * kXStepBytes, prod,      \
                         wl[((P) + 1) & 3], wl[P], ks((J) + kWDepth), wtile + (((P) + 1) & 1) * kWTileBytes); \
    step_barrier<WAIT>();                                                                                      \
  } while (0)
  int64_t j = 0;
  for (; j + 4 <= nk; j += 4) {
    RQ_GEMM8_STEP(j, 0, Prod::kLoads);
    RQ_GEMM8_STEP(j + 1, 1, Prod::kLoads);
    RQ_GEMM8_STEP(j + 2, 2, Prod::kLoads);
    RQ_GEMM8_STEP(j + 3, 3, Prod::kLoads);
  }
  const int64_t rem = nk - j;
  if (rem > 0) RQ_GEMM8_STEP(j, 0, 0);
  if (rem > 1) RQ_GEMM8_STEP(j + 1, 1, 0);
  if (rem > 2) RQ_GEMM8_STEP(j + 2, 2, 0);
#undef RQ_GEMM8_STEP
  wait_vmcnt<0>();  // nothing may still be landing in LDS when the epilogue reuses it

  // ---- K splits: every split stores its tile; the last to count itself
  // sums all of them in split order (the same sums whichever split is last).
  // The partials move by device-coherent stores and loads, so that no cache
  // write-back or invalidation is needed: each thread waits for its stores
  // to complete before the workgroup counts itself.
  if (nsplit > 1) {
    // A split's tile is 16 chunks of 16 bytes per thread, chunk c of thread t
    // at 16 (512 c + t) bytes: each store and load instruction of a wave moves
    // 1 KiB contiguous.  (With 64 four-byte atomic stores and loads per
    // thread the splits' exchange took 9.6 us at the k/v shapes.)
    constexpr uint32_t kTileBytes = kGemm8Threads * 64 * 4;
    const int64_t n_split_tiles = 8 * (T / 8 - a.lf);
    const __amdgpu_buffer_rsrc_t part = buffer_rsrc(a.part, uint32_t(nsplit * n_split_tiles * kTileBytes));
    const uint32_t lane_off = uint32_t(tid) * 16u;
    auto chunk = [&](int sp, int c) {  // wave-uniform part of the offset
      return __builtin_amdgcn_readfirstlane(uint32_t((int64_t(sp) * n_split_tiles + ti) * kTileBytes) +
                                            uint32_t(c * kGemm8Threads) * 16u);
    };
#pragma unroll
    for (int mb = 0; mb < kGemm8MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < kGemm8NB; ++nb)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          buf_store16_coherent(part, lane_off, chunk(split, (mb * kGemm8NB + nb) * 4 + r4),
                               u32x4{__float_as_uint(acc[mb][nb][4 * r4]), __float_as_uint(acc[mb][nb][4 * r4 + 1]),
                                     __float_as_uint(acc[mb][nb][4 * r4 + 2]),
                                     __float_as_uint(acc[mb][nb][4 * r4 + 3])});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    uint32_t* flag = reinterpret_cast<uint32_t*>(lds);  // the table's LDS is free now
    if (tid == 0) {
      const uint32_t old = __hip_atomic_fetch_add(&a.tile_cnt[ti], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old == uint32_t(nsplit - 1);
      if (last) __hip_atomic_store(&a.tile_cnt[ti], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *flag = last ? 1u : 0u;
    }
    __syncthreads();
    const uint32_t last = __builtin_amdgcn_readfirstlane(*flag);
    __syncthreads();  // every wave has read the flag before the LDS is reused
    if (!last) return;
    // a block's chunks of every split in flight together, this split's too
    // (just written, so read from the L2): the loads and the split-order sum
    // are then the same in every workgroup, with no branch between a load
    // and its use (the planner makes 2 or 4 splits)
    auto reduce = [&](auto splits) {
      constexpr int S = decltype(splits)::value;
#pragma unroll
      for (int mb = 0; mb < kGemm8MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < kGemm8NB; ++nb) {
          u32x4 o[S][4];
#pragma unroll
          for (int sp = 0; sp < S; ++sp)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
              o[sp][r4] = buf_load16_coherent(part, lane_off, chunk(sp, (mb * kGemm8NB + nb) * 4 + r4));
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float v = 0.0f;
#pragma unroll
            for (int sp = 0; sp < S; ++sp) v = __fadd_rn(v, __uint_as_float(o[sp][r >> 2][r & 3]));
            acc[mb][nb][r] = v;
          }
          __builtin_amdgcn_sched_barrier(0);  // one block's loads in flight at a time (registers)
        }
    };
    static_assert(kGemmMaxSplits == 4, "the planner's split counts are 2 and 4");
    if (nsplit == 2) reduce(std::integral_constant<int, 2>{});
    else reduce(std::integral_constant<int, 4>{});
  }

  // ---- epilogue.  y = RND(RND(acc + RND(bias)) + RND(RND(lora) * scaling))
  // (dX with LoRA dropout: scaling replaced by mask ? mask_scale : 0)
  // with lora = RND(u) RND(B)^T accumulated by MFMA in chunks of 64 ranks,
  // both operands staged into LDS (u rows and B rows of the tile, 144-byte
  // pitch).
  const int rank = e.rank;
  f32x16 lo[kGemm8MB][kGemm8NB];
#pragma unroll
  for (int mb = 0; mb < kGemm8MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kGemm8NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) lo[mb][nb][r] = 0.0f;
  if (rank > 0) {
    constexpr int kP = 72;  // staging pitch in elements
    uint16_t* us = reinterpret_cast<uint16_t*>(lds);  // [256][kP]
    uint16_t* bs = us + kGemmBM * kP;                 // [128][kP]
    for (int j0 = 0; j0 < e.rank16; j0 += 64) {
      const int w8 = (e.rank16 - j0 < 64 ? e.rank16 - j0 : 64) / 8;  // 16-byte chunks per row
      __syncthreads();  // the tiles, ring and table (first chunk) or the last chunk's operands are free
      if (Prod::kLoraRegs && e.lora_regs) {  // the only chunk, read in the prologue
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int idx = tid + kGemm8Threads * i, r = idx >> 3, c = idx & 7;
          if (c < w8) *reinterpret_cast<u32x4*>(us + r * kP + 8 * c) = lu[i];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int idx = tid + kGemm8Threads * i, r = idx >> 3, c = idx & 7;
          if (c < w8)
            *reinterpret_cast<u32x4*>(bs + r * kP + 8 * c) =
                8 * c < e.rank ? raw8_to_x<XT>(lb[i][0], lb[i][1], e.b_dt) : u32x4{0u, 0u, 0u, 0u};
        }
      } else {
      for (int idx = tid; idx < kGemmBM * w8; idx += kGemm8Threads) {
        const int r = idx / w8, c = idx - r * w8;
        int64_t m = m0 + r;
        m = m < a.M ? m : a.M - 1;
        *reinterpret_cast<u32x4*>(us + r * kP + 8 * c) =
            *reinterpret_cast<const u32x4*>(e.u + m * e.rank16 + j0 + 8 * c);
      }
      for (int idx = tid; idx < kGemmBN * w8; idx += kGemm8Threads) {
        const int r = idx / w8, c = idx - r * w8;
        int64_t n = n0 + r;
        n = n < a.N ? n : a.N - 1;
        const int j = j0 + 8 * c;
        *reinterpret_cast<u32x4*>(bs + r * kP + 8 * c) =
            e.b_sj == 1 ? load_a8_masked<XT>(e.braw, e.b_dt, n * e.b_sn + j, e.rank - j, e.b_vec)
                        : load_a8_strided<XT>(e.braw, e.b_dt, n * e.b_sn + j * e.b_sj, e.b_sj, e.rank - j);
      }
      }
      __syncthreads();
      for (int s = 0; s < w8 / 2; ++s) {
        u32x4 ua[kGemm8MB];
#pragma unroll
        for (int mb = 0; mb < kGemm8MB; ++mb)
          ua[mb] = *reinterpret_cast<const u32x4*>(us + (64 * rb + 32 * mb + i32) * kP + 16 * s + 8 * q);
#pragma unroll
        for (int nb = 0; nb < kGemm8NB; ++nb) {
          const u32x4 ub =
              *reinterpret_cast<const u32x4*>(bs + (64 * ch + 32 * nb + i32) * kP + 16 * s + 8 * q);
#pragma unroll
          for (int mb = 0; mb < kGemm8MB; ++mb) lo[mb][nb] = mfma32x32x16<XT>(ub, ua[mb], lo[mb][nb]);
        }
      }
    }
  }
  // The weights are the MFMAs' A operand, so lane (i32, q) holds row
  // m0w + 32 mb + i32 of block (mb, nb) and its columns 8 h + 4 q .. + 3 in
  // acc[mb][nb][4 h ..] (h < 4): four runs of four adjacent outputs.
  float bias[kGemm8NB][4][4];
#pragma unroll
  for (int nb = 0; nb < kGemm8NB; ++nb)
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t n = n0 + 64 * ch + 32 * nb + 8 * h + 4 * q + c;
        bias[nb][h][c] = e.bias && n < a.N ? round_x<XT>(load_as_f32(e.bias, n, e.bias_dt)) : -0.0f;
      }
  uint32_t pk[kGemm8MB][kGemm8NB][4][2];
  if (rank == 0) gemm8_outputs<XT, 0>(acc, lo, bias, e, a, m0w + i32, n0 + 64 * ch + 4 * q, pk);
  else if (!e.mask) gemm8_outputs<XT, 1>(acc, lo, bias, e, a, m0w + i32, n0 + 64 * ch + 4 * q, pk);
  else gemm8_outputs<XT, 2>(acc, lo, bias, e, a, m0w + i32, n0 + 64 * ch + 4 * q, pk);

  // A tile wholly inside the output goes out through LDS: each wave writes its
  // 64 x 64 block into its own region (the ring and weight tiles, free since
  // the last step's barrier), reads it back as 16-byte row chunks and stores
  // eight 128-byte row pieces per instruction.  (Stored from the MFMA layout,
  // an instruction wrote 16 bytes of each of 32 rows; the tile's output took
  // 3 us where these stores take a fraction of that.)
  if (m0 + kGemmBM <= a.M && n0 + kGemmBN <= a.N && (reinterpret_cast<uintptr_t>(e.y) & 15u) == 0 &&
      (e.ldy & 7) == 0) {
    uint8_t* ws = lds + kGemm8EpiOff + wave * kGemm8EpiWaveBytes;
#pragma unroll
    for (int mb = 0; mb < kGemm8MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < kGemm8NB; ++nb)
#pragma unroll
        for (int h = 0; h < 4; ++h)
          *reinterpret_cast<u32x2*>(ws + (32 * mb + i32) * kGemm8EpiPitch + (32 * nb + 8 * h + 4 * q) * 2) =
              u32x2{pk[mb][nb][h][0], pk[mb][nb][h][1]};
    uint16_t* ybase = e.y + m0w * e.ldy + n0 + 64 * ch + 8 * (lane & 7);
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int r = 8 * it + (lane >> 3);
      *reinterpret_cast<u32x4*>(ybase + r * e.ldy) =
          *reinterpret_cast<const u32x4*>(ws + r * kGemm8EpiPitch + 16 * (lane & 7));
    }
    return;
  }
  const bool vec = (reinterpret_cast<uintptr_t>(e.y) & 7u) == 0 && (e.ldy & 3) == 0;
#pragma unroll
  for (int mb = 0; mb < kGemm8MB; ++mb) {
    const int64_t m = m0w + 32 * mb + i32;
    if (m >= a.M) continue;
    uint16_t* yrow = e.y + m * e.ldy;
#pragma unroll
    for (int nb = 0; nb < kGemm8NB; ++nb)
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int64_t n = n0 + 64 * ch + 32 * nb + 8 * h + 4 * q;
        const uint32_t p0 = pk[mb][nb][h][0], p1 = pk[mb][nb][h][1];
        if (vec && n + 3 < a.N) {
          *reinterpret_cast<u32x2*>(yrow + n) = u32x2{p0, p1};
        } else {
          const uint16_t o[4] = {uint16_t(p0), uint16_t(p0 >> 16), uint16_t(p1), uint16_t(p1 >> 16)};
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (n + c < a.N) yrow[n + c] = o[c];
        }
      }
  }
}

}  // namespace rq
