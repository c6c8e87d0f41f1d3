// NF4 / double-quant / INT8 codecs for gfx950.
//
// All of these are HBM-bound byte/float streams.  The fast paths move 16 B
// per lane per access (dwordx4), keep the NF4 code book and the quantizer's
// decision table in LDS, and write packed nibbles as whole dwords.  Generic
// paths (odd block sizes, unaligned views, ragged tails) use one wave per
// segment with a strided loop.  Results are bit-identical to the PyTorch CPU
// semantics of quantization/quant_ops.py and quantization/double_quant.py
// (NaN payloads aside).
#include "rq_common.h"
#include "rq_mfma.h"
#include "nf4_tables.h"
#include "rq_launch.h"

#include <type_traits>

namespace rq {

// ---------------------------------------------------------------------------
// NF4 decision: idx = argmin_i |n - T_i| (first minimum), via the exact cell
// table (gen_nf4_tables.py).  n is the fp32 value of the normalised weight
// (already rounded to the input dtype).  NaN -> 0, as torch.argmin returns the
// first NaN.
// ---------------------------------------------------------------------------
struct NF4CellTable {
  u32x2 e[65];  // {threshold bits, base index} of each 1/32-wide cell; e[64] = e[63] (n = 1)
};

__device__ __forceinline__ void load_cell_table(NF4CellTable* t) {
  for (int i = threadIdx.x; i < 65; i += blockDim.x) {
    const int c = i < 64 ? i : 63;
    t->e[i] = u32x2{kNF4CellThr[c], kNF4CellBase[c]};
  }
}

__device__ __forceinline__ uint32_t nf4_decide(float n, const NF4CellTable* t) {
  float c = __fmul_rn(__fadd_rn(n, 1.0f), 32.0f);
  c = fminf(fmaxf(c, 0.0f), 63.0f);   // NaN -> 0 (v_max returns the non-NaN operand)
  const u32x2 cell = t->e[int(c)];
  return cell.y + (n > u2f(cell.x) ? 1u : 0u);
}

// normalised value as torch computes `reshaped / scales` in the input dtype
template <int DT>
__device__ __forceinline__ float nf4_normalise(float x, float s) {
  float q = __fdiv_rn(x, s);
  if (DT == RQ_DTYPE_F32) return q;
  return round_to(q, DT);
}

template <int DT>
__device__ __forceinline__ void load8(const void* __restrict__ w, int64_t e0, int64_t numel, bool vec,
                                      float (&v)[8]) {
  if (vec && e0 + 8 <= numel) {
    if (DT == RQ_DTYPE_F32) {
      const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(w) + e0);
      f32x4 a = __builtin_nontemporal_load(p);
      f32x4 b = __builtin_nontemporal_load(p + 1);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      u32x4 a = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(w) + e0));
      uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint16_t lo = uint16_t(u[j] & 0xFFFFu), hi = uint16_t(u[j] >> 16);
        if (DT == RQ_DTYPE_BF16) { v[2 * j] = bf16_to_f32(lo); v[2 * j + 1] = bf16_to_f32(hi); }
        else { v[2 * j] = f16_to_f32(lo); v[2 * j + 1] = f16_to_f32(hi); }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (e0 + j < numel) ? load_as_f32(w, e0 + j, DT) : 0.0f;
  }
}

// Fast path: block_size = 8 * L, L a power of two <= 64.  Each lane owns 8
// consecutive weights; the L lanes of a block reduce the absmax with xor
// shuffles.  One dword of packed nibbles per lane.
template <int DT>
__global__ __launch_bounds__(256) void nf4_quantize_fast(const void* __restrict__ w, int64_t numel,
                                                         int64_t n_lanes, int log2_l, bool vec,
                                                         uint8_t* __restrict__ packed,
                                                         void* __restrict__ absmax) {
  __shared__ NF4CellTable table;
  load_cell_table(&table);
  __syncthreads();
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  // lanes past the end still take part in the shuffles with zeros
  const bool live = t < n_lanes;
  const int64_t e0 = t * 8;
  float v[8];
  if (live) load8<DT>(w, e0, numel, vec, v);
  else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = 0.0f;
  }
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = absmax_nan(m, v[j]);
  for (int o = 1; o < (1 << log2_l); o <<= 1) m = max_nan(m, __shfl_xor(m, o));
  const float s = clamp_floor(m, DT);
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) word |= nf4_decide(nf4_normalise<DT>(v[j], s), &table) << (4 * j);
  if (!live) return;
  reinterpret_cast<uint32_t*>(packed)[t] = word;
  if ((t & ((int64_t(1) << log2_l) - 1)) == 0) store_from_f32(absmax, t >> log2_l, DT, s);
}

// ---------------------------------------------------------------------------
// 16-bit input fast path (bf16 / fp16, block_size = 8 * L, L a power of two
// <= 64, 16-byte aligned weights): the same decisions as nf4_quantize_fast
// in fewer instructions per weight (the stream is instruction-bound):
//  * absmax over the raw 16-bit patterns: |x| is h & 0x7FFF, and for
//    non-negative 16-bit floats the integer order is the value order with
//    every NaN above infinity, so a packed unsigned 16-bit max gives the
//    block maximum, NaN if the block holds one (torch's max propagates NaN);
//    the L lanes of a block reduce with DPP lane swaps (xor 1, xor 2, mirror
//    in 8, mirror in 16) and LDS permutes beyond 16 lanes;
//  * n = RND(x / s) by div_round's shortcut, the rare elements it flags
//    divided exactly (one branch per 8 weights), rounded by the hardware
//    RNE conversions (NaN stays NaN, whose decision is 0 either way);
//  * the cell index as int(fma(n, 32, 32)): 32 (n + 1) is exact up to the
//    rounding of n + 1, which scaling by 32 commutes with; -1 <= n <= 1 gives
//    0 .. 64 (cell 64, n = 1 exactly, repeats cell 63) and a NaN converts
//    to 0.
// The absmax and rs = RN(1/s) are finite or the quotient is NaN / a signed
// zero on both routes: s >= the clamp floor (bf16 1e-12; fp16 s >= 2^-24 or
// 0, where x = 0 and both routes give NaN), so non-finite products need no
// check.  A workgroup covers kQGroups * 256 groups of 8 weights, lane group g
// of thread i being group (blockIdx * kQGroups + g) * 256 + i; workgroups
// wholly inside the tensor issue their four 16-byte loads first.
// ---------------------------------------------------------------------------
constexpr int kQGroups = 4;
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t m, int ctrl_sel) {
  uint32_t o;
  switch (ctrl_sel) {
    case 0: o = uint32_t(__builtin_amdgcn_update_dpp(int(m), int(m), 0xB1, 0xF, 0xF, false)); break;   // xor 1
    case 1: o = uint32_t(__builtin_amdgcn_update_dpp(int(m), int(m), 0x4E, 0xF, 0xF, false)); break;   // xor 2
    case 2: o = uint32_t(__builtin_amdgcn_update_dpp(int(m), int(m), 0x141, 0xF, 0xF, false)); break;  // 7 - i
    default: o = uint32_t(__builtin_amdgcn_update_dpp(int(m), int(m), 0x140, 0xF, 0xF, false)); break; // 15 - i
  }
  return m > o ? m : o;
}

// Maximum of m over the 2^log2_l lanes of this lane's aligned group.
__device__ __forceinline__ uint32_t group_max_u32(uint32_t m, int log2_l) {
  if (log2_l >= 1) m = dpp_max_u32(m, 0);
  if (log2_l >= 2) m = dpp_max_u32(m, 1);
  if (log2_l >= 3) m = dpp_max_u32(m, 2);
  if (log2_l >= 4) m = dpp_max_u32(m, 3);
  for (int o = 16; o < (1 << log2_l); o <<= 1) {
    const uint32_t p = uint32_t(__shfl_xor(int(m), o));
    m = m > p ? m : p;
  }
  return m;
}

template <int DT>
__device__ __forceinline__ bool needs_exact(float r) {
  const uint32_t b = f2u(r);
  constexpr uint32_t kLow = DT == RQ_DTYPE_BF16 ? 0xFFFFu : 0x1FFFu;
  constexpr uint32_t kMid = DT == RQ_DTYPE_BF16 ? 0x8000u : 0x1000u;
  bool e = ((b & kLow) - (kMid - 4u)) <= 8u;
  if constexpr (DT == RQ_DTYPE_F16) e = e || (b & 0x7FFFFFFFu) < 0x38800000u;
  return e;
}

__device__ __forceinline__ uint32_t nf4_decide_fma(float n, const NF4CellTable* t) {
  const u32x2 cell = t->e[int(__builtin_fmaf(n, 32.0f, 32.0f))];
  return cell.y + (n > u2f(cell.x) ? 1u : 0u);
}

// Element h (0: low half, 1: high half) of a dword of two 16-bit floats.
template <int DT>
__device__ __forceinline__ float half16(uint32_t w, int h) {
  if constexpr (DT == RQ_DTYPE_BF16) return u2f(h ? (w & 0xFFFF0000u) : (w << 16));
  else return f16_to_f32(uint16_t(h ? (w >> 16) : (w & 0xFFFFu)));
}

template <int DT>
__device__ __forceinline__ void quantize_group16(const u32x4& raw, int64_t t, int log2_l, bool live,
                                                 const NF4CellTable* table, uint8_t* __restrict__ packed,
                                                 void* __restrict__ absmax) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  u16x2 a[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) a[j] = __builtin_bit_cast(u16x2, w[j] & 0x7FFF7FFFu);
  const u16x2 m2 = __builtin_elementwise_max(__builtin_elementwise_max(a[0], a[1]),
                                             __builtin_elementwise_max(a[2], a[3]));
  uint32_t mb = m2.x > m2.y ? uint32_t(m2.x) : uint32_t(m2.y);
  mb = group_max_u32(mb, log2_l);
  const float s = clamp_floor(from_x16<DT>(mb), DT);
  const float rs = recip_rn(s);
  float x[8], r[8];
  bool any = false;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    x[j] = half16<DT>(w[j >> 1], j & 1);
    r[j] = __fmul_rn(x[j], rs);
    any |= needs_exact<DT>(r[j]);
  }
  if (any) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (needs_exact<DT>(r[j])) r[j] = __fdiv_rn(x[j], s);
  }
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const uint32_t pk = cvt_pk<DT>(r[j], r[j + 1]);
    word |= nf4_decide_fma(half16<DT>(pk, 0), table) << (4 * j);
    word |= nf4_decide_fma(half16<DT>(pk, 1), table) << (4 * j + 4);
  }
  if (!live) return;
  reinterpret_cast<uint32_t*>(packed)[t] = word;
  if ((t & ((int64_t(1) << log2_l) - 1)) == 0) store_from_f32(absmax, t >> log2_l, DT, s);
}

template <int DT>
__global__ __launch_bounds__(256) void nf4_quantize16_kernel(const uint16_t* __restrict__ w, int64_t numel,
                                                             int64_t n_lanes, int log2_l,
                                                             uint8_t* __restrict__ packed,
                                                             void* __restrict__ absmax) {
  __shared__ NF4CellTable table;
  load_cell_table(&table);
  __syncthreads();
  const int64_t t0 = int64_t(blockIdx.x) * (256 * kQGroups) + threadIdx.x;
  const int64_t end = int64_t(blockIdx.x + 1) * (256 * kQGroups);  // groups of this workgroup
  if (end * 8 <= numel) {
    u32x4 raw[kQGroups];
#pragma unroll
    for (int g = 0; g < kQGroups; ++g)
      raw[g] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + (t0 + 256 * g) * 8));
#pragma unroll
    for (int g = 0; g < kQGroups; ++g) quantize_group16<DT>(raw[g], t0 + 256 * g, log2_l, true, &table, packed, absmax);
    return;
  }
  for (int g = 0; g < kQGroups; ++g) {
    const int64_t t = t0 + 256 * g;
    // lanes past the end still take part in the reductions with zeros
    const bool live = t < n_lanes;
    uint32_t h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (live && t * 8 + j < numel) ? uint32_t(w[t * 8 + j]) : 0u;
    const u32x4 raw = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    quantize_group16<DT>(raw, t, log2_l, live, &table, packed, absmax);
  }
}

// Generic path: one wave per block of any even size; lane l handles element
// pairs (2l, 2l+1) + 128 k.
template <int DT>
__global__ __launch_bounds__(256) void nf4_quantize_generic(const void* __restrict__ w, int64_t numel,
                                                            int64_t n_blocks, int64_t bs,
                                                            uint8_t* __restrict__ packed,
                                                            void* __restrict__ absmax) {
  __shared__ NF4CellTable table;
  load_cell_table(&table);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t b = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (b >= n_blocks) return;
  const int64_t base = b * bs;
  float m = 0.0f;
  for (int64_t i = lane; i < bs; i += 64) {
    int64_t e = base + i;
    if (e < numel) m = absmax_nan(m, load_as_f32(w, e, DT));
  }
  for (int o = 1; o < 64; o <<= 1) m = max_nan(m, __shfl_xor(m, o));
  const float s = clamp_floor(m, DT);
  for (int64_t i = 2 * lane; i < bs; i += 128) {
    int64_t e = base + i;
    float x0 = e < numel ? load_as_f32(w, e, DT) : 0.0f;
    float x1 = e + 1 < numel ? load_as_f32(w, e + 1, DT) : 0.0f;
    uint32_t lo = nf4_decide(nf4_normalise<DT>(x0, s), &table);
    uint32_t hi = nf4_decide(nf4_normalise<DT>(x1, s), &table);
    packed[e >> 1] = uint8_t(lo | (hi << 4));
  }
  if (lane == 0) store_from_f32(absmax, b, DT, s);
}

// ---------------------------------------------------------------------------
// NF4 dequantize.  Fast path: block_size % 16 == 0, each lane expands 8 packed
// bytes (16 weights, inside one block) with the code book in LDS.
// ---------------------------------------------------------------------------
// (b_off: the block index of the first weight of the launch's range)
struct ScaleSingle {
  const void* absmax;
  int dt;
  int64_t b_off;
  __device__ __forceinline__ float operator()(int64_t b) const { return load_as_f32(absmax, b + b_off, dt); }
};

struct ScaleDouble {
  const uint8_t* c2;
  const void* c2s;
  int c2s_dt;
  int fmt;
  int64_t block2;
  int64_t b_off;
  __device__ __forceinline__ float operator()(int64_t b) const {
    b += b_off;
    float hi = load_as_f32(c2s, b / block2, c2s_dt);
    float lo;
    if (fmt == RQ_C2_FP8_E4M3FNUZ) lo = fnuz_to_f32(c2[b]);
    else lo = __fdiv_rn(float(int8_t(c2[b])), 127.0f);
    return __fmul_rn(lo, hi);
  }
};

template <int ODT>
__device__ __forceinline__ void store16(void* __restrict__ out, int64_t e0, int64_t n_out, bool vec,
                                        const float (&v)[16]) {
  if (vec && e0 + 16 <= n_out) {
    if (ODT == RQ_DTYPE_F32) {
      f32x4* p = reinterpret_cast<f32x4*>(static_cast<float*>(out) + e0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 q = {v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
        __builtin_nontemporal_store(q, p + j);
      }
    } else {
      uint32_t u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t a = ODT == RQ_DTYPE_BF16 ? f32_to_bf16_rne(v[2 * j]) : f32_to_f16_rne(v[2 * j]);
        uint32_t b = ODT == RQ_DTYPE_BF16 ? f32_to_bf16_rne(v[2 * j + 1]) : f32_to_f16_rne(v[2 * j + 1]);
        u[j] = a | (b << 16);
      }
      u32x4* p = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + e0);
      u32x4 q0 = {u[0], u[1], u[2], u[3]}, q1 = {u[4], u[5], u[6], u[7]};
      __builtin_nontemporal_store(q0, p);
      __builtin_nontemporal_store(q1, p + 1);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (e0 + j < n_out) store_from_f32(out, e0 + j, ODT, v[j]);
  }
}

template <int ODT, class Scale>
__global__ __launch_bounds__(256) void nf4_dequant_fast(const uint8_t* __restrict__ packed, Scale scale,
                                                        int64_t n_lanes, int64_t n_packed, int64_t bs,
                                                        bool vec, void* __restrict__ out, int64_t n_out) {
  __shared__ float lut[16];
  if (threadIdx.x < 16) lut[threadIdx.x] = u2f(kNF4Bits[threadIdx.x]);
  __syncthreads();
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n_lanes) return;
  const int64_t e0 = t * 16;
  if (e0 >= n_out) return;
  u32x2 p;
  if (8 * t + 8 <= n_packed) {
    p = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(packed) + t);
  } else {  // ragged tail: byte loads, zero past the end
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = (8 * t + j < n_packed) ? packed[8 * t + j] : 0u;
    p.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    p.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
  }
  const float s = scale(e0 / bs);
  float v[16];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t w = j < 4 ? p.x : p.y;
    uint32_t byte = (w >> (8 * (j & 3))) & 0xFFu;
    v[2 * j] = __fmul_rn(lut[byte & 0xF], s);
    v[2 * j + 1] = __fmul_rn(lut[byte >> 4], s);
  }
  store16<ODT>(out, e0, n_out, vec, v);
}

// ---------------------------------------------------------------------------
// 16-bit output fast path (bf16 / fp16 out, power-of-two block sizes >= 16,
// codes 4-byte and output 16-byte aligned).  A chunk is 8 weights: one
// dword of codes, one 16-byte output vector.  Wave v of a workgroup owns
// chunks 256 v' .. 256 v' + 255 (v' = 4 blockIdx + v) and lane l takes
// chunks 256 v' + 64 j + l, j = 0..3, so that each of the wave's four
// stores writes 1 KiB of consecutive bytes and each code load reads 256
// consecutive bytes.  The scales are template policies with compile-time
// dtypes, so a lane's four code loads and its scale loads are all issued
// before the first is used.  Workgroups reaching past the end of the codes
// or of the output take the generic-width path below.
// ---------------------------------------------------------------------------
template <int SDT>
struct DqScaleAbs {
  const void* absmax;
  __device__ __forceinline__ float operator()(int64_t b) const { return load_as_f32(absmax, b, SDT); }
};

template <int SDT, int FMT>
struct DqScaleDouble {
  const uint8_t* c2;
  const void* c2s;
  int b2_log2;  // block2 = 2^b2_log2
  __device__ __forceinline__ float operator()(int64_t b) const {
    const float hi = load_as_f32(c2s, b >> b2_log2, SDT);
    const float lo = FMT == RQ_C2_FP8_E4M3FNUZ ? fnuz_to_f32(c2[b]) : __fdiv_rn(float(int8_t(c2[b])), 127.0f);
    return __fmul_rn(lo, hi);
  }
};

template <int ODT, class Scale>
__global__ __launch_bounds__(256) void nf4_dequant16_kernel(const uint32_t* __restrict__ packed, Scale scale,
                                                            int bs_log2, uint32_t* __restrict__ out) {
  __shared__ float lut[16];
  if (threadIdx.x < 16) lut[threadIdx.x] = u2f(kNF4Bits[threadIdx.x]);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t c0 = (int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 256 + lane;
  uint32_t p[4];
  float s[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = __builtin_nontemporal_load(packed + c0 + 64 * j);
#pragma unroll
  for (int j = 0; j < 4; ++j) s[j] = scale(((c0 + 64 * j) * 8) >> bs_log2);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t byte = (p[j] >> (8 * k)) & 0xFFu;
      o[k] = cvt_pk<ODT>(__fmul_rn(lut[byte & 0xF], s[j]), __fmul_rn(lut[byte >> 4], s[j]));
    }
    __builtin_nontemporal_store(u32x4{o[0], o[1], o[2], o[3]}, reinterpret_cast<u32x4*>(out) + c0 + 64 * j);
  }
}

template <int ODT, class Scale>
__global__ __launch_bounds__(256) void nf4_dequant_generic(const uint8_t* __restrict__ packed, Scale scale,
                                                           int64_t bs, void* __restrict__ out,
                                                           int64_t n_out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_out) return;
  uint32_t byte = packed[i >> 1];
  uint32_t code = (i & 1) ? (byte >> 4) : (byte & 0xF);
  store_from_f32(out, i, ODT, __fmul_rn(u2f(kNF4Bits[code]), scale(i / bs)));
}

// ---------------------------------------------------------------------------
// Double-quant second stage: per block2 of c1, c2s = clamp(absmax), c2 =
// fnuz(dtype(c1 / c2s)) or int8(round(dtype(dtype(c1 / c2s) * 127))).
// One wave per block2.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void dq_quantize_kernel(const void* __restrict__ c1, int64_t n_c1,
                                                          int64_t n_blocks, int64_t bs2, int fmt,
                                                          uint8_t* __restrict__ c2,
                                                          void* __restrict__ c2s) {
  const int lane = threadIdx.x & 63;
  const int64_t b = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (b >= n_blocks) return;
  const int64_t base = b * bs2;
  float m = 0.0f;
  for (int64_t i = lane; i < bs2; i += 64)
    if (base + i < n_c1) m = absmax_nan(m, load_as_f32(c1, base + i, DT));
  for (int o = 1; o < 64; o <<= 1) m = max_nan(m, __shfl_xor(m, o));
  const float s = clamp_floor(m, DT);
  for (int64_t i = lane; i < bs2; i += 64) {
    int64_t e = base + i;
    float x = e < n_c1 ? load_as_f32(c1, e, DT) : 0.0f;
    float nrm = round_to(__fdiv_rn(x, s), DT);
    uint8_t code;
    if (fmt == RQ_C2_FP8_E4M3FNUZ) {
      code = f32_to_fnuz_rne(nrm);
    } else {
      float r = rintf(round_to(__fmul_rn(nrm, 127.0f), DT));
      code = uint8_t(int8_t(int32_t(r)));
    }
    c2[e] = code;
  }
  if (lane == 0) store_from_f32(c2s, b, DT, s);
}

// ---------------------------------------------------------------------------
// INT8 codec: one wave per segment (block or row).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void int8_quantize_kernel(const void* __restrict__ w, int64_t numel,
                                                            int64_t n_seg, int64_t seg,
                                                            int8_t* __restrict__ q,
                                                            void* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int64_t b = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (b >= n_seg) return;
  const int64_t base = b * seg;
  float m = 0.0f;
  for (int64_t i = lane; i < seg; i += 64)
    if (base + i < numel) m = absmax_nan(m, load_as_f32(w, base + i, DT));
  for (int o = 1; o < 64; o <<= 1) m = max_nan(m, __shfl_xor(m, o));
  const float s = clamp_floor(round_to(__fdiv_rn(m, 127.0f), DT), DT);
  for (int64_t i = lane; i < seg; i += 64) {
    int64_t e = base + i;
    float x = e < numel ? load_as_f32(w, e, DT) : 0.0f;
    float r = rintf(round_to(__fdiv_rn(x, s), DT));
    q[e] = int8_t(int32_t(r));
  }
  if (lane == 0) store_from_f32(scales, b, DT, s);
}

// ---------------------------------------------------------------------------
// INT8 codec fast paths: 16-bit weights / outputs, 16-byte aligned weights
// and 8-byte aligned codes, whole segments of a multiple of 8 elements.  A
// group is 8 consecutive elements (one 16-byte weight load, one 8-byte code
// store); the absmax runs over raw 16-bit patterns as in the NF4 encoder
// (|x| = h & 0x7FFF, a NaN above infinity) and q = int8(int32(rint(
// RND(x / s)))) takes div_round's shortcut (the same bits as the division).
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ uint32_t absmax_bits16(const u32x4& raw) {
  const u16x2 m2 = __builtin_elementwise_max(
      __builtin_elementwise_max(__builtin_bit_cast(u16x2, raw.x & 0x7FFF7FFFu), __builtin_bit_cast(u16x2, raw.y & 0x7FFF7FFFu)),
      __builtin_elementwise_max(__builtin_bit_cast(u16x2, raw.z & 0x7FFF7FFFu), __builtin_bit_cast(u16x2, raw.w & 0x7FFF7FFFu)));
  return f2u(from_x16<DT>(m2.x > m2.y ? uint32_t(m2.x) : uint32_t(m2.y)));  // fp32 bits of the 16-bit max
}

template <int DT>
__device__ __forceinline__ float int8_scale(uint32_t mbits) {
  return clamp_floor(round_to(__fdiv_rn(u2f(mbits), 127.0f), DT), DT);
}

template <int DT>
__device__ __forceinline__ u32x2 int8_codes_group(const u32x4& raw, float s, float rs) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  uint32_t c[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float r = rintf(div_round<DT>(half16<DT>(w[j >> 1], j & 1), s, rs));
    c[j >> 2] |= (uint32_t(int32_t(r)) & 0xFFu) << (8 * (j & 3));
  }
  return u32x2{c[0], c[1]};
}

// Segments of L = 2^log2_l <= 64 groups (blockwise scales): the L lanes of a
// segment reduce with DPP / shuffles; groups (blockIdx * 4 + g) * 256 + i,
// all four loads first.  n_groups is a multiple of L.
template <int DT>
__global__ __launch_bounds__(256) void int8_quantize_groups16(const uint16_t* __restrict__ w, int64_t n_groups,
                                                              int log2_l, int8_t* __restrict__ q,
                                                              void* __restrict__ scales) {
  const int64_t t0 = int64_t(blockIdx.x) * 1024 + threadIdx.x;
  u32x4 raw[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t t = t0 + 256 * g;
    raw[g] = t < n_groups ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + 8 * t))
                          : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t t = t0 + 256 * g;
    const float s = int8_scale<DT>(group_max_u32(absmax_bits16<DT>(raw[g]), log2_l));
    if (t >= n_groups) continue;
    *reinterpret_cast<u32x2*>(q + 8 * t) = int8_codes_group<DT>(raw[g], s, recip_rn(s));
    if ((t & ((int64_t(1) << log2_l) - 1)) == 0) store_from_f32(scales, t >> log2_l, DT, s);
  }
}

// Segments of more than 64 groups (a row per output channel): one workgroup
// of 256 threads per segment; thread i takes groups i + 256 j, up to four of
// them held in registers for the second pass (segments of up to 8192
// elements), the rest loaded again.
template <int DT>
__global__ __launch_bounds__(256) void int8_quantize_rows16(const uint16_t* __restrict__ w, int64_t seg_groups,
                                                            int8_t* __restrict__ q, void* __restrict__ scales) {
  __shared__ uint32_t red[4];
  const int64_t b = blockIdx.x;
  const uint16_t* ws = w + b * seg_groups * 8;
  int8_t* qs = q + b * seg_groups * 8;
  u32x4 raw[4];
  uint32_t m = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t i = threadIdx.x + 256 * j;
    raw[j] = i < seg_groups ? *reinterpret_cast<const u32x4*>(ws + 8 * i) : u32x4{0u, 0u, 0u, 0u};
    const uint32_t v = absmax_bits16<DT>(raw[j]);
    m = m > v ? m : v;
  }
  for (int64_t i = threadIdx.x + 1024; i < seg_groups; i += 256) {
    const uint32_t v = absmax_bits16<DT>(*reinterpret_cast<const u32x4*>(ws + 8 * i));
    m = m > v ? m : v;
  }
  m = group_max_u32(m, 6);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) m = m > red[k] ? m : red[k];
  const float s = int8_scale<DT>(m);
  const float rs = recip_rn(s);
  if (threadIdx.x == 0) store_from_f32(scales, b, DT, s);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t i = threadIdx.x + 256 * j;
    if (i < seg_groups) *reinterpret_cast<u32x2*>(qs + 8 * i) = int8_codes_group<DT>(raw[j], s, rs);
  }
  for (int64_t i = threadIdx.x + 1024; i < seg_groups; i += 256)
    *reinterpret_cast<u32x2*>(qs + 8 * i) =
        int8_codes_group<DT>(*reinterpret_cast<const u32x4*>(ws + 8 * i), s, rs);
}

// Dequantize to a 16-bit dtype, segments a multiple of 8 elements: out =
// RND(float(q) * s) for groups (blockIdx * 4 + g) * 256 + i -- 8-byte code
// loads, one scale, 16-byte output stores (consecutive lanes, consecutive
// bytes), all four groups' loads first.
template <int ODT, int SDT>
__global__ __launch_bounds__(256) void int8_dequant16_kernel(const uint32_t* __restrict__ q, const void* scales,
                                                             int64_t seg_groups, int64_t n_groups,
                                                             u32x4* __restrict__ out) {
  const int64_t t0 = int64_t(blockIdx.x) * 1024 + threadIdx.x;
  u32x2 c[4];
  float sc[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t t = t0 + 256 * g;
    const int64_t tl = t < n_groups ? t : n_groups - 1;
    c[g] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(q) + tl);
    sc[g] = load_as_f32(scales, tl / seg_groups, SDT);
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t t = t0 + 256 * g;
    if (t >= n_groups) continue;
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t word = k < 2 ? c[g].x : c[g].y;
      const int sh = 16 * (k & 1);
      o[k] = cvt_pk<ODT>(__fmul_rn(float(int8_t(uint8_t(word >> sh))), sc[g]),
                         __fmul_rn(float(int8_t(uint8_t(word >> (sh + 8)))), sc[g]));
    }
    __builtin_nontemporal_store(u32x4{o[0], o[1], o[2], o[3]}, out + t);
  }
}

// The same to fp32: groups of 4 codes (one 4-byte load, one 16-byte store).
template <int SDT>
__global__ __launch_bounds__(256) void int8_dequant_f32_kernel(const uint32_t* __restrict__ q, const void* scales,
                                                               int64_t seg_groups, int64_t n_groups,
                                                               f32x4* __restrict__ out) {
  const int64_t t0 = int64_t(blockIdx.x) * 1024 + threadIdx.x;
  uint32_t c[4];
  float sc[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t t = t0 + 256 * g;
    const int64_t tl = t < n_groups ? t : n_groups - 1;
    c[g] = __builtin_nontemporal_load(q + tl);
    sc[g] = load_as_f32(scales, tl / seg_groups, SDT);
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t t = t0 + 256 * g;
    if (t >= n_groups) continue;
    f32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = __fmul_rn(float(int8_t(uint8_t(c[g] >> (8 * k)))), sc[g]);
    __builtin_nontemporal_store(o, out + t);
  }
}

template <int ODT>
__global__ __launch_bounds__(256) void int8_dequant_kernel(const int8_t* __restrict__ q, const void* scales,
                                                           int sdt, int64_t seg, void* __restrict__ out,
                                                           int64_t i0, int64_t n_out) {
  const int64_t i = i0 + int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_out) return;
  store_from_f32(out, i, ODT, __fmul_rn(float(q[i]), load_as_f32(scales, i / seg, sdt)));
}

}  // namespace rq

// ===========================================================================
// C ABI
// ===========================================================================
using namespace rq;

extern "C" int rq_nf4_quantize(const void* w, int w_dtype, int64_t numel, int64_t block_size,
                               uint8_t* packed, void* absmax, hipStream_t stream) {
  if (!valid_float_dtype(w_dtype)) return RQ_ERR_BAD_DTYPE;
  if (numel < 0 || block_size < 2 || (block_size & 1)) return RQ_ERR_BAD_SHAPE;
  if (numel == 0) return RQ_OK;
  if (!w || !packed || !absmax) return RQ_ERR_NULL_POINTER;
  const int64_t n_blocks = ceil_div(numel, block_size);
  const int64_t padded = n_blocks * block_size;
  int log2_l = -1;
  if (block_size % 8 == 0 && block_size <= 512) {
    int64_t l = block_size / 8;
    if ((l & (l - 1)) == 0) log2_l = __builtin_ctzll(l);
  }
  const bool vec = aligned(w, 16);
  if (log2_l >= 0 && aligned(packed, 4) && vec && w_dtype != RQ_DTYPE_F32) {
    const int64_t n_lanes = padded / 8;
    dim3 grid(unsigned(ceil_div(n_lanes, 256 * kQGroups)));
    if (w_dtype == RQ_DTYPE_BF16)
      nf4_quantize16_kernel<RQ_DTYPE_BF16><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(w), numel,
                                                                     n_lanes, log2_l, packed, absmax);
    else
      nf4_quantize16_kernel<RQ_DTYPE_F16><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(w), numel,
                                                                    n_lanes, log2_l, packed, absmax);
  } else if (log2_l >= 0 && aligned(packed, 4)) {
    const int64_t n_lanes = padded / 8;
    dim3 grid(unsigned(ceil_div(n_lanes, 256)));
    RQ_DISPATCH_DT(w_dtype, DT, nf4_quantize_fast<DT><<<grid, 256, 0, stream>>>(
                                    w, numel, n_lanes, log2_l, vec, packed, absmax));
  } else {
    dim3 grid(unsigned(ceil_div(n_blocks, 4)));
    RQ_DISPATCH_DT(w_dtype, DT, nf4_quantize_generic<DT><<<grid, 256, 0, stream>>>(
                                    w, numel, n_blocks, block_size, packed, absmax));
  }
  return rq_check_launch();
}

static int64_t dtype_bytes(int dt) { return dt == RQ_DTYPE_F32 ? 4 : 2; }

// Runs nf4_dequant16_kernel over the whole workgroups that fit (1024 chunks
// of 8 weights each) and returns the number of weights covered (0 when the
// call does not qualify); the rest goes through nf4_dequant_launch.
template <class Scale>
static int64_t nf4_dequant16_prefix(const uint8_t* packed, Scale scale, int64_t n_packed, int64_t bs,
                                    void* out, int out_dtype, int64_t n_out, hipStream_t stream) {
  if (out_dtype == RQ_DTYPE_F32 || bs < 16 || (bs & (bs - 1)) || !aligned(packed, 4) || !aligned(out, 16))
    return 0;
  const int64_t chunks = n_packed / 4 < n_out / 8 ? n_packed / 4 : n_out / 8;
  const int64_t wgs = chunks / 1024;
  if (wgs <= 0 || wgs > 0x7FFFFFFF) return 0;
  const int bs_log2 = __builtin_ctzll(uint64_t(bs));
  const uint32_t* p = reinterpret_cast<const uint32_t*>(packed);
  uint32_t* o = static_cast<uint32_t*>(out);
  if (out_dtype == RQ_DTYPE_BF16)
    nf4_dequant16_kernel<RQ_DTYPE_BF16, Scale><<<unsigned(wgs), 256, 0, stream>>>(p, scale, bs_log2, o);
  else
    nf4_dequant16_kernel<RQ_DTYPE_F16, Scale><<<unsigned(wgs), 256, 0, stream>>>(p, scale, bs_log2, o);
  return wgs * 1024 * 8;
}

template <class Scale>
static int nf4_dequant_launch(const uint8_t* packed, Scale scale, int64_t n_packed, int64_t bs,
                              void* out, int out_dtype, int64_t n_out, hipStream_t stream) {
  const bool fast = bs % 16 == 0 && aligned(packed, 8);
  const bool vec = aligned(out, 16);
  if (fast) {
    const int64_t n_lanes = ceil_div(n_packed, 8);
    dim3 grid(unsigned(ceil_div(n_lanes, 256)));
    RQ_DISPATCH_DT(out_dtype, ODT, nf4_dequant_fast<ODT, Scale><<<grid, 256, 0, stream>>>(
                                       packed, scale, n_lanes, n_packed, bs, vec, out, n_out));
  } else {
    dim3 grid(unsigned(ceil_div(n_out, 256)));
    RQ_DISPATCH_DT(out_dtype, ODT, nf4_dequant_generic<ODT, Scale><<<grid, 256, 0, stream>>>(
                                       packed, scale, bs, out, n_out));
  }
  return rq_check_launch();
}

extern "C" int rq_nf4_dequantize(const uint8_t* packed, const void* absmax, int absmax_dtype,
                                 int64_t n_packed, int64_t block_size, void* out, int out_dtype,
                                 int64_t n_out, hipStream_t stream) {
  if (!valid_float_dtype(absmax_dtype) || !valid_float_dtype(out_dtype)) return RQ_ERR_BAD_DTYPE;
  if (n_packed < 0 || block_size < 1 || n_out < 0 || n_out > 2 * n_packed) return RQ_ERR_BAD_SHAPE;
  if ((2 * n_packed) % block_size != 0) return RQ_ERR_BAD_SHAPE;
  if (n_out == 0) return RQ_OK;
  if (!packed || !absmax || !out) return RQ_ERR_NULL_POINTER;
  if (n_packed > (int64_t(1) << 36)) return RQ_ERR_BAD_SHAPE;
  int64_t done = 0;
  if (block_size <= 8192) {
    if (absmax_dtype == RQ_DTYPE_F32)
      done = nf4_dequant16_prefix(packed, DqScaleAbs<RQ_DTYPE_F32>{absmax}, n_packed, block_size, out, out_dtype,
                                  n_out, stream);
    else if (absmax_dtype == RQ_DTYPE_BF16)
      done = nf4_dequant16_prefix(packed, DqScaleAbs<RQ_DTYPE_BF16>{absmax}, n_packed, block_size, out,
                                  out_dtype, n_out, stream);
    else
      done = nf4_dequant16_prefix(packed, DqScaleAbs<RQ_DTYPE_F16>{absmax}, n_packed, block_size, out,
                                  out_dtype, n_out, stream);
  }
  if (done == n_out) return rq_check_launch();
  return nf4_dequant_launch(packed + done / 2, ScaleSingle{absmax, absmax_dtype, done / block_size},
                            n_packed - done / 2, block_size, static_cast<char*>(out) + done * dtype_bytes(out_dtype),
                            out_dtype, n_out - done, stream);
}

extern "C" int rq_dq_quantize(const void* c1, int c1_dtype, int64_t n_c1, int64_t block2,
                              int c2_format, uint8_t* c2, void* c2_scales, hipStream_t stream) {
  if (!valid_float_dtype(c1_dtype)) return RQ_ERR_BAD_DTYPE;
  if (c2_format != RQ_C2_FP8_E4M3FNUZ && c2_format != RQ_C2_INT8) return RQ_ERR_BAD_DTYPE;
  if (n_c1 < 0 || block2 < 1) return RQ_ERR_BAD_SHAPE;
  if (n_c1 == 0) return RQ_OK;
  if (!c1 || !c2 || !c2_scales) return RQ_ERR_NULL_POINTER;
  const int64_t nb = ceil_div(n_c1, block2);
  dim3 grid(unsigned(ceil_div(nb, 4)));
  RQ_DISPATCH_DT(c1_dtype, DT, dq_quantize_kernel<DT><<<grid, 256, 0, stream>>>(
                                   c1, n_c1, nb, block2, c2_format, c2, c2_scales));
  return rq_check_launch();
}

extern "C" int rq_dq_dequantize(const uint8_t* packed, const uint8_t* c2, int c2_format,
                                const void* c2_scales, int c2s_dtype, int64_t n_packed,
                                int64_t block1, int64_t block2, void* out, int out_dtype,
                                int64_t n_out, hipStream_t stream) {
  if (!valid_float_dtype(c2s_dtype) || !valid_float_dtype(out_dtype)) return RQ_ERR_BAD_DTYPE;
  if (c2_format != RQ_C2_FP8_E4M3FNUZ && c2_format != RQ_C2_INT8) return RQ_ERR_BAD_DTYPE;
  if (n_packed < 0 || block1 < 1 || block2 < 1 || n_out < 0 || n_out > 2 * n_packed)
    return RQ_ERR_BAD_SHAPE;
  if ((2 * n_packed) % block1 != 0) return RQ_ERR_BAD_SHAPE;
  if (n_out == 0) return RQ_OK;
  if (!packed || !c2 || !c2_scales || !out) return RQ_ERR_NULL_POINTER;
  int64_t done = 0;
  if (block1 <= 8192 && (block2 & (block2 - 1)) == 0) {
    const int b2 = __builtin_ctzll(uint64_t(block2));
    auto run = [&](auto sc) { return nf4_dequant16_prefix(packed, sc, n_packed, block1, out, out_dtype, n_out, stream); };
    const bool fp8 = c2_format == RQ_C2_FP8_E4M3FNUZ;
    if (c2s_dtype == RQ_DTYPE_F32)
      done = fp8 ? run(DqScaleDouble<RQ_DTYPE_F32, RQ_C2_FP8_E4M3FNUZ>{c2, c2_scales, b2})
                 : run(DqScaleDouble<RQ_DTYPE_F32, RQ_C2_INT8>{c2, c2_scales, b2});
    else if (c2s_dtype == RQ_DTYPE_BF16)
      done = fp8 ? run(DqScaleDouble<RQ_DTYPE_BF16, RQ_C2_FP8_E4M3FNUZ>{c2, c2_scales, b2})
                 : run(DqScaleDouble<RQ_DTYPE_BF16, RQ_C2_INT8>{c2, c2_scales, b2});
    else
      done = fp8 ? run(DqScaleDouble<RQ_DTYPE_F16, RQ_C2_FP8_E4M3FNUZ>{c2, c2_scales, b2})
                 : run(DqScaleDouble<RQ_DTYPE_F16, RQ_C2_INT8>{c2, c2_scales, b2});
  }
  if (done == n_out) return rq_check_launch();
  return nf4_dequant_launch(packed + done / 2,
                            ScaleDouble{c2, c2_scales, c2s_dtype, c2_format, block2, done / block1},
                            n_packed - done / 2, block1, static_cast<char*>(out) + done * dtype_bytes(out_dtype),
                            out_dtype, n_out - done, stream);
}

extern "C" int rq_int8_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols,
                                int64_t block_size, int8_t* q, void* scales, hipStream_t stream) {
  if (!valid_float_dtype(w_dtype)) return RQ_ERR_BAD_DTYPE;
  if (rows < 0 || cols < 0 || block_size < 0) return RQ_ERR_BAD_SHAPE;
  const int64_t numel = rows * cols;
  if (numel == 0) return RQ_OK;
  if (!w || !q || !scales) return RQ_ERR_NULL_POINTER;
  const int64_t seg = block_size > 0 ? block_size : cols;
  const int64_t n_seg = block_size > 0 ? ceil_div(numel, block_size) : rows;
  // 16-bit weights in whole segments of 8-element groups: the vector kernels
  if (w_dtype != RQ_DTYPE_F32 && seg % 8 == 0 && numel % seg == 0 && aligned(w, 16) && aligned(q, 8) &&
      numel / 8 < (int64_t(1) << 40)) {
    const int64_t sg = seg / 8, n_groups = numel / 8;
    const uint16_t* w16 = static_cast<const uint16_t*>(w);
    if (sg <= 64 && (sg & (sg - 1)) == 0) {
      const int log2_l = __builtin_ctzll(uint64_t(sg));
      const dim3 grid(unsigned(ceil_div(n_groups, 1024)));
      if (w_dtype == RQ_DTYPE_BF16)
        int8_quantize_groups16<RQ_DTYPE_BF16><<<grid, 256, 0, stream>>>(w16, n_groups, log2_l, q, scales);
      else
        int8_quantize_groups16<RQ_DTYPE_F16><<<grid, 256, 0, stream>>>(w16, n_groups, log2_l, q, scales);
      return rq_check_launch();
    }
    if (sg > 64 && n_seg <= 0x7FFFFFFF) {
      if (w_dtype == RQ_DTYPE_BF16)
        int8_quantize_rows16<RQ_DTYPE_BF16><<<unsigned(n_seg), 256, 0, stream>>>(w16, sg, q, scales);
      else
        int8_quantize_rows16<RQ_DTYPE_F16><<<unsigned(n_seg), 256, 0, stream>>>(w16, sg, q, scales);
      return rq_check_launch();
    }
  }
  dim3 grid(unsigned(ceil_div(n_seg, 4)));
  RQ_DISPATCH_DT(w_dtype, DT, int8_quantize_kernel<DT><<<grid, 256, 0, stream>>>(
                                  w, numel, n_seg, seg, q, scales));
  return rq_check_launch();
}

extern "C" int rq_int8_dequantize(const int8_t* q, const void* scales, int scales_dtype, int64_t rows,
                                  int64_t cols, int64_t block_size, void* out, int out_dtype,
                                  int64_t n_out, hipStream_t stream) {
  if (!valid_float_dtype(scales_dtype) || !valid_float_dtype(out_dtype)) return RQ_ERR_BAD_DTYPE;
  if (rows < 0 || cols < 0 || block_size < 0 || n_out < 0) return RQ_ERR_BAD_SHAPE;
  const int64_t seg = block_size > 0 ? block_size : cols;
  const int64_t cap = block_size > 0 ? ceil_div(rows * cols, block_size) * block_size : rows * cols;
  if (n_out > cap || (seg == 0 && n_out > 0)) return RQ_ERR_BAD_SHAPE;
  if (n_out == 0) return RQ_OK;
  if (!q || !scales || !out) return RQ_ERR_NULL_POINTER;
  // segments of whole groups (fp32 output: 4 elements, 16-bit: 8): the
  // vector kernels over the whole groups, the generic one over the rest
  int64_t done = 0;
  if (out_dtype == RQ_DTYPE_F32 && seg % 4 == 0 && aligned(q, 4) && aligned(out, 16) && n_out >= 4) {
    const int64_t n_groups = n_out / 4, sg = seg / 4;
    const dim3 grid(unsigned(ceil_div(n_groups, 1024)));
    const uint32_t* q32 = reinterpret_cast<const uint32_t*>(q);
    f32x4* o = static_cast<f32x4*>(out);
    if (scales_dtype == RQ_DTYPE_F32)
      int8_dequant_f32_kernel<RQ_DTYPE_F32><<<grid, 256, 0, stream>>>(q32, scales, sg, n_groups, o);
    else if (scales_dtype == RQ_DTYPE_BF16)
      int8_dequant_f32_kernel<RQ_DTYPE_BF16><<<grid, 256, 0, stream>>>(q32, scales, sg, n_groups, o);
    else
      int8_dequant_f32_kernel<RQ_DTYPE_F16><<<grid, 256, 0, stream>>>(q32, scales, sg, n_groups, o);
    done = n_groups * 4;
    if (done == n_out) return rq_check_launch();
  } else if (out_dtype != RQ_DTYPE_F32 && seg % 8 == 0 && aligned(q, 8) && aligned(out, 16) && n_out >= 8) {
    const int64_t n_groups = n_out / 8, sg = seg / 8;
    const dim3 grid(unsigned(ceil_div(n_groups, 1024)));
    const uint32_t* q32 = reinterpret_cast<const uint32_t*>(q);
    u32x4* o = static_cast<u32x4*>(out);
    auto run = [&](auto odt, auto sdt) {
      int8_dequant16_kernel<decltype(odt)::value, decltype(sdt)::value><<<grid, 256, 0, stream>>>(
          q32, scales, sg, n_groups, o);
    };
    using BF = std::integral_constant<int, RQ_DTYPE_BF16>;
    using F16 = std::integral_constant<int, RQ_DTYPE_F16>;
    using F32 = std::integral_constant<int, RQ_DTYPE_F32>;
    if (out_dtype == RQ_DTYPE_BF16) {
      if (scales_dtype == RQ_DTYPE_F32) run(BF{}, F32{});
      else if (scales_dtype == RQ_DTYPE_BF16) run(BF{}, BF{});
      else run(BF{}, F16{});
    } else {
      if (scales_dtype == RQ_DTYPE_F32) run(F16{}, F32{});
      else if (scales_dtype == RQ_DTYPE_BF16) run(F16{}, BF{});
      else run(F16{}, F16{});
    }
    done = n_groups * 8;
    if (done == n_out) return rq_check_launch();
  }
  dim3 grid(unsigned(ceil_div(n_out - done, 256)));
  RQ_DISPATCH_DT(out_dtype, ODT, int8_dequant_kernel<ODT><<<grid, 256, 0, stream>>>(
                                     q, scales, scales_dtype, seg, out, done, n_out));
  return rq_check_launch();
}
