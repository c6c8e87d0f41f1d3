// gfx950 matrix-core helpers shared by the NF4 linear kernels.
//
// Lane layouts (checked on the hardware for v_mfma_f32_16x16x32_{bf16,f16}):
//   A[16 x 32]: lane l holds A[l % 16][8 * (l / 16) + e], e = 0..7
//   B[32 x 16]: lane l holds B[8 * (l / 16) + e][l % 16]
//   D[16 x 16]: lane l, register r holds D[4 * (l / 16) + r][l % 16]
// and for v_mfma_f32_32x32x16_{bf16,f16}:
//   A[32 x 16]: lane l holds A[l % 32][8 * (l / 32) + e]
//   B[16 x 32]: lane l holds B[8 * (l / 32) + e][l % 32]
//   D[32 x 32]: lane l, register r holds D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32]
#pragma once

#include "rq_common.h"

namespace rq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int XT>
__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (XT == RQ_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

template <int XT>
__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (XT == RQ_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Two fp32 values rounded (RNE, v_cvt_pk_*_f32) into one dword of 16-bit
// operand elements, `lo` in the low half.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <int XT>
__device__ __forceinline__ uint32_t cvt_pk(float lo, float hi) {
  const f32x2 v = {lo, hi};
  if constexpr (XT == RQ_DTYPE_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  } else {
    const f32x2 o = {f16_narrowing_barrier(lo), f16_narrowing_barrier(hi)};  // two roundings, as written
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(o, f16x2));
  }
}

// Round-to-nearest-even of an fp32 value to the 16-bit operand type, as bits
// (the hardware conversions: v_cvt_pk_bf16_f32 / v_cvt_f16_f32, which round
// finite values exactly as torch's casts do; a NaN stays a quiet NaN).
template <int XT>
__device__ __forceinline__ uint32_t to_x16(float v) {
  if constexpr (XT == RQ_DTYPE_BF16) return cvt_pk<XT>(v, 0.0f) & 0xFFFFu;
  else return f32_to_f16_rne(v);
}

template <int XT>
__device__ __forceinline__ float from_x16(uint32_t b) {
  if constexpr (XT == RQ_DTYPE_BF16) return bf16_to_f32(uint16_t(b));
  else return f16_to_f32(uint16_t(b));
}

// RND: the fp32 value an fp32 -> operand-dtype -> fp32 round trip yields.
template <int XT>
__device__ __forceinline__ float round_x(float v) {
  if constexpr (XT == RQ_DTYPE_BF16) return u2f(cvt_pk<XT>(v, 0.0f) << 16);
  else return f16_to_f32(f32_to_f16_rne(v));
}

// RND of two values, by one conversion for bf16 (two for fp16).
template <int XT>
__device__ __forceinline__ void round2(float& x, float& y) {
  if constexpr (XT == RQ_DTYPE_BF16) {
    const uint32_t p = cvt_pk<XT>(x, y);
    x = u2f(p << 16);
    y = u2f(p & 0xFFFF0000u);
  } else {
    x = round_x<XT>(x);
    y = round_x<XT>(y);
  }
}

// ---------------------------------------------------------------------------
// Byte -> fp32 codebook pair table for exact dequantization.  Entry e (a
// packed NF4 byte) holds fp32 T[e & 15] (the even element) and T[e >> 4].
// Each lane multiplies by its block scale and rounds once, which reproduces
// the reference's RND(T[code] * scale) bit for bit.  The table is replicated
// 32 times (entry e, copy c at qword e * 32 + c, lane l uses copy l % 32):
// a ds_read_b64 serves 16 lanes per cycle, and those 16 lanes read 16
// distinct copies covering all 32 banks, so lookups never conflict.
// ---------------------------------------------------------------------------
constexpr int kF32PairLutQwords = 256 * 32;  // 64 KiB

// Fill by NT (512 or 1024) threads.  Thread t writes copy t % 32 of the
// entries whose low nibble is (t / 32) % 16 and whose high nibble is in its
// share of 0..15; each unrolled store's high-nibble value is an immediate, so
// the fill issues no loads at all.
__device__ __forceinline__ uint32_t nf4_bits(int i) {
  uint32_t v = kNF4Bits[0];
#pragma unroll
  for (int j = 1; j < 16; ++j) v = (i == j) ? kNF4Bits[j] : v;
  return v;
}

// The high nibbles a wave writes are the same in all its lanes and its low
// nibbles take two values (lanes 0-31, 32-63), so the code-book selections
// run on wave-uniform values (scalar ops) and one per-lane select remains.
template <int NT>
__device__ __forceinline__ void fill_f32pair_lut(u32x2* lut, int tid) {
  static_assert(NT == 512 || NT == 1024, "table fill expects 512 or 1024 threads");
  constexpr int kPer = 16 / (NT / 512);
  const int c = tid & 31, lo = (tid >> 5) & 15;
  const int lo0 = __builtin_amdgcn_readfirstlane((tid >> 5) & 15);  // lanes 0-31; lanes 32-63 hold lo0 + 1
  const int j0 = __builtin_amdgcn_readfirstlane(tid >> 9) * kPer;
  const uint32_t b0 = nf4_bits(lo0), b1 = nf4_bits((lo0 + 1) & 15);
  const uint32_t lo_bits = lo == lo0 ? b0 : b1;
#pragma unroll
  for (int j = 0; j < kPer; ++j) lut[(lo + 16 * (j0 + j)) * 32 + c] = u32x2{lo_bits, nf4_bits(j0 + j)};
}

// RND(T * s) for the 8 codes of one packed dword (k ascending), as an MFMA
// operand.  lane_off = (lane % 32) * 8 sits in byte 0; v_perm_b32 builds the
// byte address (code byte << 8) | lane_off.
template <int XT>
__device__ __forceinline__ u32x4 expand8_scaled(const u32x2* lut, uint32_t word, uint32_t lane_off, float s) {
  uint32_t r[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t addr = __builtin_amdgcn_perm(word, lane_off, 0x0C0C0000u | (uint32_t(4 + j) << 8));
    const u32x2 p = *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(lut) + addr);
    r[j] = cvt_pk<XT>(__fmul_rn(u2f(p.x), s), __fmul_rn(u2f(p.y), s));
  }
  return u32x4{r[0], r[1], r[2], r[3]};
}

}  // namespace rq
