// Shared device/host helpers for the rocm-qlora MI355X (gfx950) kernels.
//
// Numeric conventions follow the PyTorch CPU semantics that rocm_qlora's
// quantized-linear path is written in (quantization/quant_ops.py,
// quantization/double_quant.py): reduced-precision arithmetic is done in fp32
// and rounded to the storage type with round-to-nearest-even; divisions are
// IEEE correctly rounded (hipcc's default for fp32 '/').
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rocm_qlora_amd.h"

namespace rq {

// ---------------------------------------------------------------------------
// NF4 code book.  quant_ops.py:10-15 lists 16 Python doubles; torch rounds
// them to fp32 (quant_ops.py:87, :134).  The fp32 bit patterns are written out
// so no decimal-literal double rounding can creep in.
// ---------------------------------------------------------------------------
constexpr uint32_t kNF4Bits[16] = {
    0xBF800000u, 0xBF3239B1u, 0xBF066B30u, 0xBECA32A0u,
    0xBE91A24Du, 0xBE3D353Fu, 0xBDBA7871u, 0x00000000u,
    0x3DA2FAFFu, 0x3E24CAE3u, 0x3E7C04DDu, 0x3EAD033Au,
    0x3EE1A4B8u, 0x3F1007ABu, 0x3F3913B3u, 0x3F800000u};

// fp32 value of the clamp floor `1e-12` once cast to each storage dtype
// (torch.clamp(min=1e-12) casts the bound to the tensor dtype; fp16 underflows
// to zero).
constexpr uint32_t kClampF32 = 0x2B8CBCCCu;  // fp32(1e-12)
constexpr uint32_t kClampBF16 = 0x2B8D0000u; // bf16(1e-12)

// Native clang vector types (required by the nontemporal load/store builtins
// and by the MFMA builtins).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// bf16 <-> fp32 -------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return u2f(uint32_t(b) << 16); }

// Round-to-nearest-even fp32 -> bf16 bits.  NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return uint16_t((u >> 16) | 0x0040u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// fp16 <-> fp32 (hardware conversions are IEEE RNE) -------------------------
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return float(__builtin_bit_cast(_Float16, h));
}
// Keeps an fp32 value opaque to the instruction selector, so that the fp16
// narrowing after it stays a separate rounding: without it the compiler folds
// fptrunc(fmul / fadd) into one v_fma_mix{lo,hi}_f16, which rounds the exact
// product once to fp16 instead of first to fp32 -- a one-ulp difference
// whenever the fp32 result lands on an fp16 rounding tie.  Emits nothing.
__device__ __forceinline__ float f16_narrowing_barrier(float f) {
  asm("" : "+v"(f));
  return f;
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f16_narrowing_barrier(f)));
}

// Load/store one element of a runtime-selected float dtype ------------------
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dt) {
  if (dt == RQ_DTYPE_F32) return static_cast<const float*>(p)[i];
  if (dt == RQ_DTYPE_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// Round an fp32 value to the storage dtype and back (the value torch would
// hold after an op whose result dtype is `dt`).
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == RQ_DTYPE_BF16) return bf16_to_f32(f32_to_bf16_rne(v));
  if (dt == RQ_DTYPE_F16) return f16_to_f32(f32_to_f16_rne(v));
  return v;
}

__device__ __forceinline__ void store_from_f32(void* p, int64_t i, int dt, float v) {
  if (dt == RQ_DTYPE_F32) static_cast<float*>(p)[i] = v;
  else if (dt == RQ_DTYPE_BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(v);
  else static_cast<uint16_t*>(p)[i] = f32_to_f16_rne(v);
}

// NaN-propagating max of |v| (torch's max reduction returns NaN if any input
// is NaN; fmaxf would drop it).
__device__ __forceinline__ float absmax_nan(float m, float v) {
  float a = fabsf(v);
  return (a > m || a != a) ? a : m;
}
__device__ __forceinline__ float max_nan(float m, float a) {
  return (a > m || a != a || m != m) ? ((m != m) ? m : a) : m;
}

// RND_DT(RN32(x / s)) -- a tensor division in a 16-bit dtype as torch's
// CPU kernels compute it -- given rs = RN32(1 / s).
//
// For 16-bit DT the correctly rounded quotient is needed only up to its
// rounding to DT.  When rs is finite, r = RN32(x * rs) lies within 2 fp32
// ulps of RN32(x / s) (|rs - 1/s| <= 2^-24 / s, so |x * rs - x/s| <= one ulp
// of x/s, plus half an ulp for each of the two roundings), and RND_DT changes
// value only at the fp32 numbers whose bits below DT's precision are exactly
// the midpoint pattern (bf16: low 16 bits 0x8000; fp16 normals: low 13 bits
// 0x1000).  So RND_DT(r) = RND_DT(RN32(x / s)) unless those bits of r are
// within 4 of the midpoint, r is not finite (an infinite x or rs, a NaN) or
// |r| is below fp16's normal range (whose rounding drops more bits); those
// rare elements divide exactly.  (x = 0 with s = 0 or s = inf gives the same
// NaN or signed zero either way.)  fp32 input divides exactly.
template <int DT>
__device__ __forceinline__ float div_round(float x, float s, float rs) {
  if constexpr (DT == RQ_DTYPE_F32) {
    return __fdiv_rn(x, s);
  } else {
    constexpr uint32_t kLow = DT == RQ_DTYPE_BF16 ? 0xFFFFu : 0x1FFFu;
    constexpr uint32_t kMid = DT == RQ_DTYPE_BF16 ? 0x8000u : 0x1000u;
    float r = __fmul_rn(x, rs);
    const uint32_t b = f2u(r);
    bool exact = ((b & kLow) - (kMid - 4u)) <= 8u || (b & 0x7F800000u) == 0x7F800000u;
    if constexpr (DT == RQ_DTYPE_F16) exact = exact || (b & 0x7FFFFFFFu) < 0x38800000u;  // |r| < 2^-14
    if (exact) r = __fdiv_rn(x, s);
    return round_to(r, DT);
  }
}

// RN32(1 / s) for div_round (one correctly rounded division per scale).
__device__ __forceinline__ float recip_rn(float s) { return __fdiv_rn(1.0f, s); }

// torch.clamp(s, min=1e-12) in storage dtype `dt` (NaN propagates).
__device__ __forceinline__ float clamp_floor(float s, int dt) {
  float lo = (dt == RQ_DTYPE_F32) ? u2f(kClampF32) : (dt == RQ_DTYPE_BF16 ? u2f(kClampBF16) : 0.0f);
  return (s != s) ? s : fmaxf(s, lo);
}

// ---------------------------------------------------------------------------
// float8_e4m3fnuz: sign bit 7, 4 exponent bits (bias 8), 3 mantissa bits; no
// infinities, no negative zero, 0x80 is the only NaN; max finite 240.
// ---------------------------------------------------------------------------
__host__ __device__ inline float fnuz_to_f32(uint8_t c) {
  if (c == 0x80) return __builtin_nanf("");
  uint32_t e = (c >> 3) & 0xF, m = c & 0x7;
  float mag;
  if (e == 0) {
    mag = float(m) * (1.0f / 1024.0f);              // m * 2^-10
  } else {
    // (8 + m) * 2^(e - 11), built exactly from exponent bits
    uint32_t bits = ((e - 8 + 127) << 23) | (m << 20);
    mag = __builtin_bit_cast(float, bits);
  }
  return (c & 0x80) ? -mag : mag;
}

// fp32 -> e4m3fnuz with round-to-nearest-even.  |v| that rounds to >= 256, and
// NaN, give 0x80 (the format's NaN), as torch's cast does; values that round to
// zero give +0 (the format has no -0).
__host__ __device__ inline uint8_t f32_to_fnuz_rne(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 0x80;             // NaN
  if (a >= 0x43800000u) return 0x80;            // >= 256 (incl. inf)
  uint32_t code;
  if (a < 0x3C000000u) {                        // below 2^-7: subnormal range
    // quantum 2^-10: q = round_even(|v| * 2^10), exact scaling by 2^10
    float s = __builtin_bit_cast(float, a) * 1024.0f;
    uint32_t sb = __builtin_bit_cast(uint32_t, s);
    // round_even of s in [0, 8): manual RNE on the fp32 encoding
    int32_t ex = int32_t((sb >> 23) & 0xFF) - 127;
    uint32_t q;
    if (sb == 0) {
      q = 0;
    } else if (ex < -1) {
      q = 0;                                    // s < 0.5
    } else {
      uint32_t mant = (sb & 0x7FFFFFu) | 0x800000u;
      int32_t sh = 23 - ex;                     // bits below the integer point
      uint32_t ip = mant >> sh;
      uint32_t rem = mant & ((1u << sh) - 1u);
      uint32_t half = 1u << (sh - 1);
      if (rem > half || (rem == half && (ip & 1u))) ip += 1;
      q = ip;
    }
    code = q;                                   // q == 8 lands on 2^-7 (e=1,m=0)
  } else {
    uint32_t e = ((a >> 23) & 0xFF) - 127 + 8;  // 1..15
    uint32_t mant = a & 0x7FFFFFu;
    uint32_t keep = mant >> 20;                 // top 3 bits
    uint32_t rem = mant & 0xFFFFFu;
    code = (e << 3) | keep;
    if (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) code += 1;
    if (code >= 0x80) return 0x80;              // rounded past 240 -> NaN
  }
  if (code == 0) return 0;
  return uint8_t(code | sign);
}

// float8_e4m3fn (OCP, the gfx950 MFMA format): bias 7, max 448, 0x7F/0xFF NaN.
// fnuz value v has the same bit pattern as fn value 2v; the value-preserving
// re-encoding used for the MFMA operands is f32_to_fn_rne(fnuz_to_f32(c)).
__host__ __device__ inline uint8_t f32_to_fn_rne(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 0x7F;
  if (a >= 0x43E80000u) return uint8_t(0x7E | sign);   // >= 464: saturate (not hit)
  uint32_t code;
  if (a < 0x3C800000u) {                               // below 2^-6: subnormal
    float s = __builtin_bit_cast(float, a) * 512.0f;   // quantum 2^-9
    uint32_t sb = __builtin_bit_cast(uint32_t, s);
    int32_t ex = int32_t((sb >> 23) & 0xFF) - 127;
    uint32_t q;
    if (sb == 0 || ex < -1) {
      q = 0;
    } else {
      uint32_t mant = (sb & 0x7FFFFFu) | 0x800000u;
      int32_t sh = 23 - ex;
      uint32_t ip = mant >> sh;
      uint32_t rem = mant & ((1u << sh) - 1u);
      uint32_t half = 1u << (sh - 1);
      if (rem > half || (rem == half && (ip & 1u))) ip += 1;
      q = ip;
    }
    code = q;
  } else {
    uint32_t e = ((a >> 23) & 0xFF) - 127 + 7;
    uint32_t mant = a & 0x7FFFFFu;
    uint32_t keep = mant >> 20;
    uint32_t rem = mant & 0xFFFFFu;
    code = (e << 3) | keep;
    if (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) code += 1;
    if (code >= 0x7F) code = 0x7E;                      // saturate at 448
  }
  return uint8_t(code | sign);
}

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Raw buffer accesses (stride 0, 32-bit byte offsets, bounds checked against
// the resource's size: an access past it reads zero and writes nothing)
// ---------------------------------------------------------------------------
// Word 3 of a raw buffer resource on gfx9-family GPUs, gfx950 included:
// 32-bit data, bounds checked against num_records.
constexpr int kBufferRsrcWord3 = 0x00020000;
// Cache policy of a buffer load or store that is device coherent (sc1), as
// the agent-scope atomic loads and stores are.
constexpr int kCoherent = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, int(bytes), kBufferRsrcWord3);
}
// A buffer offset past the end of any resource of at most 0xFFFFFFF0 bytes:
// a load there returns zero.  (kOobOffset + 16 wraps to 0, so a second
// piece of a dead lane needs its own select.)
constexpr uint32_t kOobOffset = 0xFFFFFFF0u;
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return uint32_t(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
// voff: per-lane byte offset; soff: a wave-uniform byte offset added to it
__device__ __forceinline__ u32x4 buf_load16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kCoherent));
}
__device__ __forceinline__ void buf_store16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, kCoherent);
}

}  // namespace rq
