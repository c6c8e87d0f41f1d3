// Device and host helpers shared by the NF4 linear kernels (GEMV, GEMM, dX).
#pragma once

#include "rq_mfma.h"
#include "rq_linear.h"

namespace rq {

// ---------------------------------------------------------------------------
// Element loads with the dtype fixed at compile time (no branches in the
// kernels' load sequences).
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float ld_f32(const void* __restrict__ p, int64_t i) {
  if constexpr (DT == RQ_DTYPE_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == RQ_DTYPE_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// Scale providers: the fp32 scale of flat block b in two steps -- load()
// issues the loads and returns raw bits, value() converts them where the
// scale is used (single quantization: absmax of dtype SDT; double
// quantization: c2 code times its c2_scales entry).
template <int SDT>
struct ScaleAbsmax {
  static constexpr int kLoads = 1;  // vector-memory loads per scale
  static constexpr bool kTransposed = false;  // index n * blocks_per_row + block
  const void* p;
  typedef uint32_t Raw;
  __device__ __forceinline__ Raw load(int64_t b) const {
    if constexpr (SDT == RQ_DTYPE_F32) return static_cast<const uint32_t*>(p)[b];
    else return static_cast<const uint16_t*>(p)[b];
  }
  __device__ __forceinline__ float value(Raw r) const {
    if constexpr (SDT == RQ_DTYPE_F32) return u2f(r);
    else if constexpr (SDT == RQ_DTYPE_BF16) return bf16_to_f32(uint16_t(r));
    else return f16_to_f32(uint16_t(r));
  }
  __device__ __forceinline__ float operator()(int64_t b) const { return value(load(b)); }
};

template <int SDT>
struct ScaleDQ {
  static constexpr int kLoads = 2;  // vector-memory loads per scale
  static constexpr bool kTransposed = false;
  const uint8_t* c2;
  const void* c2s;
  int fmt;
  int bs2_shift;  // log2(block2), or -1 when block2 is not a power of two
  int64_t bs2;
  struct Raw {
    uint32_t code, hi;
  };
  __device__ __forceinline__ Raw load(int64_t b) const {
    const int64_t g = bs2_shift >= 0 ? (b >> bs2_shift) : b / bs2;
    Raw r;
    r.code = c2[b];
    if constexpr (SDT == RQ_DTYPE_F32) r.hi = static_cast<const uint32_t*>(c2s)[g];
    else r.hi = static_cast<const uint16_t*>(c2s)[g];
    return r;
  }
  __device__ __forceinline__ float value(Raw r) const {
    float hi;
    if constexpr (SDT == RQ_DTYPE_F32) hi = u2f(r.hi);
    else if constexpr (SDT == RQ_DTYPE_BF16) hi = bf16_to_f32(uint16_t(r.hi));
    else hi = f16_to_f32(uint16_t(r.hi));
    const uint8_t c = uint8_t(r.code);
    const float lo = fmt == RQ_C2_FP8_E4M3FNUZ ? fnuz_to_f32(c) : __fdiv_rn(float(int8_t(c)), 127.0f);
    return __fmul_rn(lo, hi);
  }
  __device__ __forceinline__ float operator()(int64_t b) const { return value(load(b)); }
};

// Decoded fp32 scales stored transposed, [blocks_per_row][rows]: the dX
// producer's scales of one step (64 consecutive weight rows, one block)
// are then 256 contiguous bytes instead of 64 rows' scattered words.
struct ScaleT {
  static constexpr int kLoads = 1;
  static constexpr bool kTransposed = true;  // index block * rows + n
  const void* p;
  typedef uint32_t Raw;
  __device__ __forceinline__ Raw load(int64_t b) const { return static_cast<const uint32_t*>(p)[b]; }
  __device__ __forceinline__ float value(Raw r) const { return u2f(r); }
  __device__ __forceinline__ float operator()(int64_t b) const { return value(load(b)); }
};

// 8 consecutive activations of one row as an MFMA operand.
__device__ __forceinline__ u32x4 load_x8(const uint16_t* __restrict__ p, bool vec) {
  if (vec) return *reinterpret_cast<const u32x4*>(p);
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = uint32_t(p[2 * j]) | (uint32_t(p[2 * j + 1]) << 16);
  return u32x4{w[0], w[1], w[2], w[3]};
}

// ---------------------------------------------------------------------------
// Epilogue shared by the GEMV, the split-K finisher and the GEMM.  Every
// global load of a finishing step is issued before its first use, so a tile
// pays one memory round trip, not one per LoRA rank.
// ---------------------------------------------------------------------------
template <int XT>
__device__ __forceinline__ float finish_value(const LinearEpi& e, int64_t n, float acc, float lora_sum) {
  float v = acc;
  if (e.bias) v = __fadd_rn(v, round_x<XT>(load_as_f32(e.bias, n, e.bias_dt)));
  v = round_x<XT>(v);
  if (e.rank > 0) {
    const float l = round_x<XT>(__fmul_rn(round_x<XT>(lora_sum), e.scaling));
    v = round_x<XT>(__fadd_rn(v, l));
  }
  return v;
}

// Stage RND(u[m, :]) for rows [m0, m0 + rows) into LDS: the sum of the
// u_splits partial products lora_u_kernel wrote (8 loads in flight).
template <int XT>
__device__ __forceinline__ void stage_u(const LinearEpi& e, int64_t M, int64_t m0, int rows, float* us,
                                        int tid, int nthreads) {
  if (e.rank <= 0) return;
  const int total = rows * e.rank;
  for (int i = tid; i < total; i += nthreads) {
    const int64_t m = m0 + i / e.rank;
    const int j = i % e.rank;
    float s = 0.0f;
    if (m < M) {
      for (int k0 = 0; k0 < e.u_splits; k0 += 8) {
        float p[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
          p[k] = (k0 + k < e.u_splits) ? e.u[(int64_t(k0 + k) * M + m) * e.rank + j] : 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (k0 + k < e.u_splits) s = __fadd_rn(s, p[k]);
      }
    }
    us[i] = round_x<XT>(s);
  }
}

// One element of a runtime float dtype as two raw 16-bit loads, the same
// whatever the dtype (fp32: both halves; 16-bit: the element twice), so that
// no load depends on a branch.  The halves stay apart until raw_to_f32, at
// the point of use, so carrying them never forces a wait on the load.
struct Raw16x2 {
  uint32_t lo, hi;
};
__device__ __forceinline__ Raw16x2 load_raw(const void* p, int64_t i, int dt) {
  const uint16_t* h = static_cast<const uint16_t*>(p);
  const int64_t lo = dt == RQ_DTYPE_F32 ? 2 * i : i;
  const int64_t hi = dt == RQ_DTYPE_F32 ? 2 * i + 1 : i;
  return Raw16x2{h[lo], h[hi]};
}
__device__ __forceinline__ float raw_to_f32(const Raw16x2& r, int dt) {
  return dt == RQ_DTYPE_F32 ? u2f(r.lo | (r.hi << 16))
                            : (dt == RQ_DTYPE_BF16 ? bf16_to_f32(uint16_t(r.lo)) : f16_to_f32(uint16_t(r.lo)));
}

// LoRA A row chunk: 8 consecutive values of A (fp32 or 16-bit), rounded to
// the activation dtype as lora_layer.py:67's `self.lora_A.to(x.dtype)` does.
template <int XT>
__device__ __forceinline__ u32x4 load_a8(const void* p, int dt, int64_t off, bool live, bool vec32) {
  if (!live) return u32x4{0u, 0u, 0u, 0u};
  if (dt == RQ_DTYPE_F32 && vec32) {
    const f32x4* v = reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + off);
    const f32x4 a = v[0], b = v[1];
    return u32x4{cvt_pk<XT>(a.x, a.y), cvt_pk<XT>(a.z, a.w), cvt_pk<XT>(b.x, b.y), cvt_pk<XT>(b.z, b.w)};
  }
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = cvt_pk<XT>(load_as_f32(p, off + 2 * j, dt), load_as_f32(p, off + 2 * j + 1, dt));
  return u32x4{w[0], w[1], w[2], w[3]};
}

// 8 consecutive LoRA values loaded raw as 16-byte pieces (fp32: lo holds
// the first 4, hi the next 4; 16-bit: lo holds all 8), rounded to the
// activation dtype as load_a8 rounds them.
template <int XT>
__device__ __forceinline__ u32x4 raw8_to_x(const u32x4& lo, const u32x4& hi, int dt) {
  if (dt == RQ_DTYPE_F32)
    return u32x4{cvt_pk<XT>(u2f(lo.x), u2f(lo.y)), cvt_pk<XT>(u2f(lo.z), u2f(lo.w)), cvt_pk<XT>(u2f(hi.x), u2f(hi.y)),
                 cvt_pk<XT>(u2f(hi.z), u2f(hi.w))};
  const uint32_t w[4] = {lo.x, lo.y, lo.z, lo.w};
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = dt == RQ_DTYPE_BF16 ? bf16_to_f32(uint16_t(w[j])) : f16_to_f32(uint16_t(w[j]));
    const float b = dt == RQ_DTYPE_BF16 ? bf16_to_f32(uint16_t(w[j] >> 16)) : f16_to_f32(uint16_t(w[j] >> 16));
    o[j] = cvt_pk<XT>(a, b);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// 8 consecutive values p[off + e] (e < n_live, zeros past), rounded to the
// activation dtype; the vector path when all 8 are live.
template <int XT>
__device__ __forceinline__ u32x4 load_a8_masked(const void* p, int dt, int64_t off, int n_live, bool vec32) {
  if (n_live >= 8) return load_a8<XT>(p, dt, off, true, vec32);
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = cvt_pk<XT>(2 * j < n_live ? load_as_f32(p, off + 2 * j, dt) : 0.0f,
                      2 * j + 1 < n_live ? load_as_f32(p, off + 2 * j + 1, dt) : 0.0f);
  return u32x4{w[0], w[1], w[2], w[3]};
}

// 8 values p[off + e * stride] (e < n_live, zeros past), rounded to the
// activation dtype.
template <int XT>
__device__ __forceinline__ u32x4 load_a8_strided(const void* p, int dt, int64_t off, int64_t stride, int n_live) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = cvt_pk<XT>(2 * j < n_live ? load_as_f32(p, off + (2 * j) * stride, dt) : 0.0f,
                      2 * j + 1 < n_live ? load_as_f32(p, off + (2 * j + 1) * stride, dt) : 0.0f);
  return u32x4{w[0], w[1], w[2], w[3]};
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------
inline int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

inline int pow2_shift(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

}  // namespace rq
