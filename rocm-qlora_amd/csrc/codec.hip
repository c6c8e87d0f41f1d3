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
#include "nf4_tables.h"
#include "rq_launch.h"

namespace rq {

// ---------------------------------------------------------------------------
// NF4 decision: idx = argmin_i |n - T_i| (first minimum), via the exact cell
// table (gen_nf4_tables.py).  n is the fp32 value of the normalised weight
// (already rounded to the input dtype).  NaN -> 0, as torch.argmin returns the
// first NaN.
// ---------------------------------------------------------------------------
struct NF4CellTable {
  uint32_t thr[64];
  uint32_t base[64];
};

__device__ __forceinline__ void load_cell_table(NF4CellTable* t) {
  for (int i = threadIdx.x; i < 64; i += blockDim.x) {
    t->thr[i] = kNF4CellThr[i];
    t->base[i] = kNF4CellBase[i];
  }
}

__device__ __forceinline__ uint32_t nf4_decide(float n, const NF4CellTable* t) {
  float c = __fmul_rn(__fadd_rn(n, 1.0f), 32.0f);
  c = fminf(fmaxf(c, 0.0f), 63.0f);   // NaN -> 0 (v_max returns the non-NaN operand)
  int g = int(c);
  return t->base[g] + (n > u2f(t->thr[g]) ? 1u : 0u);
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
struct ScaleSingle {
  const void* absmax;
  int dt;
  __device__ __forceinline__ float operator()(int64_t b) const { return load_as_f32(absmax, b, dt); }
};

struct ScaleDouble {
  const uint8_t* c2;
  const void* c2s;
  int c2s_dt;
  int fmt;
  int64_t block2;
  __device__ __forceinline__ float operator()(int64_t b) const {
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

template <int ODT>
__global__ __launch_bounds__(256) void int8_dequant_kernel(const int8_t* __restrict__ q, const void* scales,
                                                           int sdt, int64_t seg, void* __restrict__ out,
                                                           int64_t n_out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
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
  if (log2_l >= 0 && aligned(packed, 4)) {
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
  return nf4_dequant_launch(packed, ScaleSingle{absmax, absmax_dtype}, n_packed, block_size, out,
                            out_dtype, n_out, stream);
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
  return nf4_dequant_launch(packed, ScaleDouble{c2, c2_scales, c2s_dtype, c2_format, block2},
                            n_packed, block1, out, out_dtype, n_out, stream);
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
  dim3 grid(unsigned(ceil_div(n_out, 256)));
  RQ_DISPATCH_DT(out_dtype, ODT, int8_dequant_kernel<ODT><<<grid, 256, 0, stream>>>(
                                     q, scales, scales_dtype, seg, out, n_out));
  return rq_check_launch();
}
