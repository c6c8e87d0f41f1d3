// Fused AdamW step over many tensors (the LoRA parameters), for gfx950.
//
// PagedAdamW.step (optim/paged_adamw.py:67-127, the update :84-113)
// updates each parameter with its own sequence of torch ops, each state pair
// copied host -> device and back around them.  Here one launch updates every tensor of the step: each
// 2048-element chunk of the (padded, concatenated) state buffers is one
// workgroup of 256 threads, 8 consecutive elements per thread, and the
// workgroup finds its tensor by binary search over the tensors' state
// offsets in a small descriptor table.
//
// Per element, the reference's ops with the roundings torch's GPU kernels
// give them (the reference moves the states to the parameter's device and
// updates there; its element-wise kernels evaluate `a + alpha * b`,
// `a + alpha * (b * c)` and `a + alpha * (b / c)` in fp32 with the multiply
// and add fused, and divide by a host scalar by multiplying with its
// reciprocal, taken in double and rounded to fp32):
//   p  = RND_p(RND(p * decay))                 p.mul_(1 - lr * wd)     (wd != 0)
//   m  = fma(1 - b1, g, RND(m * b1))           exp_avg.mul_(b1).add_(g, alpha=1 - b1)
//   v  = fma(1 - b2, RND(g * g), RND(v * b2))  exp_avg_sq.mul_(b2).addcmul_(g, g, value=1 - b2)
//   d  = RND(RND(sqrt(v)) * RND(1 / sqrt(bc2))) + eps
//                                              (exp_avg_sq.sqrt() / bc2 ** 0.5).add_(eps)
//   p  = RND_p(fma(-step, RND(m / d), p))      p.addcdiv_(exp_avg, denom, value=-step_size)
// with RND_p the rounding to the parameter's dtype (fp32, bf16, fp16), m and
// v fp32, and the square root and division correctly rounded.  The memory
// traffic is 4 reads and 3 writes per element (p, g, m, v): HBM-bound.
#include "rq_common.h"
#include "rq_launch.h"

namespace rq {

constexpr int kAdamThreads = 256;
constexpr int kAdamPer = 8;
static_assert(kAdamThreads * kAdamPer == RQ_ADAMW_CHUNK, "chunk = one workgroup's elements");
static_assert(sizeof(rq_adamw_tensor) == 72, "descriptor layout");

template <int DT>
__device__ __forceinline__ float round_param(float v) {
  if constexpr (DT == RQ_DTYPE_F32) return v;
  else return round_to(v, DT);
}

template <int DT>
__device__ __forceinline__ void adam_update(const rq_adamw_tensor& e, float& p, float g, float& m, float& v) {
  if (e.apply_decay) p = round_param<DT>(__fmul_rn(p, e.decay));
  m = __builtin_fmaf(e.one_minus_beta1, g, __fmul_rn(m, e.beta1));
  v = __builtin_fmaf(e.one_minus_beta2, __fmul_rn(g, g), __fmul_rn(v, e.beta2));
  // __builtin_sqrtf is correctly rounded under hipcc's default fp32 options
  // (HIP's __fsqrt_rn is the approximate hardware square root unless
  // OCML_BASIC_ROUNDED_OPERATIONS is defined)
  const float d = __fadd_rn(__fmul_rn(__builtin_sqrtf(v), e.inv_bias_correction2_sqrt), e.eps);
  p = round_param<DT>(__builtin_fmaf(e.neg_step_size, __fdiv_rn(m, d), p));
}

// 8 elements from offset i of a tensor of dtype DT (16-byte aligned run).
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t i, float* out) {
  if constexpr (DT == RQ_DTYPE_F32) {
    const f32x4* q = reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + i);
    const f32x4 a = q[0], b = q[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i);
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint16_t h = uint16_t(d[k >> 1] >> (16 * (k & 1)));
      out[k] = DT == RQ_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
    }
  }
}

template <int DT>
__device__ __forceinline__ void store8(void* base, int64_t i, const float* in) {
  if constexpr (DT == RQ_DTYPE_F32) {
    f32x4* q = reinterpret_cast<f32x4*>(static_cast<float*>(base) + i);
    q[0] = f32x4{in[0], in[1], in[2], in[3]};
    q[1] = f32x4{in[4], in[5], in[6], in[7]};
  } else {
    uint32_t d[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = DT == RQ_DTYPE_BF16 ? f32_to_bf16_rne(in[2 * k]) : f32_to_f16_rne(in[2 * k]);
      const uint32_t hi = DT == RQ_DTYPE_BF16 ? f32_to_bf16_rne(in[2 * k + 1]) : f32_to_f16_rne(in[2 * k + 1]);
      d[k] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + i) = u32x4{d[0], d[1], d[2], d[3]};
  }
}

template <int DT>
__device__ __forceinline__ void adam_run(const rq_adamw_tensor& e, int64_t i0, float* m, float* v) {
  const int64_t n = e.numel - i0;  // > 0
  const bool vec = n >= kAdamPer && ((reinterpret_cast<uintptr_t>(e.param) | reinterpret_cast<uintptr_t>(e.grad)) % 16) == 0;
  if (vec) {
    float p8[8], g8[8], m8[8], v8[8];
    load8<DT>(e.param, i0, p8);
    load8<DT>(e.grad, i0, g8);
    load8<RQ_DTYPE_F32>(m, 0, m8);
    load8<RQ_DTYPE_F32>(v, 0, v8);
#pragma unroll
    for (int k = 0; k < 8; ++k) adam_update<DT>(e, p8[k], g8[k], m8[k], v8[k]);
    store8<DT>(e.param, i0, p8);
    store8<RQ_DTYPE_F32>(m, 0, m8);
    store8<RQ_DTYPE_F32>(v, 0, v8);
    return;
  }
  const int cnt = n < kAdamPer ? int(n) : kAdamPer;
  for (int k = 0; k < cnt; ++k) {
    float p = load_as_f32(e.param, i0 + k, DT), mk = m[k], vk = v[k];
    adam_update<DT>(e, p, load_as_f32(e.grad, i0 + k, DT), mk, vk);
    store_from_f32(e.param, i0 + k, DT, p);
    m[k] = mk;
    v[k] = vk;
  }
}

// Chunks chunk0 + blockIdx.x of the state space; the state buffers hold
// the elements from chunk0 * RQ_ADAMW_CHUNK on.
__global__ __launch_bounds__(kAdamThreads) void adamw_kernel(const rq_adamw_tensor* __restrict__ tab, int n,
                                                             int64_t chunk0, float* __restrict__ m_base,
                                                             float* __restrict__ v_base) {
  const int64_t c = chunk0 + blockIdx.x;
  const int64_t s = c * RQ_ADAMW_CHUNK;
  // the last tensor whose state offset is at or below s
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tab[mid].state_offset <= s) lo = mid;
    else hi = mid - 1;
  }
  const rq_adamw_tensor e = tab[lo];
  if (e.state_offset > s) return;  // a gap before the first tensor
  const int64_t i0 = s - e.state_offset + int64_t(threadIdx.x) * kAdamPer;
  if (i0 >= e.numel) return;        // padding, or a tensor without a gradient this step
  const int64_t off = s - chunk0 * RQ_ADAMW_CHUNK + int64_t(threadIdx.x) * kAdamPer;
  float* m = m_base + off;
  float* v = v_base + off;
  if (e.dtype == RQ_DTYPE_F32) adam_run<RQ_DTYPE_F32>(e, i0, m, v);
  else if (e.dtype == RQ_DTYPE_BF16) adam_run<RQ_DTYPE_BF16>(e, i0, m, v);
  else adam_run<RQ_DTYPE_F16>(e, i0, m, v);
}

}  // namespace rq

extern "C" int rq_adamw_step(const rq_adamw_tensor* tensors, int64_t n_tensors, void* device_table,
                             int64_t device_table_bytes, int64_t chunk_begin, int64_t chunk_end, float* exp_avg,
                             float* exp_avg_sq, hipStream_t stream) {
  using namespace rq;
  if (!tensors || !device_table || !exp_avg || !exp_avg_sq) return RQ_ERR_NULL_POINTER;
  if (n_tensors <= 0 || n_tensors > 0x7FFFFFFF) return RQ_ERR_BAD_SHAPE;
  const int64_t table_bytes = n_tensors * int64_t(sizeof(rq_adamw_tensor));
  if (device_table_bytes < table_bytes) return RQ_ERR_WORKSPACE;
  if (!aligned(device_table, 8) || !aligned(exp_avg, 16) || !aligned(exp_avg_sq, 16)) return RQ_ERR_BAD_ALIGNMENT;
  if (chunk_begin < 0 || chunk_end <= chunk_begin || chunk_end - chunk_begin > 0x7FFFFFFF) return RQ_ERR_BAD_SHAPE;
  int64_t prev_end = 0;
  for (int64_t t = 0; t < n_tensors; ++t) {
    const rq_adamw_tensor& e = tensors[t];
    if (!e.param || !e.grad) return RQ_ERR_NULL_POINTER;
    if (!valid_float_dtype(e.dtype)) return RQ_ERR_BAD_DTYPE;
    if (e.numel < 0 || e.state_offset < prev_end || e.state_offset % RQ_ADAMW_CHUNK != 0) return RQ_ERR_BAD_SHAPE;
    prev_end = e.state_offset + (e.numel + RQ_ADAMW_CHUNK - 1) / RQ_ADAMW_CHUNK * RQ_ADAMW_CHUNK;
  }
  if (hipMemcpyAsync(device_table, tensors, size_t(table_bytes), hipMemcpyHostToDevice, stream) != hipSuccess)
    return RQ_ERR_HIP;
  adamw_kernel<<<unsigned(chunk_end - chunk_begin), kAdamThreads, 0, stream>>>(
      static_cast<const rq_adamw_tensor*>(device_table), int(n_tensors), chunk_begin, exp_avg, exp_avg_sq);
  return rq_check_launch();
}
