/*
 * rocm_qlora_amd -- C ABI of the MI355X (gfx950) quantized-linear library.
 *
 * Every entry point takes plain device pointers, 64-bit sizes and dtype codes,
 * launches asynchronously on the given HIP stream, never allocates device
 * memory, never synchronises the host, and returns an rq status code
 * (RQ_OK == 0).  Argument validation happens before any launch, so a non-zero
 * status means nothing was enqueued (except RQ_ERR_HIP, reported from
 * hipGetLastError after a launch).
 *
 * Buffer layouts are the ones rocm_qlora's QuantLinear keeps in its
 * state_dict (quantization/quant_linear.py:38-53, double_quant.py:185-196):
 * flat row-major [N, K] weights, NF4 packed two codes per byte with the even
 * element in the low nibble (quant_ops.py:119-124), one absmax per block of
 * `block_size` consecutive flat elements.
 */
#ifndef ROCM_QLORA_AMD_H
#define ROCM_QLORA_AMD_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes for float tensors */
#define RQ_DTYPE_F32  0
#define RQ_DTYPE_BF16 1
#define RQ_DTYPE_F16  2

/* second-level (double-quant) code formats, double_quant.py:72-87 */
#define RQ_C2_FP8_E4M3FNUZ 0   /* torch.float8_e4m3fnuz codes */
#define RQ_C2_INT8         1   /* round(c1 / c2s * 127) int8 fallback */

/* weight formats of rq_merge_lora */
#define RQ_WEIGHT_NF4      0   /* flat packed NF4 codes, two per byte */
#define RQ_WEIGHT_INT8     1   /* flat int8 codes */

/* rounding of rq_merge_lora */
#define RQ_MERGE_SUM_THEN_ROUND  0   /* RND(W + d): LoRALinear.merge_lora */
#define RQ_MERGE_ROUND_THEN_SUM  1   /* RND(RND(W) + RND(d)): the export path */

/* status codes */
#define RQ_OK                 0
#define RQ_ERR_NULL_POINTER   1
#define RQ_ERR_BAD_DTYPE      2
#define RQ_ERR_BAD_SHAPE      3
#define RQ_ERR_BAD_ALIGNMENT  4
#define RQ_ERR_UNSUPPORTED    5
#define RQ_ERR_WORKSPACE      6
#define RQ_ERR_HIP            7
#define RQ_ERR_SCRATCH_LIMIT  8   /* needs more than rq_nf4_linear_noalloc's scratch */

/* Human-readable text for a status code (static storage). */
const char* rq_status_string(int status);

/* Library ABI version (major * 10000 + minor * 100 + patch). */
int rq_version(void);

/* Target architecture the code objects were built for ("gfx950"). */
const char* rq_build_arch(void);

/* Identifier of the graph capture active on `stream`, 0 when none (no
 * counterpart in the reference: for callers that keep one rq_nf4_linear
 * workspace per captured graph, since a graph's replays reuse the
 * workspace it was captured with). */
int rq_stream_capture_id(hipStream_t stream, uint64_t* id);

/* ------------------------------------------------------------------------
 * NF4 codec
 * ------------------------------------------------------------------------ */

/* Replaces quantize_int4(tensor, block_size) -- quant_ops.py:80-126.
 * w: `numel` elements of w_dtype.  The flat tensor is zero-padded to a
 * multiple of block_size (then to even), numel_padded = result.
 * packed: numel_padded / 2 bytes.  absmax: numel_padded / block_size values
 * of w_dtype (clamped at 1e-12 in that dtype, as torch.clamp does).
 * block_size must be even and >= 2. */
int rq_nf4_quantize(const void* w, int w_dtype, int64_t numel, int64_t block_size,
                    uint8_t* packed, void* absmax, hipStream_t stream);

/* Replaces dequantize_int4(packed, scales, block_size) -- quant_ops.py:128-150
 * followed by the caller's `[:n_out].to(out_dtype)` (quant_linear.py:191-193).
 * out[i] = dtype(T[code_i] * float(absmax[i / block_size])) for i < n_out,
 * n_out <= 2 * n_packed, (2 * n_packed) % block_size == 0. */
int rq_nf4_dequantize(const uint8_t* packed, const void* absmax, int absmax_dtype,
                      int64_t n_packed, int64_t block_size,
                      void* out, int out_dtype, int64_t n_out, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Double quantization of the NF4 absmax
 * ------------------------------------------------------------------------ */

/* Second stage of double_quantize -- double_quant.py:58-87.
 * c1: n_c1 absmax values of c1_dtype.  Zero-padded to a multiple of block2.
 * c2: ceil(n_c1 / block2) * block2 codes (c2_format); c2_scales:
 * ceil(n_c1 / block2) values of c1_dtype. */
int rq_dq_quantize(const void* c1, int c1_dtype, int64_t n_c1, int64_t block2,
                   int c2_format, uint8_t* c2, void* c2_scales, hipStream_t stream);

/* Replaces double_dequantize(state) -- double_quant.py:99-122:
 * c1'[b] = float(c2[b]) * float(c2_scales[b / block2])   (fnuz), or
 *        = (float(c2[b]) / 127) * float(c2_scales[...])  (int8);
 * out[i] = dtype(T[code_i] * c1'[i / block1]) for i < n_out. */
int rq_dq_dequantize(const uint8_t* packed, const uint8_t* c2, int c2_format,
                     const void* c2_scales, int c2s_dtype,
                     int64_t n_packed, int64_t block1, int64_t block2,
                     void* out, int out_dtype, int64_t n_out, hipStream_t stream);

/* ------------------------------------------------------------------------
 * INT8 codec
 * ------------------------------------------------------------------------ */

/* Replaces quantize_int8(tensor, block_size, per_channel) -- quant_ops.py:17-53.
 * block_size > 0: blockwise over the flat rows*cols elements (zero-padded to a
 *   multiple of block_size); q has numel_padded entries, scales numel_padded /
 *   block_size values of w_dtype.
 * block_size == 0: per output row; q is [rows, cols], scales [rows].
 * scale = clamp(absmax / 127, 1e-12) in w_dtype; q = int8(round_half_even(w / scale)). */
int rq_int8_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols,
                     int64_t block_size, int8_t* q, void* scales, hipStream_t stream);

/* Replaces dequantize_int8 -- quant_ops.py:55-78 (+ caller's cast):
 * out[i] = dtype(float(q[i]) * float(scale)), scale per block (block_size > 0)
 * or per row of `cols` elements (block_size == 0). */
int rq_int8_dequantize(const int8_t* q, const void* scales, int scales_dtype,
                       int64_t rows, int64_t cols, int64_t block_size,
                       void* out, int out_dtype, int64_t n_out, hipStream_t stream);

/* ------------------------------------------------------------------------
 * NF4 quantized linear with bias and LoRA
 * ------------------------------------------------------------------------ */

/* Bytes of device workspace rq_nf4_linear needs for these sizes (0 when
 * none).  The caller allocates it (256-byte aligned) and passes it in (the
 * MFMA GEMM, M > 16, also runs with less: then without K splits).  Its
 * first RQ_LINEAR_SYNC_BYTES are a synchronization area (the decode GEMV's
 * LoRA down-projection partials, exchanged between the workgroups of one
 * launch, and the GEMM's K-split tile counters): it must be zero before the
 * workspace's first use, and every call leaves it ready for the next one
 * once its kernels have finished (not necessarily zero: the GEMV keeps the
 * parity of its partial regions there), so a workspace is reused as it is
 * by calls ordered on one stream.  Calls that may overlap need workspaces of
 * their own. */
#define RQ_LINEAR_SYNC_BYTES 131328
int rq_nf4_linear_workspace_size(int x_dtype, int64_t M, int64_t K, int64_t N, int64_t rank,
                                 int64_t* bytes);

/* Replaces QuantLinear.forward for bits=4 (quant_linear.py:121-197, single
 * and double quant branches) fused with LoRALinear.forward
 * (lora_layer.py:51-70), and the reference's native entry point
 * launch_int4_dequant_matmul (hip_kernels/int4_matmul.hip:413-437):
 *   y[M, N] = RND(RND(x W^T + RND(bias)) + RND(RND(RND(xl A^T) RND(B)^T) * scaling))
 * with RND the rounding to x_dtype (bf16 or fp16) and W = T[code] * scale.
 * x_dtype fp32 computes everything in fp32 as the reference's fp32 path does
 * (W = T[code] * scale rounded to fp32, no other roundings); its workspace
 * holds the LoRA operand u after the synchronization area.
 *   x: [M, K] rows of stride ldx; w_packed: the flat N*K codes, two per byte
 *   (element 2j in the low nibble of byte j), as quantize_int4 packs the
 *   flattened weight; block_size any (blocks run over the flat weight and may
 *   straddle rows); absmax: ceil(N*K/block_size) scales of absmax_dtype, or --
 *   when c2 != NULL -- the c2_scales of the double quantization (one per
 *   block2 codes in c2, format c2_format).  Any K, block size and operand
 *   alignment (elements aligned to their size) is taken: calls outside the
 *   specialized kernels' shapes (K % 64 != 0, a block size that is not a
 *   power of two >= 64 dividing K, operands they cannot read 16 bytes at a
 *   time, fp32 activations with rank > 64) run on generic kernels with the
 *   same roundings.
 *   bias: [N] or NULL.  LoRA (rank > 0, lora_a and lora_b non-NULL): xl
 *   (lora_x, or x when NULL) [M, K] stride ld_lora_x, A [rank, K], B [N, rank]
 *   stride ld_lora_b, both of lora_dtype.  y: [M, N] stride ldy, x_dtype.
 * M <= 16 runs the decode GEMV; larger M the MFMA GEMM. */
int rq_nf4_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                  const uint8_t* w_packed, int64_t N, int64_t block_size,
                  const void* absmax, int absmax_dtype,
                  const uint8_t* c2, int c2_format, int64_t block2,
                  const void* bias, int bias_dtype,
                  const void* lora_x, int64_t ld_lora_x, const void* lora_a, const void* lora_b,
                  int64_t ld_lora_b, int lora_dtype, int64_t rank, float scaling,
                  void* y, int64_t ldy, void* workspace, int64_t workspace_bytes,
                  hipStream_t stream);

/* Bytes of the device scratch array behind rq_nf4_linear_noalloc (per GPU,
 * held until the process ends). */
#define RQ_NOALLOC_SCRATCH_BYTES (32u << 20)

/* rq_nf4_linear without a workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * workspace is a static device array of RQ_NOALLOC_SCRATCH_BYTES per GPU,
 * shared by every call on that GPU.  Allocates nothing and calls no
 * allocating routine.  The MFMA GEMM (M > 16) runs without K splits when
 * their partial tiles do not fit; a call that still needs more than the array
 * returns RQ_ERR_SCRATCH_LIMIT before launching anything.
 * The first call on a device also launches a fill kernel that clears the
 * array's synchronization area; every call leaves it clear.  Calls that may
 * overlap on one GPU (other streams, other threads) race on the array: order
 * them on one stream, or use rq_nf4_linear with workspaces of their own. */
int rq_nf4_linear_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                          const uint8_t* w_packed, int64_t N, int64_t block_size,
                          const void* absmax, int absmax_dtype,
                          const uint8_t* c2, int c2_format, int64_t block2,
                          const void* bias, int bias_dtype,
                          const void* lora_x, int64_t ld_lora_x, const void* lora_a, const void* lora_b,
                          int64_t ld_lora_b, int lora_dtype, int64_t rank, float scaling,
                          void* y, int64_t ldy, hipStream_t stream);

/* Test hook, no counterpart in the reference: how long (microseconds, timed
 * on the device's constant-rate real-time counter) a decode-GEMV workgroup
 * polls for the workgroups that compute the LoRA down-projection inside the
 * same launch before it computes the down-projection itself (the same sums
 * in the same order).  0 forces that path; the default is 40.  Returns the
 * previous value. */
uint32_t rq_set_gemv_wait_us(uint32_t us);

/* Tile configuration of the MFMA GEMM behind rq_nf4_linear (M > 16),
 * rq_nf4_linear_dx and rq_int8_linear: out[0..4] = rows and
 * columns of a workgroup tile, k per step, wavefronts per workgroup, LDS
 * pipeline stages.  Replaces the tile table of get_kernel_config
 * (kernels/kernel_config.py:18-48), which describes the reference's Triton
 * tiles. */
int rq_gemm_tile_config(int32_t* out);

/* Bytes of device workspace rq_nf4_linear_dx needs (0 when none; dy_dtype
 * fp32, bf16 or fp16). */
int rq_nf4_linear_dx_workspace_size(int dy_dtype, int64_t M, int64_t N, int64_t K, int64_t rank,
                                    int64_t* bytes);

/* Replaces the backward of _FusedNF4MatmulFunc (kernels/dequant_matmul.py:
 * 338-351: dX = dY . W_deq in dY's dtype) together with the adapter's input
 * gradient of LoRALinear.forward (lora_layer.py:67 differentiated):
 *   dX[M, K] = RND(RND(dY W) + RND(RND(RND(RND(dY * scaling) RND(B)) RND(A)) * d))
 * with RND the rounding to dy_dtype (bf16 or fp16; fp32: none), W = T[code] * scale, and
 * d = 1, or -- with the adapter's input dropout (lora_layer.py:67's
 * self.lora_dropout(x)) -- dropout's backward d = lora_mask[m, k] ? mask_scale
 * : 0 (mask_scale = 1 / (1 - p)).
 *   dy: [M, N] rows of stride lddy; w_packed, block_size, absmax, c2,
 *   c2_format, block2 as for rq_nf4_linear (any K and block size: shapes
 *   outside the MFMA kernel's -- N or K not multiples of 64, other block
 *   sizes, fp32 dy, dy rows not 16-byte aligned -- run on generic kernels);
 *   LoRA (rank > 0, lora_a and lora_b non-NULL): A [rank, K], B [N, rank]
 *   stride ld_lora_b, both of lora_dtype; lora_mask: NULL or [M, K] bytes
 *   (non-zero = kept) of row stride ld_lora_mask.  dx: [M, K] stride lddx,
 *   dy_dtype. */
int rq_nf4_linear_dx(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t lddy,
                     const uint8_t* w_packed, int64_t K, int64_t block_size,
                     const void* absmax, int absmax_dtype,
                     const uint8_t* c2, int c2_format, int64_t block2,
                     const void* lora_a, const void* lora_b, int64_t ld_lora_b, int lora_dtype,
                     int64_t rank, float scaling, const uint8_t* lora_mask, int64_t ld_lora_mask,
                     float mask_scale, void* dx, int64_t lddx,
                     void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * INT8 and FP8 linears
 * ------------------------------------------------------------------------ */

/* Replaces QuantLinear.forward for bits=8 (quant_linear.py:189-197 with
 * dequantize_int8, quant_ops.py:55-78) and the reference's native entry point
 * launch_int8_dequant_matmul (hip_kernels/int4_matmul.hip:440-458):
 *   y[M, N] = RND(x W^T + RND(bias)),  W = RND(float(q) * scale)
 *   with RND the rounding to x_dtype (fp32: none).
 *   x: [M, K] fp32/bf16/fp16 rows of stride ldx; q: [N, K] int8;
 *   block_size 0: one scale per output row (scales [N]); otherwise blockwise
 *   over the flat weight (scales [ceil(N*K/block)]); scales of scales_dtype;
 *   bias [N] or NULL; y: [M, N] stride ldy.
 * 16-bit x with K % 64 == 0, a power-of-two block >= 64 dividing K (or per
 * row) and 16-byte aligned rows runs a weight-streaming GEMV (M <= 16) or the
 * MFMA GEMM; every other call runs on generic kernels with the same
 * roundings. */
int rq_int8_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                   const int8_t* q, int64_t N, int64_t block_size,
                   const void* scales, int scales_dtype, const void* bias, int bias_dtype,
                   void* y, int64_t ldy, hipStream_t stream);

/* Replaces the backward of _FusedInt8MatmulFunc (kernels/dequant_matmul.py:
 * 308-324: dX = dY . W_deq in dY's dtype):
 *   dX[M, K] = RND(dY RND(W)),  W = float(q) * scale
 * with RND the rounding to dy_dtype (fp32: none); dy: [M, N] fp32/bf16/fp16
 * rows of stride lddy; q, block_size, scales, scales_dtype as for
 * rq_int8_linear; dx: [M, K] stride lddx.  Runs on the generic kernels (the
 * int8 codes decoded inside the multiply, MFMA for 16-bit dY). */
int rq_int8_linear_dx(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t lddy, const int8_t* q,
                      int64_t K, int64_t block_size, const void* scales, int scales_dtype, void* dx,
                      int64_t lddx, hipStream_t stream);

/* Bytes of workspace rq_fp8_quantize needs. */
int rq_fp8_quantize_workspace_size(int64_t* bytes);

/* Replaces the per-tensor FP8 quantization of _FP8LinearFunc.forward
 * (fp8/fp8_linear.py:33-42): *scale = fp32(double(max|t|) / 240) (device
 * fp32), codes[r, c] = e4m3fnuz(RND_dtype(float(t[r, c]) / *scale)).
 * t: [rows, cols] of t_dtype (fp32/bf16/fp16), row stride ld; codes dense. */
int rq_fp8_quantize(const void* t, int t_dtype, int64_t rows, int64_t cols, int64_t ld,
                    uint8_t* codes, float* scale, void* workspace, int64_t workspace_bytes,
                    hipStream_t stream);

/* e4m3fnuz codes (the reference's torch.float8_e4m3fnuz, as rq_fp8_quantize
 * writes them) -> e4m3fn codes of the same values, the OCP format gfx950's
 * fp8 matrix cores read (torch.float8_e4m3fn; in place when out == codes).
 * Exact except the 8 odd-mantissa magnitudes below 2^-6, which round to
 * the nearest even e4m3fn code (a change of at most 2^-10), as torch's own
 * .to(torch.float8_e4m3fn) does; 0x80 (NaN) becomes 0x7F (NaN).  No
 * counterpart in the reference, which multiplies decoded fnuz values
 * (fp8/fp8_linear.py:44-52); a weight is converted once, when it is
 * quantized.  codes, out: 16-byte aligned. */
int rq_fp8_fnuz_to_e4m3fn(const uint8_t* codes, int64_t n, uint8_t* out, hipStream_t stream);

/* Bytes of workspace rq_fp8_linear needs for M rows of K activations. */
int rq_fp8_linear_workspace_size(int64_t M, int64_t K, int64_t* bytes);

/* Replaces _FP8LinearFunc.forward (fp8/fp8_linear.py:27-60) for a weight
 * already quantized (rq_fp8_quantize, then rq_fp8_fnuz_to_e4m3fn): x is
 * quantized per tensor the same way (scale = fp32(double(max|x|) / 240),
 * codes = e4m3fnuz(RND(x / scale)) re-encoded to e4m3fn), then
 *   y = RND(RND(sum_k x8 w8 * x_scale * w_scale) + RND(bias))
 * with the fp8 products summed by the fp8 matrix cores in fp32.
 *   x: [M, K] fp32/bf16/fp16 stride ldx; w_codes: [N, K] e4m3fn;
 *   w_scale: device fp32; bias [N] or NULL; y: [M, N] stride ldy.
 * 16-bit x with K % 64 == 0 and 16-byte aligned rows runs a weight-streaming
 * GEMV (M <= 16) or the fp8 MFMA GEMM.  Every other call (fp32 x among them)
 * quantizes x to e4m3fnuz codes the same way and runs on generic kernels as
 * the reference computes it: y = RND(RND(sum_k (x8 x_scale)(w8 w_scale)) +
 * RND(bias)), each code decoded and multiplied by its scale in fp32 (the
 * e4m3fn weight codes hold the reference's values but for the 8 re-encoded
 * magnitudes below 2^-6 noted at rq_fp8_fnuz_to_e4m3fn). */
int rq_fp8_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                  const uint8_t* w_codes, int64_t N, const float* w_scale,
                  const void* bias, int bias_dtype, void* y, int64_t ldy,
                  void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * W8A8 INT8 mode (int8 activations x int8 weights on the int8 matrix cores)
 *
 * No counterpart in the reference, whose INT8 linear multiplies dequantized
 * weights with 16-bit activations (rq_int8_linear above).  This mode
 * quantizes the activations too, per row, with quantize_int8's per-row recipe
 * (quantization/quant_ops.py:29-35) computed in fp32, and sums the int8
 * products exactly in int32; its outputs differ from rq_int8_linear's by the
 * activation rounding, so it is a separate mode, not a replacement.
 * ------------------------------------------------------------------------ */

/* Per-row int8 quantization of 16-bit activations:
 *   scales[m] = max(fp32(max_k |x[m, k]|) / 127, 1e-12)  (device fp32)
 *   codes[m, k] = RNE(fp32(x[m, k]) / scales[m])  in [-127, 127]
 * x: [M, K] bf16/fp16 stride ldx (K % 8 == 0, 16-byte aligned rows);
 * codes: [M, K] dense, 8-byte aligned.  A row holding NaN gets a NaN scale
 * and zero codes. */
int rq_int8_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                          int8_t* codes, float* scales, hipStream_t stream);

/* Bytes of workspace rq_int8_linear_w8a8 needs for M rows of K activations. */
int rq_int8_linear_w8a8_workspace_size(int64_t M, int64_t K, int64_t* bytes);

/* y = RND(RND(float(sum_k xq[m, k] wq[n, k]) * xs[m] * ws[n]) + RND(bias[n]))
 * with (xq, xs) = rq_int8_quantize_rows(x) and wq, ws the weight's per-row
 * codes and scales (quantize_int8(w, per_channel=True),
 * quant_ops.py:29-35); the int32 sum is exact, its conversion to fp32
 * rounds to nearest even, and the two scale products round in that order.
 *   x: [M, K] bf16/fp16 stride ldx (K % 64 == 0); w: [N, K] int8 dense;
 *   w_scales: [N] fp32/bf16/fp16; bias [N] or NULL; y: [M, N] stride ldy.
 * M <= 16 runs the weight-streaming GEMV, larger M the int8 MFMA GEMM. */
int rq_int8_linear_w8a8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                        const int8_t* w, int64_t N, const void* w_scales, int w_scales_dtype,
                        const void* bias, int bias_dtype, void* y, int64_t ldy,
                        void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Merged LoRA weights
 * ------------------------------------------------------------------------ */

/* Replaces the dequantize-then-add of LoRALinear.merge_lora
 * (lora/lora_layer.py:72-106) and of the export path's _export_dequant_layer
 * (export/gguf_export.py:30-79): a 16-bit [N, K] weight
 *   mode RQ_MERGE_SUM_THEN_ROUND: out = RND_o(W + d)
 *   mode RQ_MERGE_ROUND_THEN_SUM: out = RND_o(RND_o(W) + RND_o(d))
 * with W the fp32 dequantized base weight (NF4: T[code] * scale, the scale
 * c2 * c2_scale when c2 is non-NULL; INT8: float(q) * scale) and d =
 * RND_L(RND_L(B A) * scaling) the LoRA delta in the adapters' dtype L (the
 * sum over the rank an fp32 fma chain in ascending rank order), RND_o the
 * rounding to out_dtype (bf16 or fp16).
 *   w: flat codes (RQ_WEIGHT_NF4: packed, byte e / 2 holds element e's code
 *   in its low (even e) or high nibble; RQ_WEIGHT_INT8: int8), element
 *   n * K + k; block_size: a power of two (INT8: 0 = one scale per row);
 *   scales: [N*K / block_size] (per row: [N]) of scales_dtype, or with c2
 *   the c2_scales [ceil(blocks / block2)]; c2: [blocks] codes or NULL;
 *   lora_a [rank, K], lora_b [N, rank] of row stride ld_lora_b, both of
 *   lora_dtype (rank 0: no delta); out [N, K] of row stride ld_out. */
int rq_merge_lora(const void* w, int w_format, int64_t N, int64_t K, int64_t block_size,
                  const void* scales, int scales_dtype, const uint8_t* c2, int c2_format, int64_t block2,
                  const void* lora_a, const void* lora_b, int64_t ld_lora_b, int lora_dtype, int64_t rank,
                  float scaling, int mode, void* out, int out_dtype, int64_t ld_out, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Optimizer step for the LoRA parameters
 * ------------------------------------------------------------------------ */

/* Elements per chunk: tensors' state offsets are multiples of it, and one
 * workgroup updates one chunk. */
#define RQ_ADAMW_CHUNK 2048

/* One tensor of a fused AdamW step (72 bytes).  The fp32 scalars are the
 * reference's Python doubles rounded to fp32 (as torch passes them to its
 * GPU kernels), for this tensor's step count t:
 *   decay = 1 - lr * weight_decay (applied when apply_decay, i.e. wd != 0),
 *   beta1, one_minus_beta1 = 1 - beta1, beta2, one_minus_beta2 = 1 - beta2,
 *   inv_bias_correction2_sqrt = 1 / (1 - beta2 ** t) ** 0.5 (the reciprocal
 *   taken in double: torch's GPU division by a host scalar multiplies by it),
 *   eps, neg_step_size = -(lr / (1 - beta1 ** t)). */
typedef struct rq_adamw_tensor {
  void* param;            /* [numel] of dtype, updated in place */
  const void* grad;       /* [numel] of dtype */
  int64_t numel;
  int64_t state_offset;   /* first element in the state buffers; multiple of RQ_ADAMW_CHUNK */
  int32_t dtype;          /* RQ_DTYPE_F32 / BF16 / F16, parameter and gradient */
  int32_t apply_decay;
  float decay, beta1, one_minus_beta1, beta2, one_minus_beta2, inv_bias_correction2_sqrt, eps, neg_step_size;
} rq_adamw_tensor;

/* Replaces the per-parameter update of PagedAdamW.step
 * (optim/paged_adamw.py:84-113): AdamW with decoupled weight decay on every
 * listed tensor in one launch, with the roundings of the reference's ops as
 * torch runs them on the GPU (the reference moves the states to the
 * parameter's device for the update) --
 *   p = RND_p(RND(p * decay)); m = fma(1 - b1, g, RND(m * b1));
 *   v = fma(1 - b2, RND(g * g), RND(v * b2));
 *   d = RND(RND(sqrt(v)) * inv_bias_correction2_sqrt) + eps;
 *   p = RND_p(fma(neg_step_size, RND(m / d), p))
 * (fp32 arithmetic, the square root and division correctly rounded, RND_p
 * the rounding to the parameter's dtype).  The exp_avg (m) and exp_avg_sq (v) states are fp32 buffers
 * indexed by state offset: this call updates the chunks chunk_begin ..
 * chunk_end - 1, and exp_avg / exp_avg_sq (16-byte aligned) point at the
 * element chunk_begin * RQ_ADAMW_CHUNK and hold (chunk_end - chunk_begin) *
 * RQ_ADAMW_CHUNK elements (so a caller can stream the states through a
 * device page).  tensors: host array of n_tensors descriptors in ascending,
 * non-overlapping state order (each spans numel rounded up to a chunk),
 * copied to device_table (>= n_tensors * 72 bytes) on the stream before the
 * launch; tensors without a gradient are left out of the array. */
int rq_adamw_step(const rq_adamw_tensor* tensors, int64_t n_tensors, void* device_table,
                  int64_t device_table_bytes, int64_t chunk_begin, int64_t chunk_end,
                  float* exp_avg, float* exp_avg_sq, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ROCM_QLORA_AMD_H */
