// Host/device interfaces shared by the NF4 linear kernels (GEMV, GEMM, dX).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "rq_common.h"

namespace rq {

// Largest activation row count served by the decode GEMV; larger M goes to
// the MFMA GEMM.
constexpr int64_t kGemvMaxM = 16;

// rq_nf4_linear's workspace starts with RQ_LINEAR_SYNC_BYTES of
// synchronization area, zero before its first use:
//   [0, 256)               the decode GEMV's in-launch down-projection: its
//                          job count (word 0, zero between launches)
//                          and state (words 32-34: the parity of its next
//                          partial region, the extents of regions 0 and 1)
//   [256, 256 + 64 KiB)    its two partial regions of kGemvPartBytes; the
//                          one the parity names is zero between launches
//   [.., + 64 KiB)         the GEMM's and the decode GEMV's K-split
//                          counters, zero between launches
// Every call leaves the area in that state once its kernels are done; the
// GEMM's workspace and the split-K partials start after the area.
constexpr size_t kLinearSyncBytes = RQ_LINEAR_SYNC_BYTES;
constexpr size_t kLinearCountBytes = 256;
constexpr size_t kLinearParityWord = 32;
constexpr size_t kGemvPartBytes = 32768;
constexpr size_t kGemvPartWords = kGemvPartBytes / 4;
constexpr size_t kGemmCountBytes = 65536;
static_assert(kLinearSyncBytes == kLinearCountBytes + 2 * kGemvPartBytes + kGemmCountBytes,
              "synchronization area layout");

// Unpacked arguments of rq_nf4_linear (see include/rocm_qlora_amd.h).
struct LinearArgs {
  const void* x;
  int x_dtype;
  int64_t M, K, ldx;
  const uint8_t* w_packed;
  int64_t N, block_size;
  const void* absmax;  // absmax, or c2_scales when c2 != nullptr
  int absmax_dtype;
  const uint8_t* c2;
  int c2_format;
  int64_t block2;
  const void* bias;
  int bias_dtype;
  const void* lora_x;
  int64_t ld_lora_x;
  const void* lora_a;
  const void* lora_b;
  int64_t ld_lora_b;
  int lora_dtype;
  int64_t rank;
  float scaling;
  void* y;
  int64_t ldy;
};

// Epilogue inputs as the kernels see them.
struct LinearEpi {
  const void* bias;
  int bias_dt;
  int rank;
  const float* u;  // [u_splits, M, rank] fp32 partials of x . A^T
  int u_splits;
  const void* lora_b;
  int64_t ld_lora_b;
  int lora_dt;
  float scaling;
  void* y;
  int64_t ldy;
};

struct GemvPlan {
  int S, TS, U, nseg, grid, u_splits;
  int jobs;  // LoRA down-projection wave jobs inside the launch (0: none)
  bool direct, xslice;
  bool fold;  // K splits finished by the last split of each column (no finisher launch)
  size_t lds_bytes, ws_bytes, u_offset;
};

GemvPlan plan_gemv(int64_t M, int64_t N, int64_t K, int64_t rank, int cus, bool xvec, bool gather,
                   bool lora_vec, bool lora_prod);
// Microseconds the GEMV waits for its LoRA producers before a workgroup
// computes the down-projection itself (a test hook: 0 forces that path).
// Returns the previous value.
uint32_t set_gemv_wait_us(uint32_t us);
int validate_linear(const LinearArgs& L);
bool linear_fast_ok(const LinearArgs& L);
LinearEpi make_epi(const LinearArgs& L, float* u_parts, int u_splits);
int run_lora_u(const LinearArgs& L, int ks, float* up, hipStream_t stream);
int gemv_workspace(const LinearArgs& L, size_t* bytes);
int run_nf4_gemv(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream);
int gemm_workspace(const LinearArgs& L, size_t* bytes);
// the GEMM's workspace without K splits (the smallest it runs with)
size_t gemm_min_workspace(const LinearArgs& L);
// fp32 activations (any M): the fp32-MFMA GEMV over 16-row blocks
int f32_linear_workspace(const LinearArgs& L, size_t* bytes);
int run_nf4_linear_f32(const LinearArgs& L, void* workspace, size_t ws_bytes, hipStream_t stream);
// tile_cnt: n_cnt zeroed counters the GEMM's K splits use (and leave zero);
// without them the GEMM runs unsplit.
int run_nf4_gemm(const LinearArgs& L, void* workspace, size_t ws_bytes, uint32_t* tile_cnt, size_t n_cnt,
                 hipStream_t stream);

// Unpacked arguments of rq_nf4_linear_dx (see include/rocm_qlora_amd.h).
struct DxArgs {
  const void* dy;
  int dy_dtype;
  int64_t M, N, lddy;
  const uint8_t* w_packed;
  int64_t K, block_size;
  const void* absmax;  // absmax, or c2_scales when c2 != nullptr
  int absmax_dtype;
  const uint8_t* c2;
  int c2_format;
  int64_t block2;
  const void* lora_a;
  const void* lora_b;
  int64_t ld_lora_b;
  int lora_dtype;
  int64_t rank;
  float scaling;
  const uint8_t* lora_mask;  // dropout mask [M][K] (row stride ld_lora_mask), or nullptr
  int64_t ld_lora_mask;
  float mask_scale;
  void* dx;
  int64_t lddx;
};

int validate_dx(const DxArgs& D);
int dx_workspace(const DxArgs& D, size_t* bytes);
int run_nf4_dx(const DxArgs& D, void* workspace, size_t ws_bytes, hipStream_t stream);

}  // namespace rq
