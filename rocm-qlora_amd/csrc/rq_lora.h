// Host interface of the LoRA operand kernels (rq_lora.hip).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "rq_common.h"

namespace rq {

struct LoraRowsPlan {
  int splits;           // K splits of lora_rows_kernel
  int jb;               // 16-rank blocks per workgroup (1, 2 or 4)
  int waves;            // waves of 16 activation rows per workgroup (4 or 8)
  int64_t k_per_split;  // multiple of 64
  size_t part_bytes;    // fp32 partials [splits][M][R], 256-byte padded
};

LoraRowsPlan plan_lora_rows(int64_t M, int64_t K, int64_t R, int cus);

// out[M][R16] = RND(sum_k RND(X[m,k] (* scale if prescale)) . RND(S[j,k]))
// with S[j,k] at s[j * s_j + k * s_k], s_k == 1 or s_j == 1; part is the
// plan's scratch (part_bytes).  K must be a multiple of 64.
int run_lora_rows(int xt, const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const void* s, int s_dt,
                  int64_t s_j, int64_t s_k, int R, bool prescale, float scale, const LoraRowsPlan& p, float* part,
                  uint16_t* out, int R16, hipStream_t stream);

}  // namespace rq
