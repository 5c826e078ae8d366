// Score keys shared by the MoD top-k kernels.
#pragma once
#include <cstdint>

namespace hydra {

// Order-preserving map of a float to u32 (ascending), with -0.0 folded into
// +0.0 and every NaN mapped above +inf (torch.topk treats NaN as largest).
__device__ __forceinline__ uint32_t score_key_asc(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN
  if (u == 0x80000000u) u = 0u;                               // -0.0 -> +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP: row shifts
// within each 16-lane row, then the broadcasts of lane 15 to rows 1 and 3 and
// of lane 31 to rows 2 and 3.
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

// Rows longer than the bucket kernel takes: composites radix-sorted in
// global memory (mod_topk_large.hip).
int mod_topk_large(const void* scores, int64_t B, int64_t L, int64_t s_rs, int64_t k,
                   int64_t* idx_desc, int64_t* idx_sorted, void* mask, int score_dtype,
                   int mask_dtype, hipStream_t st);

}  // namespace hydra
