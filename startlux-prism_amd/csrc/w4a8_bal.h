// Host side of the balanced-grid Q4_K decode kernel (w4a8_q4k_bal.hip), called by prism_w4a8_q4k_gemm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

// M in 1..16 and the activation image (M rows of K bytes, the split sums and scales) within LDS.
bool q4k_bal_fits(int64_t M, int64_t N, int64_t K);
// One 64-bit handoff word per (workgroup, output of a 16 x 16 tile).
int64_t q4k_bal_workspace_bytes(int64_t N);
// hand: a zero-initialised workspace of at least q4k_bal_workspace_bytes(N) (left zeroed by every launch).
int q4k_bal_launch(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs, const uint8_t* qv,
                   const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int64_t M, int64_t N,
                   int64_t K, int epi, void* hand, int64_t hand_bytes, hipStream_t st);

}  // namespace prism
