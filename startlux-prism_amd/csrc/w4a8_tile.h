// Host side of the Q4_K prefill tile kernel (w4a8_q4k_tile.hip), called by prism_w4a8_q4k_gemm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

// Any M (grid rows over 64 activation rows), N % 16 == 0, K % 256 == 0; operands as prism_w4a8_q4k_gemm's.
void q4k_tile_launch(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs, const uint8_t* qv,
                     const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int epi,
                     hipStream_t st);

}  // namespace prism
