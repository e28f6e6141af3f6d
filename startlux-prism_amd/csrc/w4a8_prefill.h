// Host side of the W4A8 prefill tile kernels (w4a8_prefill.hip), called by prism_w4a8_q4k_gemm and prism_w4a8_q6k_gemm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

// Any M (grid rows over 128 activation rows), N % 16 == 0, K % 256 == 0; operands as prism_w4a8_q4k_gemm's; stage
// offsets are 32-bit (the caller checks).
void q4k_tile_launch(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs, const uint8_t* qv,
                     const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int epi,
                     hipStream_t st);

// The Q6_K prefill tile kernel, operands as prism_w4a8_q6k_gemm's; stage offsets are 32-bit (the caller checks).
void q6k_tile_launch(const int8_t* xq, const float* a, int64_t a_sb, const uint8_t* qv, const uint8_t* meta,
                     void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int epi, hipStream_t st);

}  // namespace prism
