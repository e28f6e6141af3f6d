// W4A8 GEMM on Q4_K (placeholder until the kernels land).
#include "common.h"
extern "C" int prism_w4a8_q4k_gemm(const int8_t*, const float*, int64_t, const int8_t*, const uint8_t*, const uint8_t*,
                                   const uint8_t*, const float*, const float*, void*, int64_t, const int32_t*, int64_t,
                                   int64_t, int64_t, int, int, void*) {
    return PRISM_ERR_ARG;
}
