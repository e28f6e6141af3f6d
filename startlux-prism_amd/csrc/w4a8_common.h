// Q4_K / Q6_K helpers shared by the W4A8 kernels (w4a8.hip, w4a8_q4k_bal.hip): the two-plane weight operand, the
// mins on the MFMA, one row's meta and the super-block term.  Arithmetic and layouts as w4a8.hip's header states.
#pragma once

#include "common.h"

namespace prism {

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

// A lane's 8 bytes of a sub-block pair (w0, w1) times its sub-block scale sc = 8 hi + lo (3-bit parts, given packed
// as split_scale(sc) = lo | hi << 16) as two MFMA weight operands: the 16 nibbles (<= 15) times lo and times hi
// (<= 105: still int8, no carry between bytes of a packed 16-bit multiply).  acc = (x . lo q) + 8 (x . hi q) exactly.
__device__ __forceinline__ uint32_t split_scale(int sc) { return (uint32_t)(sc & 7) | ((uint32_t)(sc >> 3) << 16); }

__device__ __forceinline__ void two_plane(uint32_t w0, uint32_t w1, uint32_t sp, v4i& lo, v4i& hi) {
    const us2 s = __builtin_bit_cast(us2, sp);
    const us2 sl = __builtin_shufflevector(s, s, 0, 0), sh = __builtin_shufflevector(s, s, 1, 1);
    const uint32_t n[4] = {w0 & 0x0f0f0f0fu, w1 & 0x0f0f0f0fu, (w0 >> 4) & 0x0f0f0f0fu, (w1 >> 4) & 0x0f0f0f0fu};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        lo[e] = (int)__builtin_bit_cast(uint32_t, (us2)(__builtin_bit_cast(us2, n[e]) * sl));
        hi[e] = (int)__builtin_bit_cast(uint32_t, (us2)(__builtin_bit_cast(us2, n[e]) * sh));
    }
}

// mins = sum_g mn[n, g] S[m, g] for a 16 x 16 tile as two MFMAs over k = 0..7 (lanes q > 0 carry zeros): the weight
// rows' 8 mins (bytes) against the 8 low parts S & 63, then against the 8 high parts S >> 6; mins = lo + 64 hi.
__device__ __forceinline__ v4i mins_mfma(int64_t mn8, int64_t slo, int64_t shi) {
    const v4i zero = {0, 0, 0, 0};
    const v4i lo = __builtin_amdgcn_mfma_i32_16x16x32_i8(mn8, slo, zero, 0, 0, 0);
    const v4i hi = __builtin_amdgcn_mfma_i32_16x16x32_i8(mn8, shi, zero, 0, 0, 0);
    v4i r;
#pragma unroll
    for (int e = 0; e < 4; e++) r[e] = lo[e] + 64 * hi[e];
    return r;
}

// Q6_K meta per (16-row tile, super-block): the 16 rows' 16 int8 scales, then their fp16 d.
constexpr int Q6_META = 288;

__device__ __forceinline__ int sbyte(v4u m, int j) { return (int)(int8_t)(m[j >> 2] >> (8 * (j & 3))); }

// One row's 16 meta bytes -> d, dmin (fp32) and the 8 scales and 8 mins (ggml get_scale_min_k4).
__device__ __forceinline__ void row_meta(v4u m, float& d, float& dm, int* sc, int* mn) {
    d = f16_to_f32(m[0] & 0xffffu);
    dm = f16_to_f32(m[0] >> 16);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t s0 = (m[1] >> (8 * j)) & 0xff, s4 = (m[2] >> (8 * j)) & 0xff, s8 = (m[3] >> (8 * j)) & 0xff;
        sc[j] = s0 & 63;
        mn[j] = s4 & 63;
        sc[j + 4] = (s8 & 0xf) | ((s0 >> 6) << 4);
        mn[j + 4] = (s8 >> 4) | ((s4 >> 6) << 4);
    }
}

// The split scales (split_scale) of the four sub-blocks a lane's MFMA operands take, 2 p + h for p = 0..3 (h, the
// lane's 32-input half of each 64-input piece), read straight from the row's GGUF packing (get_scale_min_k4 as in
// row_meta: sub-block j < 4 is bits 8 j .. 8 j + 5 of m[1]; j >= 4 is bits 8 (j - 4) .. + 3 of m[3] with bits
// 8 (j - 4) + 6 .. + 7 of m[1] above them), with no unpacking of the other twelve values and no per-lane select.
__device__ __forceinline__ void q4k_lane_splits(v4u m, int h, uint32_t* sp) {
    const uint32_t s = m[1] >> (8 * h), c = m[3] >> (8 * h);
    sp[0] = (s & 7) | (((s >> 3) & 7) << 16);
    sp[1] = ((s >> 16) & 7) | (((s >> 19) & 7) << 16);
    sp[2] = (c & 7) | ((((c >> 3) & 1) | (((s >> 6) & 3) << 1)) << 16);
    sp[3] = ((c >> 16) & 7) | ((((c >> 19) & 1) | (((s >> 22) & 3) << 1)) << 16);
}

// The row's eight mins as the bytes of the mins MFMA operand (mins_mfma), from the same packing: mins 0..3 are the
// low six bits of m[2]'s bytes, mins 4..7 the high nibbles of m[3]'s bytes with m[2]'s top two bits above them.
__device__ __forceinline__ int64_t q4k_mins8(v4u m) {
    const uint32_t lo = m[2] & 0x3f3f3f3fu;
    const uint32_t hi = ((m[3] >> 4) & 0x0f0f0f0fu) | ((m[2] >> 2) & 0x30303030u);
    return (int64_t)lo | ((int64_t)hi << 32);
}

// t = RN(d float(acc)); t = fma(-dm, float(mins), t)   (kernels/w4a8.py:191)
__device__ __forceinline__ float q4k_term(float d, float dm, int acc, int mins) {
    return fmaf(-dm, (float)mins, mul_rn(d, (float)acc));
}

}  // namespace prism
