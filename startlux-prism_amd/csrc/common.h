// Shared device helpers for the gfx950 kernels: float-format conversions with explicit rounding, wave
// reductions, MFMA operand types and the launch-status plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/prism_amd.h"

namespace prism {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN kept quiet (the same rule as torch's .to(torch.bfloat16)).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;
}

// IEEE (correctly rounded) fp32 division; the library is built with -fhip-fp32-correctly-rounded-divide-sqrt,
// so '/' is the IEEE operation, written through one helper so every kernel rounds alike.
__device__ __forceinline__ float div_rn(float a, float b) { return __fdiv_rn(a, b); }

// Correctly rounded fp32 square root.  sqrtf under -fhip-fp32-correctly-rounded-divide-sqrt expands to the refined
// sequence; __fsqrt_rn on this toolchain is the bare v_sqrt_f32 (about 1 ulp), so it is not used.
__device__ __forceinline__ float sqrt_rn(float a) { return sqrtf(a); }

// Explicitly rounded fp32 multiply / add: the compiler never contracts these into an fma.
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }

// rint(RN(y / s)) for a quantizer: s = RN(max(amax, 1e-10) / 127) of a group holding y (so |y / s| <= 127.0001), and
// r = RN(1 / s) computed once per scale.  q0 = RN(y r) is within |y / s| (3u + u^2) <= 2^-15.4 of RN(y / s) (u = 2^-24:
// r, the product and the quotient each round once; an underflowing product only moves values far below 1/2), so
// rint(q0) is rint(RN(y / s)) unless q0 lies within 2^-15 of a half-integer, where the two could fall on different
// sides or RN(y / s) could be a tie: those few, and non-finite q0, take the exact division.  Bits equal the division's.
__device__ __forceinline__ float quant_rint(float y, float s, float r) {
    const float q0 = __fmul_rn(y, r);
    const float fr = fabsf(q0 - truncf(q0));                 // exact below 2^23
    if (__builtin_expect(fabsf(fr - 0.5f) > 0x1p-15f, 1)) return rintf(q0);
    return rintf(__fdiv_rn(y, s));
}

// RN(x * float(h)) for the fp16 half H (0 low, 1 high) of word, in one v_fma_mix_f32 (fp16 operand widened exactly,
// one rounding; the -0.0 addend leaves every product, signed zeros included, as the plain product).
template <int H>
__device__ __forceinline__ float mul_f16_rn(float x, uint32_t word) {
    float r;
    const float nz = -0.0f;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,%4,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(x), "v"(word), "v"(nz), "n"(H));
    return r;
}

// Every listed kernel argument in scalar registers at this point, with one wait: the compiler otherwise loads each
// argument where it is first used, one scalar memory round trip after another, and a decode-size kernel's first
// weight request then waits behind several of them.  Up to 16 arguments (all wave-uniform values).
#define PRISM_S_(x) "s"(x)
#define PRISM_MAP1(f, x) f(x)
#define PRISM_MAP2(f, x, ...) f(x), PRISM_MAP1(f, __VA_ARGS__)
#define PRISM_MAP3(f, x, ...) f(x), PRISM_MAP2(f, __VA_ARGS__)
#define PRISM_MAP4(f, x, ...) f(x), PRISM_MAP3(f, __VA_ARGS__)
#define PRISM_MAP5(f, x, ...) f(x), PRISM_MAP4(f, __VA_ARGS__)
#define PRISM_MAP6(f, x, ...) f(x), PRISM_MAP5(f, __VA_ARGS__)
#define PRISM_MAP7(f, x, ...) f(x), PRISM_MAP6(f, __VA_ARGS__)
#define PRISM_MAP8(f, x, ...) f(x), PRISM_MAP7(f, __VA_ARGS__)
#define PRISM_MAP9(f, x, ...) f(x), PRISM_MAP8(f, __VA_ARGS__)
#define PRISM_MAP10(f, x, ...) f(x), PRISM_MAP9(f, __VA_ARGS__)
#define PRISM_MAP11(f, x, ...) f(x), PRISM_MAP10(f, __VA_ARGS__)
#define PRISM_MAP12(f, x, ...) f(x), PRISM_MAP11(f, __VA_ARGS__)
#define PRISM_MAP13(f, x, ...) f(x), PRISM_MAP12(f, __VA_ARGS__)
#define PRISM_MAP14(f, x, ...) f(x), PRISM_MAP13(f, __VA_ARGS__)
#define PRISM_MAP15(f, x, ...) f(x), PRISM_MAP14(f, __VA_ARGS__)
#define PRISM_MAP16(f, x, ...) f(x), PRISM_MAP15(f, __VA_ARGS__)
#define PRISM_NARG_(_1, _2, _3, _4, _5, _6, _7, _8, _9, _10, _11, _12, _13, _14, _15, _16, N, ...) N
#define PRISM_NARG(...) PRISM_NARG_(__VA_ARGS__, 16, 15, 14, 13, 12, 11, 10, 9, 8, 7, 6, 5, 4, 3, 2, 1)
#define PRISM_CAT_(a, b) a##b
#define PRISM_CAT(a, b) PRISM_CAT_(a, b)
#define kernel_args_now(...) \
    asm volatile("" ::PRISM_CAT(PRISM_MAP, PRISM_NARG(__VA_ARGS__))(PRISM_S_, __VA_ARGS__))

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS operations, not for its outstanding global
// loads (__syncthreads() also drains those, which would empty a kernel's prefetch pipeline at every barrier).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// LDS-DMA: each lane's 16 (or 1) bytes from its own global address to the wave's LDS base + lane x 16 (x 4: the
// one-byte form fills a dword per lane).  `lds` must be the same for every lane of the wave.
__device__ __forceinline__ void dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void dma1(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 1, 0, 0);
}

// Buffer loads: a wave-uniform base in a buffer resource (SGPRs), the uniform part of the offset in soffset (an
// SGPR) and the lane's fixed part in one VGPR, so a streaming loop computes no per-load addresses in VGPRs.  Streamed
// that way the compiler has no address temporaries to place in registers still awaiting an earlier load (which makes
// it wait for the previous requests before issuing the next ones).  Raw buffer (stride 0): the range check compares
// voffset + soffset with the record count, here the largest, so it never clips a valid offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}
// The same with the record count set to `bytes` from the base: a load past it returns zeros instead of reading beyond
// the caller's buffer (the check is per dword).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc_n(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
constexpr int kBufNT = 2;                 // the cache-policy bit of a non-temporal (streaming) load
template <int AUX = 0>
__device__ __forceinline__ v4i buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, AUX));
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ uint32_t buf_load1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ v2u buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(v2u, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0));
}

// Waits until at most N vector-memory operations of this wave are outstanding.  The compiler does not count LDS-DMA
// writes as producers of later LDS reads, so every DMA stage is closed by an explicit wait (then a barrier).
template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The same wait through the compiler's builtin, which the compiler's own wait insertion takes into account: after
// it, loads older than the last N count as complete (an LDS-DMA among them then needs no further wait before the
// LDS reads that follow).  gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their
// maxima.
template <int N>
__device__ __forceinline__ void vm_wait_tracked() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Dynamic LDS above the default 64 KB needs the kernel's limit raised (up to the CU's 160 KB) before its launch.
template <typename F>
inline void allow_lds(F* fn, size_t bytes) {
    if (bytes > 64 * 1024)
        (void)hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

__device__ __forceinline__ int wave_sum_width(int v, int width) {
    for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Tile order for a grid of tiles_m x tiles_n output tiles: the hardware hands workgroup i to XCD i % 8, so logical
// tile t = (i % 8) * (tiles / 8) + i / 8 gives each XCD a contiguous range of tiles, walked in groups of 8 tile-rows
// (m fastest); the workgroups that run together on one XCD then share 8 m-tiles and 8 n-tiles through its L2.
__device__ __forceinline__ void xcd_tile_coords(int pid, int tiles_m, int tiles_n, int& pm, int& pn) {
    const int total = tiles_m * tiles_n;
    int t = pid;
    if ((total & 7) == 0) t = (pid & 7) * (total >> 3) + (pid >> 3);
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    const int first_m = (t / per_group) * GM;
    const int gm = min(tiles_m - first_m, GM);
    const int r = t % per_group;
    pm = first_m + r % gm;
    pn = r / gm;
}

}  // namespace prism

// Launch-status helper for the C ABI: a rejected launch becomes PRISM_ERR_LAUNCH.
#define PRISM_LAUNCH_CHECK()                                                        \
    do {                                                                            \
        hipError_t _e = hipGetLastError();                                          \
        if (_e != hipSuccess) return PRISM_ERR_LAUNCH;                             \
    } while (0)

#define PRISM_ALIGNED(p, n) ((((uintptr_t)(p)) & ((n) - 1)) == 0)
