// Activation quantizers for the W8A8 and W4A8 GEMMs (gfx950).
//
// One workgroup (256 threads, four wave64s) per row: each thread owns 16-byte chunks of 8 bf16 inputs, read with
// one 128-bit load each and kept in registers between the max pass and the quantization pass, so a row is read
// from HBM once.  All three kernels are HBM-bound: per input 2 bytes read and 1 byte written (plus the scales).
//
// Reference arithmetic (StartLux-Prism):
//   rows_q8   kernels/quant.py:287-309   scale = max(amax, 1e-10) / 127, q = rint(y / scale), y = x * inv_s
//   quant_rows kernels/w8a8.py:101-112   the same per (row, group of gk inputs)
//   rows_g    kernels/quant.py:314-330, kernels/w4a8.py:144-155 (quantize_ref): per group scale, per-32 sums
// Divisions are IEEE (correctly rounded) and rint rounds ties to even, so the results are bit-exact against the
// CPU oracle.
#include "common.h"

namespace prism {

constexpr int kQThreads = 256;

__device__ __forceinline__ void unpack_bf16x8(v4u w, float* f) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        f[2 * j] = __uint_as_float(w[j] << 16);
        f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
}

__device__ __forceinline__ uint32_t pack_i8x4(const float* f) {
    uint32_t r = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) r |= ((uint32_t)(int)f[j] & 0xffu) << (8 * j);
    return r;
}

__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kQThreads / kWave; i++) r = fmaxf(r, red[i]);
    return r;
}

// ---------------------------------------------------------------------------------------------- rows_q8
template <int NCH>
__global__ __launch_bounds__(kQThreads) void quant_rows_i8_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                  const float* __restrict__ inv_s,
                                                                  int8_t* __restrict__ q, float* __restrict__ s,
                                                                  const int32_t* __restrict__ n_rows, int K) {
    __shared__ float red[kQThreads / kWave];
    kernel_args_now(x, ldx, inv_s, q, s, n_rows, K);
    const int64_t row = blockIdx.x;
    const int nch = K / 8;
    const v4u* xr = reinterpret_cast<const v4u*>(x + row * ldx);
    float v[NCH][8];
    float amax = 0.f;
    // every chunk's loads first, unconditionally (indices clamped into the row), so they are in flight together;
    // a load inside a per-chunk branch would wait before the next chunk's went out
    v4u raw[NCH];
#pragma unroll
    for (int c = 0; c < NCH; c++) raw[c] = __builtin_nontemporal_load(xr + min((int)threadIdx.x + c * kQThreads, nch - 1));
    v4f isc[NCH][2];
    if (inv_s) {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const v4f* ip = reinterpret_cast<const v4f*>(inv_s + min((int)threadIdx.x + c * kQThreads, nch - 1) * 8);
            isc[c][0] = ip[0];
            isc[c][1] = ip[1];
        }
    }
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * kQThreads;
        unpack_bf16x8(raw[c], v[c]);
        if (inv_s) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[c][j] = mul_rn(v[c][j], isc[c][0][j]);
                v[c][j + 4] = mul_rn(v[c][j + 4], isc[c][1][j]);
            }
        }
        if (idx < nch) {
#pragma unroll
            for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[c][j]));
        }
    }
    amax = block_max(amax, red);
    if (row >= (int64_t)__ldg(n_rows)) return;                 // read after the row's loads went out (see above)
    const float scale = div_rn(fmaxf(amax, 1e-10f), 127.0f), rs = div_rn(1.0f, scale);
    v2u* qr = reinterpret_cast<v2u*>(q + row * K);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * kQThreads;
        if (idx < nch) {
            float r[8];
#pragma unroll
            for (int j = 0; j < 8; j++) r[j] = quant_rint(v[c][j], scale, rs);
            v2u o;
            o[0] = pack_i8x4(r);
            o[1] = pack_i8x4(r + 4);
            qr[idx] = o;
        }
    }
    if (threadIdx.x == 0) s[row] = scale;
}

// ---------------------------------------------------------------------------------------------- quant_rows (gk)
// Groups of gk inputs, gk / 8 a power of two <= 64: one 256-thread block covers 2048 inputs of a row (a whole number
// of groups); a group's max is a reduction over gk / 8 neighbouring lanes.
__global__ __launch_bounds__(kQThreads) void quant_rows_groups_kernel(const uint16_t* __restrict__ x,
                                                                      int8_t* __restrict__ q, float* __restrict__ s,
                                                                      const int32_t* __restrict__ n_rows, int K,
                                                                      int gk) {
    kernel_args_now(x, q, s, n_rows, K, gk);
    const int64_t row = blockIdx.y;
    const int idx = blockIdx.x * kQThreads + threadIdx.x;       // chunk of 8 inputs
    const int nch = K / 8, width = gk / 8;
    const bool live = idx < nch;
    float v[8];
    float amax = 0.f;
    if (live) {
        unpack_bf16x8(reinterpret_cast<const v4u*>(x + row * K)[idx], v);
#pragma unroll
        for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[j]));
    }
    for (int o = width / 2; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, kWave));
    if (!live || row >= (int64_t)__ldg(n_rows)) return;        // read after the row's loads went out
    const float scale = div_rn(fmaxf(amax, 1e-10f), 127.0f), rs = div_rn(1.0f, scale);
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; j++) r[j] = quant_rint(v[j], scale, rs);
    v2u o;
    o[0] = pack_i8x4(r);
    o[1] = pack_i8x4(r + 4);
    reinterpret_cast<v2u*>(q + row * K)[idx] = o;
    if ((idx % width) == 0) s[row * (K / gk) + idx / width] = scale;
}

// Any other gk (a multiple of 32): one block per (row, group), strided over the group.
__global__ __launch_bounds__(kQThreads) void quant_rows_groups_slow_kernel(const uint16_t* __restrict__ x,
                                                                           int8_t* __restrict__ q,
                                                                           float* __restrict__ s,
                                                                           const int32_t* __restrict__ n_rows,
                                                                           int K, int gk) {
    __shared__ float red[kQThreads / kWave];
    const int64_t row = blockIdx.y;
    if (row >= (int64_t)__ldg(n_rows)) return;
    const int g = blockIdx.x;
    const uint16_t* xr = x + row * K + (int64_t)g * gk;
    float amax = 0.f;
    for (int i = threadIdx.x; i < gk; i += kQThreads) amax = fmaxf(amax, fabsf(bf16_to_f32(xr[i])));
    amax = block_max(amax, red);
    const float scale = div_rn(fmaxf(amax, 1e-10f), 127.0f), rs = div_rn(1.0f, scale);
    for (int i = threadIdx.x; i < gk; i += kQThreads)
        q[row * K + (int64_t)g * gk + i] = (int8_t)(int)quant_rint(bf16_to_f32(xr[i]), scale, rs);
    if (threadIdx.x == 0) s[row * (K / gk) + g] = scale;
}

// ---------------------------------------------------------------------------------------------- rows_g (W4A8)
// GROUP_ROW: one scale for the whole row (group == K); otherwise one per 256 inputs (32 chunks = half a wave).
template <int NCH, bool GROUP_ROW>
__global__ __launch_bounds__(kQThreads) void quant_rows_g_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                 int8_t* __restrict__ xq, float* __restrict__ a,
                                                                 int8_t* __restrict__ xs,
                                                                 const int32_t* __restrict__ n_rows, int M, int K) {
    __shared__ float red[kQThreads / kWave];
    kernel_args_now(x, ldx, xq, a, xs, n_rows, M, K);
    const int64_t row = blockIdx.x;
    const int nch = K / 8;
    const v4u* xr = reinterpret_cast<const v4u*>(x + row * ldx);
    float v[NCH][8];
    float amax[NCH];
    float rmax = 0.f;
    v4u raw[NCH];                                      // all loads first (see rows_q8)
#pragma unroll
    for (int c = 0; c < NCH; c++) raw[c] = __builtin_nontemporal_load(xr + min((int)threadIdx.x + c * kQThreads, nch - 1));
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * kQThreads;
        amax[c] = 0.f;
        unpack_bf16x8(raw[c], v[c]);
        if (idx < nch) {
#pragma unroll
            for (int j = 0; j < 8; j++) amax[c] = fmaxf(amax[c], fabsf(v[c][j]));
        }
        rmax = fmaxf(rmax, amax[c]);
    }
    if (GROUP_ROW) rmax = block_max(rmax, red);
    if (row >= (int64_t)__ldg(n_rows)) return;                 // read after the row's loads went out
    v2u* qr = reinterpret_cast<v2u*>(xq + row * K);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * kQThreads;   // all lanes of a half-wave share the validity of idx
        float gmax = rmax;
        if (!GROUP_ROW) {
            gmax = amax[c];
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) gmax = fmaxf(gmax, __shfl_xor(gmax, o, kWave));
        }
        const float scale = div_rn(fmaxf(gmax, 1e-10f), 127.0f), rs = div_rn(1.0f, scale);
        int sum = 0;
        if (idx < nch) {
            float r[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                r[j] = quant_rint(v[c][j], scale, rs);
                sum += (int)r[j];
            }
            v2u o;
            o[0] = pack_i8x4(r);
            o[1] = pack_i8x4(r + 4);
            qr[idx] = o;
        }
        sum = wave_sum_width(sum, 4);                  // the 4 chunks of a sub-block of 32 are neighbouring lanes
        if (idx < nch) {
            const int b = idx / 32, j = (idx % 32) / 4;
            if ((idx % 4) == 0) {
                int8_t* p = xs + ((int64_t)b * M + row) * 16;
                p[j] = (int8_t)(sum & 63);
                p[8 + j] = (int8_t)(sum >> 6);
            }
            if (!GROUP_ROW && (idx % 32) == 0) a[(int64_t)b * M + row] = scale;
        }
    }
    if (GROUP_ROW && threadIdx.x == 0) a[row] = div_rn(fmaxf(rmax, 1e-10f), 127.0f);
}

}  // namespace prism

using namespace prism;

extern "C" int prism_quant_rows_i8(const uint16_t* x, int64_t ldx, const float* inv_s, int8_t* q, float* s,
                                   const int32_t* n_rows, int64_t M, int64_t K, void* stream) {
    if (!x || !q || !s || !n_rows) return PRISM_ERR_ARG;
    if (M < 0 || K <= 0 || K % 8 || K > 65536 || ldx < K || ldx % 8) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(x, 16) || !PRISM_ALIGNED(q, 16) || (inv_s && !PRISM_ALIGNED(inv_s, 16)))
        return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    const int need = (int)((K / 8 + kQThreads - 1) / kQThreads);
    dim3 grid((unsigned)M);
#define QR(N) hipLaunchKernelGGL(quant_rows_i8_kernel<N>, grid, dim3(kQThreads), 0, st, x, ldx, inv_s, q, s, n_rows, (int)K)
    if (need <= 1) QR(1);
    else if (need <= 2) QR(2);
    else if (need <= 4) QR(4);
    else if (need <= 8) QR(8);
    else if (need <= 16) QR(16);
    else QR(32);
#undef QR
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_quant_rows_groups(const uint16_t* x, int8_t* q, float* s, const int32_t* n_rows, int64_t M,
                                       int64_t K, int64_t gk, void* stream) {
    if (!x || !q || !s || !n_rows) return PRISM_ERR_ARG;
    if (gk <= 0 || gk % 32 || K <= 0 || K % gk || M < 0 || K > (1 << 30)) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(x, 16) || !PRISM_ALIGNED(q, 16)) return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    const int64_t width = gk / 8;
    if (gk <= 512 && (width & (width - 1)) == 0) {
        dim3 grid((unsigned)((K / 8 + kQThreads - 1) / kQThreads), (unsigned)M);
        hipLaunchKernelGGL(quant_rows_groups_kernel, grid, dim3(kQThreads), 0, st, x, q, s, n_rows, (int)K, (int)gk);
    } else {
        dim3 grid((unsigned)(K / gk), (unsigned)M);
        hipLaunchKernelGGL(quant_rows_groups_slow_kernel, grid, dim3(kQThreads), 0, st, x, q, s, n_rows, (int)K,
                           (int)gk);
    }
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_quant_rows_g(const uint16_t* x, int64_t ldx, int8_t* xq, float* a, int8_t* xs,
                                  const int32_t* n_rows, int64_t M, int64_t K, int64_t group, void* stream) {
    if (!x || !xq || !a || !xs || !n_rows) return PRISM_ERR_ARG;
    if (M < 0 || K <= 0 || K % 256 || K > 65536 || ldx < K || ldx % 8) return PRISM_ERR_SHAPE;
    if (group != 256 && group != K) return PRISM_ERR_ARG;
    if (!PRISM_ALIGNED(x, 16) || !PRISM_ALIGNED(xq, 16)) return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    const int need = (int)((K / 8 + kQThreads - 1) / kQThreads);
    dim3 grid((unsigned)M);
    const bool row = group == K && K != 256;
#define QG(N)                                                                                                       \
    do {                                                                                                            \
        if (row)                                                                                                    \
            hipLaunchKernelGGL((quant_rows_g_kernel<N, true>), grid, dim3(kQThreads), 0, st, x, ldx, xq, a, xs,    \
                               n_rows, (int)M, (int)K);                                                             \
        else                                                                                                        \
            hipLaunchKernelGGL((quant_rows_g_kernel<N, false>), grid, dim3(kQThreads), 0, st, x, ldx, xq, a, xs,   \
                               n_rows, (int)M, (int)K);                                                             \
    } while (0)
    if (need <= 1) QG(1);
    else if (need <= 2) QG(2);
    else if (need <= 4) QG(4);
    else if (need <= 8) QG(8);
    else if (need <= 16) QG(16);
    else QG(32);
#undef QG
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}
