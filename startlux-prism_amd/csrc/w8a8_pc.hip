// Per-channel W8A8 GEMM (gk = K: one activation scale per token, one weight scale per output channel) for gfx950.
// The engine's production projections (kernels/w8a8.py:183-231 with gk == K; the CUDA w8a8_kernel epilogue,
// csrc/w8a8_gemm.cu:298-402): P = sum_k a w in int32 (exact), y = RN(RN(float(P) sa) sw); epilogue 0 stores bf16(y),
// epilogue 1 out = RN(out + y).  With a single group there is no per-block fp32 work, so this is a plain int8 MFMA
// GEMM with an epilogue, and the int32 sum is exact in any order.
//
// Tile: 256 x 256 outputs per 256-thread workgroup, 4 waves of 128 x 128 (4 x 4 v_mfma_i32_32x32x32_i8 per 32
// inputs, 256 int32 accumulators per lane).  Operands go global -> LDS by LDS-DMA (global_load_lds_dwordx4), NS
// stages of 64 inputs: per stage and operand 256 rows x 64 bytes, each DMA instruction 16 rows x 64 bytes (lane L:
// row L / 4, 16-byte chunk L % 4 XOR-swizzled by row so that the fragment reads of 8 consecutive rows hit distinct
// banks).  MFMA operand mapping: lane l holds row l % 32 and the 16 inputs of chunk 2 s + l / 32 for the stage's
// 32-input step s, the same for both operands.
#include "common.h"

namespace prism {

constexpr int PCT = 256;                        // tile rows and columns
constexpr int PCK = 64;                         // inputs per stage
constexpr int PC_OPER = PCT * PCK;              // bytes per operand per stage (16 KB)
constexpr int PC_STAGE = 2 * PC_OPER;

__device__ __forceinline__ int pc_swz(int row) { return (row >> 1) & 3; }

__device__ __forceinline__ void pc_dma(const void* g, uint8_t* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void pc_vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <bool WS16, int EPI, int NS>
__global__ __launch_bounds__(256, 1) void w8a8_pc_tile_kernel(const int8_t* __restrict__ a,
                                                              const float* __restrict__ a_s, int64_t as_sm,
                                                              const int8_t* __restrict__ w,
                                                              const void* __restrict__ w_s, void* __restrict__ out,
                                                              int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                              int N, int K, int tiles_m, int tiles_n) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];   // NS x [A 256 x 64 | W 256 x 64]
    __shared__ float sal[PCT], swl[PCT];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * PCT, n0 = pn * PCT;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int KS = K / PCK;

    // epilogue scales of the tile
    sal[tid] = a_s[(int64_t)min(m0 + tid, M - 1) * as_sm];
    {
        const int n = min(n0 + tid, N - 1);
        swl[tid] = WS16 ? f16_to_f32(static_cast<const uint16_t*>(w_s)[n]) : static_cast<const float*>(w_s)[n];
    }

    // DMA sources: instruction i of wave wv covers operand rows 16 (4 wv + i) .. + 15
    const int8_t* asrc[4];
    const int8_t* wsrc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = 16 * (4 * wv + i) + (lane >> 2);
        const int c = (lane & 3) ^ pc_swz(row);
        asrc[i] = a + (int64_t)min(m0 + row, M - 1) * K + 16 * c;
        wsrc[i] = w + (int64_t)min(n0 + row, N - 1) * K + 16 * c;
    }
    auto issue = [&](int st, int buf) {
        uint8_t* b = lds + buf * PC_STAGE;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pc_dma(asrc[i] + (int64_t)st * PCK, b + (4 * wv + i) * 1024);
            pc_dma(wsrc[i] + (int64_t)st * PCK, b + PC_OPER + (4 * wv + i) * 1024);
        }
    };

    const int wm = wv >> 1, wn = wv & 1;
    const int r = lane & 31, h = lane >> 5;
    // fragment byte offsets within an operand stage, for the two 32-input steps s
    int aoff[2][4], woff[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int ra = 128 * wm + 32 * t + r, rw = 128 * wn + 32 * t + r;
            aoff[s][t] = ra * PCK + 16 * ((2 * s + h) ^ pc_swz(ra));
            woff[s][t] = rw * PCK + 16 * ((2 * s + h) ^ pc_swz(rw));
        }

    v16i acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[t][u][e] = 0;

#pragma unroll
    for (int i = 0; i < NS - 1; i++)
        if (i < KS) issue(i, i);

    for (int st = 0; st < KS; st++) {
        const int pend = min(KS - 1, st + NS - 2) - st;     // stages issued after this one
        if (NS >= 4 && pend >= 2) pc_vm_wait<16>();
        else if (pend >= 1) pc_vm_wait<8>();
        else pc_vm_wait<0>();
        lds_barrier();
        if (st + NS - 1 < KS) issue(st + NS - 1, (st + NS - 1) % NS);
        const uint8_t* b = lds + (st % NS) * PC_STAGE;
#pragma unroll
        for (int s = 0; s < 2; s++) {
            v4i fa[4], fw[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                fa[t] = *reinterpret_cast<const v4i*>(b + aoff[s][t]);
                fw[t] = *reinterpret_cast<const v4i*>(b + PC_OPER + woff[s][t]);
            }
            // D = W x A: lane l holds activation row l % 32 of the m-subtile and weight rows
            // 8 (e / 4) + 4 (l / 32) + e % 4 of the n-subtile
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int u = 0; u < 4; u++)
                    acc[t][u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[u], fa[t], acc[t][u], 0, 0, 0);
        }
    }

#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int ml = 128 * wm + 32 * t + r;
        const int m = m0 + ml;
        if (m >= live) continue;
        const float sa = sal[ml];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int nl = 128 * wn + 32 * u + 8 * g + 4 * h;
                const int n = n0 + nl;
                if (n >= N) continue;
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = mul_rn(mul_rn((float)acc[t][u][4 * g + e], sa), swl[nl + e]);
                if (EPI == 0) {
                    uint16_t* o = static_cast<uint16_t*>(out) + (int64_t)m * ldo + n;
                    *reinterpret_cast<v2u*>(o) = v2u{f32_to_bf16(y[0]) | (f32_to_bf16(y[1]) << 16),
                                                     f32_to_bf16(y[2]) | (f32_to_bf16(y[3]) << 16)};
                } else {
                    float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * ldo + n);
                    const float4 p = *o;
                    *o = make_float4(add_rn(p.x, y[0]), add_rn(p.y, y[1]), add_rn(p.z, y[2]), add_rn(p.w, y[3]));
                }
            }
    }
}

template <typename F>
static void pc_allow(F* fn, size_t bytes) {
    (void)hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

// Launch the per-channel tile kernel; the caller has checked K % 64 == 0, 16-byte aligned a / w, and (for the
// vector stores) ldo % 4 == 0 with an 8 / 16-byte aligned out.
int launch_w8a8_pc_tile(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* w, const void* w_s, bool ws16,
                        void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int epi, hipStream_t st) {
    constexpr int NS = 4;
    const int tiles_m = (M + PCT - 1) / PCT, tiles_n = (N + PCT - 1) / PCT;
    const size_t lds = (size_t)NS * PC_STAGE;
#define PCL(W16, E)                                                                                                \
    do {                                                                                                           \
        pc_allow(w8a8_pc_tile_kernel<W16, E, NS>, lds);                                                            \
        hipLaunchKernelGGL((w8a8_pc_tile_kernel<W16, E, NS>), dim3(tiles_m * tiles_n), dim3(256), lds, st, a, a_s,  \
                           as_sm, w, w_s, out, ldo, n_rows, M, N, K, tiles_m, tiles_n);                             \
    } while (0)
    if (ws16) { if (epi == 0) PCL(true, 0); else PCL(true, 1); }
    else { if (epi == 0) PCL(false, 0); else PCL(false, 1); }
#undef PCL
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

}  // namespace prism
