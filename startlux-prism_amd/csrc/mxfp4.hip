// MXFP4 GEMM for gfx950: e2m1 weights (one e8m0 scale per 32 inputs) against e4m3 or e2m1 activations (one e8m0
// scale per 32 inputs), fp32 accumulation on v_mfma_scale_f32_16x16x128_f8f6f4, bf16 store or fp32 residual add.
// Restates kernels/mxfp4.py (pack :57-86, quantize_act :124-185, _gemm_kernel :260-289, gemm :292-317) and the C4
// conventions of tests/quant_sim.py:66-81 (mxfp4 weights, mxfp8 activations).
//
// Device weight layout (MX4 on the GPU), N % 16 == 0 and K % 128 == 0:
//   q [N/16][K/128][64][16] bytes: tile t, step s, lane L = 16 p + i holds the 32 e2m1 codes (low nibble first) of
//                                  row 16 t + i, inputs 128 s + 32 p .. + 31 -- one MFMA A operand per lane, so a
//                                  wave's operand for one (tile, step) is 1 KB of contiguous bytes;
//   s [N/16][K/128][64] bytes:     the e8m0 scale of that lane's 32 inputs.
// Activations keep the engine's row-major layout: e4m3 q [M, K] or e2m1 q [M, K/2], e8m0 s [M, K/32].
//
// MFMA operand mapping (v_mfma_scale_f32_16x16x128_f8f6f4, A = weights, B = activations; measured on gfx950):
//   e2m1 operand, lane L = 16 p + r: row r, inputs 32 p .. 32 p + 31 (4 dwords, low nibble = lower input);
//   e4m3 operand, lane L = 16 p + r: row r, bytes 0-15 = inputs 16 p .. + 15, bytes 16-31 = inputs 64 + 16 p .. + 15;
//   scale operand, lane L = 16 p + r: the e8m0 scale of row r, inputs 32 p .. + 31 (byte 0 of the dword);
//   D, lane L: activation row L % 16, weight rows 4 (L / 16) .. + 3.
//
// Accumulation order (the same in every kernel, so an output's bits do not depend on the batch it is computed in
// nor on the kernel chosen): inputs are taken in steps of 128, one MFMA each; the steps of one 1024-input segment
// chain through the MFMA accumulator from zero; the segment sums are added left to right in fp32.
#include "common.h"

namespace prism {

typedef int v8i __attribute__((ext_vector_type(8)));

constexpr int kMxStep = 128;          // inputs per MFMA
constexpr int kMxSegSteps = 8;        // MFMA steps per accumulation segment (1024 inputs)

// ------------------------------------------------------------------------------------------------ element codes
// |x| / scale -> e2m1 magnitude code.  TIES == 0: strict thresholds, midpoints toward zero (kernels/mxfp4.py:40-54,
// :110-121).  TIES == 1: nearest, ties to the even code (the OCP conversion of the C4 weights).
template <int TIES>
__device__ __forceinline__ uint32_t e2m1_mag(float a) {
    if (TIES == 0)
        return (a > .25f) + (a > .75f) + (a > 1.25f) + (a > 1.75f) + (a > 2.5f) + (a > 3.5f) + (a > 5.f);
    return (a > .25f) + (a >= .75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) + (a > 5.f);
}

// 2^e for an integer e in [-126, 127] (exact).
__device__ __forceinline__ float pow2i(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// e2m1 code -> value: magnitudes 0, .5, 1, 1.5 (code / 2) and 2^((c >> 1) - 1) * (1 + (c & 1) / 2) above.
__device__ __forceinline__ float e2m1_val(uint32_t c) {
    const uint32_t m = c & 7;
    const float v = m < 2 ? 0.5f * (float)m : pow2i((int)(m >> 1) - 1) * ((m & 1) ? 1.5f : 1.f);
    return (c & 8) ? -v : v;
}

// floor / ceil of log2 of a positive normal fp32 value, from its exponent bits.
__device__ __forceinline__ int ilog2_floor(float v) { return (int)((__float_as_uint(v) >> 23) & 0xff) - 127; }
__device__ __forceinline__ int ilog2_ceil(float v) {
    const uint32_t u = __float_as_uint(v);
    return (int)((u >> 23) & 0xff) - 127 + ((u & 0x7fffffu) != 0);
}

// fp32 (|v| <= 448) -> e4m3 code, round to nearest even; the sign bit follows the input's.
__device__ __forceinline__ uint32_t e4m3_code(float v) {
    const uint32_t sgn = (__float_as_uint(v) >> 24) & 0x80u;
    const float a = fabsf(v);
    if (a < 0x1p-6f) return sgn | (uint32_t)__builtin_rintf(a * 512.f);
    const int E = ilog2_floor(a);
    const uint32_t m = (uint32_t)__builtin_rintf(a * pow2i(3 - E));
    return sgn | (uint32_t)((E + 6) * 8 + (int)m);
}

// ------------------------------------------------------------------------------------------------ weight pack
// fp32 [N, K] (row stride ldw) -> device layout.  One workgroup of 64 threads per (16-row tile, 128-input step);
// thread L quantizes row 16 t + L % 16, block 4 s + L / 16 and writes its 16 code bytes and scale byte.
// MODE 0 "max", 1 "mse" (kernels/mxfp4.py:57-86), 2 "ocp" (tests/quant_sim.py:66-72, nearest-even codes).
template <int MODE>
__global__ __launch_bounds__(64) void mx_pack_kernel(const float* __restrict__ w, int64_t ldw,
                                                     uint8_t* __restrict__ q, uint8_t* __restrict__ s, int K) {
    const int KS = K / kMxStep;
    const int t = blockIdx.y, st = blockIdx.x, L = threadIdx.x;
    const int row = 16 * t + (L & 15), blk = 4 * st + (L >> 4);
    const float4* src = reinterpret_cast<const float4*>(w + (int64_t)row * ldw + 32 * blk);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 f = src[i];
        v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    int e;
    if (MODE == 2) {
        e = ilog2_floor(fmaxf(amax, 1e-30f)) - 2;
    } else {
        e = min(127, max(-127, ilog2_ceil(div_rn(fmaxf(amax, 1e-30f), 6.0f))));
        if (MODE == 1) {
            // the power of two among e and e - 1 with the smaller squared error, summed as numpy sums 32 float32
            // values (eight strided partial sums, then a fixed tree)
            const int e1 = max(-127, e - 1);
            float err[2];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int ec = c ? e1 : e;
                const float sc = pow2i(ec), inv = pow2i(-ec);
                float r[8];
#pragma unroll
                for (int i = 0; i < 32; i++) {
                    const uint32_t m = e2m1_mag<0>(fabsf(v[i]) * inv);
                    float dq = mul_rn(e2m1_val(m), sc);
                    if (v[i] < 0.f && m) dq = -dq;
                    const float d = dq - v[i];
                    r[i & 7] = i < 8 ? mul_rn(d, d) : add_rn(r[i & 7], mul_rn(d, d));
                }
                err[c] = add_rn(add_rn(add_rn(r[0], r[1]), add_rn(r[2], r[3])),
                                add_rn(add_rn(r[4], r[5]), add_rn(r[6], r[7])));
            }
            if (err[1] < err[0]) e = e1;
        }
    }
    const float inv = pow2i(-e);
    uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        float a = fabsf(v[i]) * inv;
        uint32_t c = MODE == 2 ? e2m1_mag<1>(fminf(a, 6.f)) : e2m1_mag<0>(a);
        if (v[i] < 0.f && c) c |= 8;
        words[i >> 3] |= c << (4 * (i & 7));
    }
    const int64_t o = ((int64_t)t * KS + st) * 64 + L;
    reinterpret_cast<v4u*>(q)[o] = v4u{words[0], words[1], words[2], words[3]};
    s[o] = (uint8_t)(e + 127);
}

// Row-major MX4 (q [N, K/2], s [N, K/32], kernels/mxfp4.py:25-30) -> device layout; the same thread mapping.
__global__ __launch_bounds__(64) void mx_repack_kernel(const uint8_t* __restrict__ qr, const uint8_t* __restrict__ sr,
                                                       uint8_t* __restrict__ q, uint8_t* __restrict__ s, int K) {
    const int KS = K / kMxStep;
    const int t = blockIdx.y, st = blockIdx.x, L = threadIdx.x;
    const int row = 16 * t + (L & 15), blk = 4 * st + (L >> 4);
    const int64_t o = ((int64_t)t * KS + st) * 64 + L;
    reinterpret_cast<v4u*>(q)[o] = *reinterpret_cast<const v4u*>(qr + (int64_t)row * (K / 2) + 16 * blk);
    s[o] = sr[(int64_t)row * (K / 32) + blk];
}

// ------------------------------------------------------------------------------------------ activation quantizer
// Panel layout of e4m3 activations (PRISM_MX_E4M3_PANELS): 16-row blocks, each a run of K / 128 chunks of 2 KB, one
// per 128-input step, holding the step's 16 rows as the tile kernel's lanes load them: byte h 1024 + (16 p + r) 16 + i
// is row 16 b + r, input 128 st + 64 h + 16 p + i.  A wave's activation load for a step is then 2 KB in one piece
// instead of 16 rows' 128 bytes K apart.  Block b starts at byte 16 b K, as row 16 b does in the row-major layout.
__host__ __device__ __forceinline__ int64_t mx_act_panel_offset(int64_t row, int64_t k, int64_t K) {
    const int64_t st = k >> 7, h = (k >> 6) & 1, p = (k >> 4) & 3;
    return (row >> 4) * 16 * K + st * 2048 + h * 1024 + (16 * p + (row & 15)) * 16 + (k & 15);
}

// One thread per (row, 32-input block).  AF 4: kernels/mxfp4.py:124-146 (_quant_kernel; with inv, :149-170
// _quant_scaled_kernel): e = clip(ceil(log2(max(amax, 1e-30) / 6)), +-127), strict-threshold codes, the sign bit
// set for every negative input.  AF 0: tests/quant_sim.py:75-81 (mxfp8): e = floor(log2(max(amax, 1e-30))) - 8,
// codes e4m3(clamp(x / 2^e, +-448)) nearest even.  XF32: fp32 input, else bf16.  Rows >= n_rows are skipped.
// PAN (e4m3 only): q in the panel layout mx_act_panel_offset defines instead of row-major.
template <int AF, bool XF32, bool PAN = false>
__global__ __launch_bounds__(256) void mx_quant_act_kernel(const void* __restrict__ x, int64_t ldx,
                                                           const float* __restrict__ inv, uint8_t* __restrict__ q,
                                                           uint8_t* __restrict__ s,
                                                           const int32_t* __restrict__ n_rows, int M, int K) {
    const int row = blockIdx.y;
    const int blk = blockIdx.x * blockDim.x + threadIdx.x;
    const int live = n_rows ? min(M, __ldg(n_rows)) : M;
    if (row >= live || blk >= K / 32) return;
    float v[32];
    if (XF32) {
        const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(x) + row * ldx + 32 * blk);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = src[i];
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
        }
    } else {
        const v4u* src = reinterpret_cast<const v4u*>(static_cast<const uint16_t*>(x) + row * ldx + 32 * blk);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const v4u u = src[i];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[8 * i + 2 * j] = bf16_to_f32(u[j] & 0xffffu);
                v[8 * i + 2 * j + 1] = bf16_to_f32(u[j] >> 16);
            }
        }
    }
    if (inv) {
        const float4* iv = reinterpret_cast<const float4*>(inv + 32 * blk);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = iv[i];
            v[4 * i] = mul_rn(v[4 * i], f.x);
            v[4 * i + 1] = mul_rn(v[4 * i + 1], f.y);
            v[4 * i + 2] = mul_rn(v[4 * i + 2], f.z);
            v[4 * i + 3] = mul_rn(v[4 * i + 3], f.w);
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    int e;
    if (AF == 0) {
        e = ilog2_floor(fmaxf(amax, 1e-30f)) - 8;
        const float r = pow2i(-e);
        uint32_t words[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const float a = fminf(fmaxf(v[i] * r, -448.f), 448.f);
            words[i >> 2] |= e4m3_code(a) << (8 * (i & 3));
        }
        if (PAN) {                                         // the block's two 16-byte pieces p = 2 (blk % 2) + 0, 1
            uint8_t* d = q + mx_act_panel_offset(row, 32 * blk, K);
            *reinterpret_cast<v4u*>(d) = v4u{words[0], words[1], words[2], words[3]};
            *reinterpret_cast<v4u*>(d + 256) = v4u{words[4], words[5], words[6], words[7]};
        } else {
            v4u* dst = reinterpret_cast<v4u*>(q + (int64_t)row * K + 32 * blk);
            dst[0] = v4u{words[0], words[1], words[2], words[3]};
            dst[1] = v4u{words[4], words[5], words[6], words[7]};
        }
    } else {
        e = min(127, max(-127, ilog2_ceil(div_rn(fmaxf(amax, 1e-30f), 6.0f))));
        const float r = pow2i(-e);
        uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t c = e2m1_mag<0>(fabsf(v[i]) * r) | (v[i] < 0.f ? 8u : 0u);
            words[i >> 3] |= c << (4 * (i & 7));
        }
        *reinterpret_cast<v4u*>(q + (int64_t)row * (K / 2) + 16 * blk) = v4u{words[0], words[1], words[2], words[3]};
    }
    s[(int64_t)row * (K / 32) + blk] = (uint8_t)(e + 127);
}

// ------------------------------------------------------------------------------------------------ MFMA helpers
template <int AF>
__device__ __forceinline__ v4f mx_mfma(v4i w, v8i a, v4f c, uint32_t ws, uint32_t as) {
    const v8i wa = {w.x, w.y, w.z, w.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wa, a, c, 4, AF, 0, (int)ws, 0, (int)as);
}

// Epilogue for one D fragment: activation row m, weight rows n .. n + 3.  EPI 0: bf16 RNE store
// (kernels/mxfp4.py:286-287); EPI 1: out = out + y in fp32 (:283-285).
template <int EPI>
__device__ __forceinline__ void mx_store(void* out, int64_t ldo, int m, int n, v4f y) {
    if (EPI == 0) {
        uint16_t* o = static_cast<uint16_t*>(out) + (int64_t)m * ldo + n;
        *reinterpret_cast<v2u*>(o) = v2u{f32_to_bf16(y.x) | (f32_to_bf16(y.y) << 16),
                                         f32_to_bf16(y.z) | (f32_to_bf16(y.w) << 16)};
    } else {
        float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * ldo + n);
        const float4 p = *o;
        *o = make_float4(add_rn(p.x, y.x), add_rn(p.y, y.y), add_rn(p.z, y.z), add_rn(p.w, y.w));
    }
}

// ------------------------------------------------------------------------------------------------ decode kernel
// M <= 16 MT.  One workgroup per 16-row weight tile; wave w owns segments w, w + NW, ...  A wave issues every load
// of a segment (weights 16 B per lane per step, activations from L2) before its MFMAs, writes the segment's
// fp32 sums to LDS, and after one barrier the workgroup adds the segments left to right and stores.
template <int MT, int AF, int EPI>
__global__ __launch_bounds__(MT == 1 ? 1024 : 512) void mx_decode_kernel(const uint8_t* __restrict__ aq,
                                                         const uint8_t* __restrict__ as,
                                                         const uint8_t* __restrict__ wq,
                                                         const uint8_t* __restrict__ ws, void* __restrict__ out,
                                                         int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                         int K) {
    extern __shared__ __attribute__((aligned(16))) v4f part[];    // [nseg][MT][64]
    kernel_args_now(aq, as, wq, ws, out, ldo, n_rows, M, K);
    const int t = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6, NW = blockDim.x >> 6;
    const int KS = K / kMxStep, nseg = (KS + kMxSegSteps - 1) / kMxSegSteps;
    const int live = n_rows ? min(M, __ldg(n_rows)) : M;
    const int p = lane >> 4, r = lane & 15;
    const int64_t abytes = AF == 0 ? K : K / 2;
    const uint8_t* arow[MT];
    const uint8_t* srow[MT];
#pragma unroll
    for (int u = 0; u < MT; u++) {
        const int m = min(16 * u + r, M - 1);
        arow[u] = aq + (int64_t)m * abytes + 16 * p;
        srow[u] = as + (int64_t)m * (K / 32) + p;
    }
    const v4u* wbase = reinterpret_cast<const v4u*>(wq) + (int64_t)t * KS * 64 + lane;
    const uint8_t* sbase = ws + (int64_t)t * KS * 64 + lane;

    // steps loaded per batch: the whole segment while the registers allow it
    constexpr int B = MT <= 2 ? kMxSegSteps : kMxSegSteps / 2;
    for (int seg = w; seg < nseg; seg += NW) {
        const int s0 = seg * kMxSegSteps, ns = min(kMxSegSteps, KS - s0);
        v4f acc[MT];
#pragma unroll
        for (int u = 0; u < MT; u++) acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j0 = 0; j0 < kMxSegSteps; j0 += B) {
            if (j0 >= ns) break;
            v4u wv[B];
            uint32_t wsc[B];
            v8i av[B][MT];
            uint32_t asc[B][MT];
#pragma unroll
            for (int j = 0; j < B; j++) {
                const int st = min(s0 + j0 + j, KS - 1);
                wv[j] = wbase[(int64_t)st * 64];
                wsc[j] = sbase[(int64_t)st * 64];
#pragma unroll
                for (int u = 0; u < MT; u++) {
                    if (AF == 0) {
                        const v4u lo = *reinterpret_cast<const v4u*>(arow[u] + (int64_t)st * 128);
                        const v4u hi = *reinterpret_cast<const v4u*>(arow[u] + (int64_t)st * 128 + 64);
                        av[j][u] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z,
                                       (int)hi.w};
                    } else {
                        const v4u lo = *reinterpret_cast<const v4u*>(arow[u] + (int64_t)st * 64);
                        av[j][u] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, 0, 0, 0, 0};
                    }
                    asc[j][u] = srow[u][st * 4];
                }
            }
#pragma unroll
            for (int j = 0; j < B; j++) {
                if (j0 + j < ns) {
                    const v4i wi = {(int)wv[j].x, (int)wv[j].y, (int)wv[j].z, (int)wv[j].w};
#pragma unroll
                    for (int u = 0; u < MT; u++) acc[u] = mx_mfma<AF>(wi, av[j][u], acc[u], wsc[j], asc[j][u]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < MT; u++) part[(seg * MT + u) * 64 + lane] = acc[u];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < MT * 64; idx += blockDim.x) {
        const int u = idx >> 6, l = idx & 63;
        const int m = 16 * u + (l & 15);
        if (m >= live) continue;
        v4f y = part[u * 64 + l];
        for (int seg = 1; seg < nseg; seg++) {
            const v4f z = part[(seg * MT + u) * 64 + l];
            y = v4f{add_rn(y.x, z.x), add_rn(y.y, z.y), add_rn(y.z, z.z), add_rn(y.w, z.w)};
        }
        mx_store<EPI>(out, ldo, m, 16 * t + 4 * (l >> 4), y);
    }
}

// ------------------------------------------------------------------------------------------------ tile kernel
// Workgroup tile: WM x WN waves of 16 AR x 64 outputs (4 x AR MFMAs per step), 16 AR WM activation rows by 64 WN
// weight rows.  Default: 64 x 256 (4 waves of 64 x 64), two LDS stages of 29 KB, two workgroups per CU.  Every step
// ends in a workgroup barrier, so the waves of one workgroup read their fragments from LDS and then run their MFMAs
// in the same phase.  Two workgroups per CU drift apart, and one's LDS reads overlap the other's MFMAs.  The 64 x 256
// tile ran 4-6% faster than one 128 x 256 workgroup of 8 waves per CU with three stages.  Operands move global -> LDS by LDS-DMA (global_load_lds_dwordx4 / _ubyte), NS stages deep,
// already in MFMA operand order, so each wave reads its fragments with contiguous ds_read_b128 and no VGPR staging.
template <int AF, int WM, int WN, int AR>
struct MxStage {
    static constexpr int TW = 4 * WN, TA = AR * WM;               // 16-row weight / activation tiles
    static constexpr int WQ = 0;                                  // TW tiles x 1 KB
    static constexpr int AQ = TW * 1024;                          // TA tiles x (2 KB e4m3 | 1 KB e2m1)
    static constexpr int WS = AQ + TA * (AF == 0 ? 2048 : 1024);  // TW tiles x 64 lanes x 4 B
    static constexpr int AS = WS + TW * 256;                      // TA tiles x 64 lanes x 4 B
    static constexpr int DUMMY = AS + TA * 256;                   // 1 KB sink for surplus copies (below)
    static constexpr int BYTES = DUMMY + (TA < WM * WN || TA * (AF == 0 ? 2 : 1) < WM * WN ? 1024 : 0);
    // DMA instructions per wave per stage: weights, activations, weight scales, activation scales
    // (activation shares below one per wave: every wave still issues one copy, so each wave's count of copies in
    // flight, which the stage waits name, is the same; the surplus copies land in the DUMMY sink)
    static constexpr int A_N = TA * (AF == 0 ? 2 : 1), W_PW = TW / (WM * WN);
    static constexpr int A_PW = A_N >= WM * WN ? A_N / (WM * WN) : 1;
    static constexpr int WS_PW = W_PW, AS_PW = TA >= WM * WN ? TA / (WM * WN) : 1;
    static_assert(W_PW >= 1 && W_PW * WM * WN == TW, "every wave copies a share of the weights");
    static_assert(A_N % (WM * WN) == 0 || A_N < WM * WN, "activation shares");
    static constexpr int LOADS = W_PW + A_PW + WS_PW + AS_PW;
};

template <int AF, int EPI, int NS, int WM, int WN, int AR>
__global__ __launch_bounds__(64 * WM * WN, WM * WN <= 4 ? 2 : 1) void mx_tile_kernel(const uint8_t* __restrict__ aq, const uint8_t* __restrict__ as,
                                                         const uint8_t* __restrict__ wq,
                                                         const uint8_t* __restrict__ ws, void* __restrict__ out,
                                                         int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                         int N, int K, int tiles_m, int tiles_n) {
    using S = MxStage<AF, WM, WN, AR>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * 16 * AR * WM, n0 = pn * 64 * WN;
    const int live = n_rows ? min(M, __ldg(n_rows)) : M;
    if (m0 >= live) return;
    const int KS = K / kMxStep, NT = N / 16;
    const int p = lane >> 4, r = lane & 15;
    const int64_t abytes = AF == 0 ? K : K / 2;

    // per-wave DMA sources (step 0); each advances by a fixed stride per step
    const uint8_t* wsrc[S::W_PW];
    const uint8_t* wssrc[S::WS_PW];
    const uint8_t* asrc[S::A_PW];
    const uint8_t* assrc[S::AS_PW];
#pragma unroll
    for (int i = 0; i < S::W_PW; i++) {
        const int tt = min(n0 / 16 + S::W_PW * w + i, NT - 1);
        wsrc[i] = wq + (int64_t)tt * KS * 1024 + lane * 16;
        wssrc[i] = ws + (int64_t)tt * KS * 64 + lane;
    }
#pragma unroll
    for (int i = 0; i < S::AS_PW; i++) {
        const int m = min(m0 + 16 * (S::AS_PW * w + i) + r, M - 1);
        assrc[i] = as + (int64_t)m * (K / 32) + p;
    }
#pragma unroll
    for (int i = 0; i < S::A_PW; i++) {
        const int idx = S::A_PW * w + i;
        const int u = AF == 0 ? idx >> 1 : idx, h = AF == 0 ? idx & 1 : 0;
        const int m = min(m0 + 16 * u + r, M - 1);
        asrc[i] = aq + (int64_t)m * abytes + 64 * h + 16 * p;
    }

    auto issue = [&](int st, int buf) {
        uint8_t* b = lds + buf * S::BYTES;
#pragma unroll
        for (int i = 0; i < S::W_PW; i++)
            dma16(wsrc[i] + (int64_t)st * 1024, b + S::WQ + (S::W_PW * w + i) * 1024);
#pragma unroll
        for (int i = 0; i < S::A_PW; i++) {
            const int idx = S::A_PW * w + i;
            dma16(asrc[i] + (int64_t)st * (AF == 0 ? 128 : 64), b + (idx < S::A_N ? S::AQ + idx * 1024 : S::DUMMY));
        }
#pragma unroll
        for (int i = 0; i < S::WS_PW; i++) dma1(wssrc[i] + (int64_t)st * 64, b + S::WS + (S::WS_PW * w + i) * 256);
#pragma unroll
        for (int i = 0; i < S::AS_PW; i++)
            dma1(assrc[i] + st * 4, b + (S::AS_PW * w + i < S::TA ? S::AS + (S::AS_PW * w + i) * 256 : S::DUMMY));
    };

    const int wn = w % WN, wm = w / WN;
    v4f acc[4][AR], tot[4][AR];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < AR; c++) acc[a][c] = tot[a][c] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int i = 0; i < NS - 1; i++)
        if (i < KS) issue(i, i);

    // segments of kMxSegSteps steps as an outer loop, so the fold below runs once per segment (as a conditional
    // inside the step loop the compiler executes it every step, predicated)
    for (int s0 = 0; s0 < KS; s0 += kMxSegSteps) {
    const int s1 = min(KS, s0 + kMxSegSteps);
    for (int st = s0; st < s1; st++) {
        const int pend = min(KS - 1, st + NS - 2) - st;
        if (NS >= 4 && pend >= 2) vm_wait<2 * S::LOADS>();
        else if (NS >= 3 && pend >= 1) vm_wait<S::LOADS>();
        else vm_wait<0>();
        lds_barrier();
        if (st + NS - 1 < KS) issue(st + NS - 1, (st + NS - 1) % NS);

        const uint8_t* b = lds + (st % NS) * S::BYTES;
        v4i wf[4];
        uint32_t wsf[4], asf[AR];
        v8i af[AR];
#pragma unroll
        for (int a = 0; a < 4; a++) {
            wf[a] = *reinterpret_cast<const v4i*>(b + S::WQ + (4 * wn + a) * 1024 + lane * 16);
            wsf[a] = *reinterpret_cast<const uint32_t*>(b + S::WS + (4 * wn + a) * 256 + lane * 4);
        }
#pragma unroll
        for (int c = 0; c < AR; c++) {
            const int u = AR * wm + c;
            if (AF == 0) {
                const v4i lo = *reinterpret_cast<const v4i*>(b + S::AQ + u * 2048 + lane * 16);
                const v4i hi = *reinterpret_cast<const v4i*>(b + S::AQ + u * 2048 + 1024 + lane * 16);
                af[c] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            } else {
                const v4i lo = *reinterpret_cast<const v4i*>(b + S::AQ + u * 1024 + lane * 16);
                af[c] = v8i{lo.x, lo.y, lo.z, lo.w, 0, 0, 0, 0};
            }
            asf[c] = *reinterpret_cast<const uint32_t*>(b + S::AS + u * 256 + lane * 4);
        }
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int c = 0; c < AR; c++) acc[a][c] = mx_mfma<AF>(wf[a], af[c], acc[a][c], wsf[a], asf[c]);
    }
    // segment sum into the running total, left to right (the first segment's sum is the total)
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < AR; c++) {
            const v4f z = acc[a][c];
            tot[a][c] = s0 == 0 ? z
                                : v4f{add_rn(tot[a][c].x, z.x), add_rn(tot[a][c].y, z.y), add_rn(tot[a][c].z, z.z),
                                      add_rn(tot[a][c].w, z.w)};
            acc[a][c] = v4f{0.f, 0.f, 0.f, 0.f};
        }
    }

#pragma unroll
    for (int c = 0; c < AR; c++) {
        const int m = m0 + 16 * (AR * wm + c) + r;
        if (m >= live) continue;
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const int n = n0 + 16 * (4 * wn + a) + 4 * p;
            if (n < N) mx_store<EPI>(out, ldo, m, n, tot[a][c]);
        }
    }
}


// Direct-weight tile kernel: the 64 x 256 tile of mx_tile_kernel's default (4 waves of 64 x 64, WM = 1), with each
// wave's weight fragments and scale bytes loaded straight into registers by buffer loads (a lane's 16 bytes of the
// 1 KB chunk and its scale byte are its MFMA operands as they lie), two steps ahead in a register ring; only the
// activation rows and their scales, which all four waves read, pass through LDS.  That takes the weights' LDS
// writes and fragment reads (about half the tile kernel's LDS traffic) off the LDS.  The activations are staged
// through registers with buffer loads and ds_write rather than LDS-DMA, so every request is a plain load and one
// counted wait covers both operands (an LDS-DMA and later buffer loads complete out of order).  Same MFMAs in the
// same order per output as mx_tile_kernel, the same segment folds: identical results.  PAN (e4m3): the activations
// in the panel layout, so each wave's load of a step is one 2 KB piece (C4: 131-138 -> 119-121 us).
template <int AF, int EPI, int WT, bool PAN = false>
__global__ __launch_bounds__(256, WT == 4 ? 2 : 1) void mx_tile_wd_kernel(const uint8_t* __restrict__ aq,
                                                            const uint8_t* __restrict__ as,
                                                            const uint8_t* __restrict__ wq,
                                                            const uint8_t* __restrict__ ws, void* __restrict__ out,
                                                            int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                            int N, int K, int tiles_m, int tiles_n) {
    constexpr int AR = 4, TA = 4;                          // activation tiles of 16 rows (one per wave to stage)
    constexpr int AT = AF == 0 ? 2048 : 1024;              // activation bytes per tile and step
    constexpr int ABUF = TA * AT + TA * 256;               // one LDS buffer: the tiles, then their scale dwords
    constexpr int AP = AF == 0 ? 2 : 1;                    // 16-byte activation loads per lane and step
    constexpr int WL = 2 * WT;                             // weight loads per step (WT fragments, WT scale bytes)
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * ABUF];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * 64, n0 = pn * 64 * WT;
    const int live = n_rows ? min(M, __ldg(n_rows)) : M;
    if (m0 >= live) return;
    const int KS = K / kMxStep, NT = N / 16;
    const int p = lane >> 4, r = lane & 15;
    const int abytes = AF == 0 ? K : K / 2;

    // wave w stages activation tile w: row m0 + 16 w + r, 16-byte piece p of each 64-byte half (e4m3: two halves)
    const int mr = min(m0 + 16 * w + r, M - 1) - m0;
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(aq + (int64_t)m0 * abytes);
    // (bounded: the last group of four steps' scales may reach past the last row when K / 128 is not a multiple of 4)
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc_n(as + (int64_t)m0 * (K / 32), (uint32_t)((M - m0) * (K / 32)));
    // activation scales: one 16-byte load per lane every fourth step, row mr's bytes of four steps (the lane's own is
    // byte 4 (st % 4) + p); single-byte loads every step measured 10% of the kernel's time at C4
    // panels: block m0 / 16 + w (clamped to the last), the lane's 16 bytes of each 1 KB half
    const uint32_t ao = PAN ? (uint32_t)((min(m0 / 16 + w, (M - 1) / 16) - m0 / 16) * 16 * K + 16 * lane)
                            : (uint32_t)(mr * abytes + 16 * p);
    const uint32_t so = (uint32_t)(mr * (K / 32));
    // weights: tile 4 w + a of the workgroup's 16 (clamped), lane slot l of its chunk, scale byte l
    const int nt0 = n0 / 16;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(wq + (int64_t)nt0 * KS * 1024);
    const __amdgpu_buffer_rsrc_t rws = buf_rsrc(ws + (int64_t)nt0 * KS * 64);
    uint32_t wo[WT], wso[WT];
#pragma unroll
    for (int a = 0; a < WT; a++) {
        const int t = min(nt0 + WT * w + a, NT - 1) - nt0;
        wo[a] = (uint32_t)(t * KS * 1024 + lane * 16);
        wso[a] = (uint32_t)(t * KS * 64 + lane);
    }
    struct Act { v4i q[AP]; };
    v4u sgrp[2];                                           // scale bytes of steps 4 g .. 4 g + 3, slot g % 2
    struct Wt { v4i f[WT]; uint32_t s[WT]; };
    Act xr[2];
    Wt wr[2];
    // st: the stage (clamped to the last for the addresses); sj: its position in the eight-step segment, known at
    // compile time, which picks the scale group's register slot (st is a multiple of 8 plus sj)
    auto load_a = [&](int st, int sj, Act& x) {
        const uint32_t sc = (uint32_t)min(st, KS - 1);
        // (issued before the step's activations: the waits below count the loads that follow those)
        if ((sj & 3) == 0) sgrp[(sj >> 2) & 1] = __builtin_bit_cast(v4u, buf_load16(rs, so, (sc & ~3u) * 4));
#pragma unroll
        for (int h = 0; h < AP; h++)
            x.q[h] = PAN ? buf_load16(ra, ao + 1024 * h, sc * 2048) : buf_load16(ra, ao + 64 * h, sc * (AF == 0 ? 128 : 64));
    };
    auto load_w = [&](int st, Wt& f) {
#pragma unroll
        for (int a = 0; a < WT; a++) f.f[a] = buf_load16(rw, wo[a], (uint32_t)st * 1024);
#pragma unroll
        for (int a = 0; a < WT; a++) f.s[a] = buf_load1(rws, wso[a], (uint32_t)st * 64);
    };
    auto stage_store = [&](int sj, const Act& x) {         // the LDS image mx_tile_kernel's DMA copies make
        uint8_t* b = lds + (sj & 1) * ABUF;
#pragma unroll
        for (int h = 0; h < AP; h++) *reinterpret_cast<v4i*>(b + w * AT + h * 1024 + lane * 16) = x.q[h];
        *reinterpret_cast<uint32_t*>(b + TA * AT + w * 256 + lane * 4) =
            __builtin_amdgcn_ubfe(sgrp[(sj >> 2) & 1][sj & 3], 8 * p, 8);
    };

    v4f acc[WT][AR], tot[WT][AR];
#pragma unroll
    for (int a = 0; a < WT; a++)
#pragma unroll
        for (int c = 0; c < AR; c++) acc[a][c] = tot[a][c] = v4f{0.f, 0.f, 0.f, 0.f};
    auto fold = [&](bool first) {                          // segment sum into the running total, left to right
#pragma unroll
        for (int a = 0; a < WT; a++)
#pragma unroll
            for (int c = 0; c < AR; c++) {
                const v4f z = acc[a][c];
                tot[a][c] = first ? z
                                  : v4f{add_rn(tot[a][c].x, z.x), add_rn(tot[a][c].y, z.y), add_rn(tot[a][c].z, z.z),
                                        add_rn(tot[a][c].w, z.w)};
                acc[a][c] = v4f{0.f, 0.f, 0.f, 0.f};
            }
    };

    // Both operands two steps ahead in two-slot register rings: step st requests stage st + 2's activations before
    // its MFMAs and its weights after them (into the slot those MFMAs free).  Stage indices past the last are
    // clamped (redundant loads into slots never read), so at step st's wait only stage st + 1's WL weight loads follow
    // stage st + 1's activations (a step whose activation scales start a group of four loads them first).
    load_a(0, 0, xr[0]);
    load_w(0, wr[0]);
    load_a(1, 1, xr[1]);
    load_w(min(1, KS - 1), wr[1]);
    vm_wait_tracked<2 * WL + AP>();                       // stage 0's scales and activations (stage 1 loads none)
    stage_store(0, xr[0]);
    lds_barrier();
    auto step = [&](int st, int sj) {                      // sj = st mod 8, known at compile time
        const int j = sj & 1;                              // the register slot
        vm_wait_tracked<WL>();
        stage_store(sj + 1, xr[j ^ 1]);                    // past the end: into the free buffer, never read
        const uint8_t* b = lds + j * ABUF;
        v8i af[AR];
        uint32_t asf[AR];
#pragma unroll
        for (int c = 0; c < AR; c++) {
            if (AF == 0) {
                const v4i lo = *reinterpret_cast<const v4i*>(b + c * AT + lane * 16);
                const v4i hi = *reinterpret_cast<const v4i*>(b + c * AT + 1024 + lane * 16);
                af[c] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            } else {
                const v4i lo = *reinterpret_cast<const v4i*>(b + c * AT + lane * 16);
                af[c] = v8i{lo.x, lo.y, lo.z, lo.w, 0, 0, 0, 0};
            }
            asf[c] = *reinterpret_cast<const uint32_t*>(b + TA * AT + c * 256 + lane * 4);
        }
        load_a(st + 2, sj + 2, xr[j]);
        lds_barrier();
#pragma unroll
        for (int a = 0; a < WT; a++)
#pragma unroll
            for (int c = 0; c < AR; c++) acc[a][c] = mx_mfma<AF>(wr[j].f[a], af[c], acc[a][c], wr[j].s[a], asf[c]);
        load_w(min(st + 2, KS - 1), wr[j]);
    };
    // segments of kMxSegSteps (8) steps, unrolled, the fold after each; the last segment may be shorter
    static_assert(kMxSegSteps == 8, "segment unroll");
    int st = 0;
    for (; st + kMxSegSteps <= KS; st += kMxSegSteps) {
#pragma unroll
        for (int j = 0; j < kMxSegSteps; j++) step(st + j, j);
        fold(st == 0);
    }
    if (st < KS) {
#pragma unroll
        for (int j = 0; j < kMxSegSteps - 1; j++)
            if (st + j < KS) step(st + j, j);
        fold(st == 0);
    }

#pragma unroll
    for (int c = 0; c < AR; c++) {
        const int m = m0 + 16 * c + r;
        if (m >= live) continue;
#pragma unroll
        for (int a = 0; a < WT; a++) {
            const int n = n0 + 16 * (WT * w + a) + 4 * p;
            if (n < N) mx_store<EPI>(out, ldo, m, n, tot[a][c]);
        }
    }
}

// ------------------------------------------------------------------------------ decode kernel, staged activations
// e4m3 activations, M <= 16.  One workgroup per NTG 16-row weight tiles; waves w = (tile w % NTG, segment lane
// w / NTG), SL segment lanes, segments taken in rounds of SL.  Per round every wave loads its segment's weights
// into registers while the workgroup copies the round's activation rows (16 rows x 1 KB per segment, one 1 KB row
// chunk per DMA instruction, rows padded to 1040 bytes so the fragment reads of 16 rows hit distinct banks) and
// their scales into LDS; the NTG tiles of a segment share one copy.  After the MFMAs each wave leaves its segment
// sum in LDS and the first NTG waves fold the round's segments, left to right, into their running sums.
constexpr int kDecRow = 1024 + 16;              // LDS bytes per staged activation row (one segment)
constexpr int kDecActSlot = 16 * kDecRow;       // one segment's 16 rows
constexpr int kDecScaleSlot = 16 * 32;          // their 32 scale bytes per row

static size_t mx_decode_staged_lds(int ntg, int sl) {
    return (size_t)sl * (kDecActSlot + kDecScaleSlot) + (size_t)sl * ntg * 64 * sizeof(v4f);
}

template <int NTG, int EPI>
__global__ __launch_bounds__(1024) void mx_decode_staged_kernel(const uint8_t* __restrict__ aq,
                                                                const uint8_t* __restrict__ as,
                                                                const uint8_t* __restrict__ wq,
                                                                const uint8_t* __restrict__ ws,
                                                                void* __restrict__ out, int64_t ldo,
                                                                const int32_t* __restrict__ n_rows, int M, int K,
                                                                int SL) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* act = lds;                                               // [SL][16][kDecRow]
    uint8_t* asl = lds + SL * kDecActSlot;                            // [SL][16][32]
    v4f* part = reinterpret_cast<v4f*>(asl + SL * kDecScaleSlot);     // [SL][NTG][64]
    kernel_args_now(aq, as, wq, ws, out, ldo, n_rows, M, K, SL);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nt = w % NTG, sl = w / NTG;
    const int t = blockIdx.x * NTG + nt;
    const int KS = K / kMxStep, nseg = (KS + kMxSegSteps - 1) / kMxSegSteps;
    const int live = n_rows ? min(M, __ldg(n_rows)) : M;
    const int p = lane >> 4, r = lane & 15;
    const v4u* wbase = reinterpret_cast<const v4u*>(wq) + (int64_t)t * KS * 64 + lane;
    const uint8_t* sbase = ws + (int64_t)t * KS * 64 + lane;
    const int nrounds = (nseg + SL - 1) / SL;
    v4f y = v4f{0.f, 0.f, 0.f, 0.f};

    for (int rd = 0; rd < nrounds; rd++) {
        const int seg = rd * SL + sl;
        const bool active = seg < nseg;
        const int s0 = min(seg, nseg - 1) * kMxSegSteps, ns = min(kMxSegSteps, KS - s0);
        // weights of the segment (registers)
        v4u wv[kMxSegSteps];
        uint32_t wsc[kMxSegSteps];
#pragma unroll
        for (int j = 0; j < kMxSegSteps; j++) {
            const int st = min(s0 + j, KS - 1);
            wv[j] = wbase[(int64_t)st * 64];
            wsc[j] = sbase[(int64_t)st * 64];
        }
        // activation rows of the segment -> LDS slot sl: the NTG waves of the slot split the 16 rows
        if (active) {
            uint8_t* slot = act + sl * kDecActSlot;
            for (int row = nt; row < 16; row += NTG) {
                const int m = min(row, M - 1);
                // a short last segment: lanes past its end re-read its last 16 bytes (never used)
                const uint8_t* src = aq + (int64_t)m * K + (int64_t)s0 * kMxStep + min(16 * lane, ns * kMxStep - 16);
                __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(slot + row * kDecRow),
                                                 16, 0, 0);
            }
            if (nt == 0) {   // 16 rows x 32 scale bytes: lane L covers row L / 8, bytes 4 (L % 8) .. + 3 (x2 instr.)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int row = 8 * h + (lane >> 3);
                    const int m = min(row, M - 1);
                    const uint8_t* src = as + (int64_t)m * (K / 32) + s0 * 4 + min(4 * (lane & 7), 4 * ns - 4);
                    __builtin_amdgcn_global_load_lds(
                        src, (__attribute__((address_space(3))) void*)(asl + sl * kDecScaleSlot + h * 256), 4, 0, 0);
                }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
        if (active) {
            const uint8_t* slot = act + sl * kDecActSlot + r * kDecRow + 16 * p;
            const uint8_t* sslot = asl + sl * kDecScaleSlot + r * 32 + p;
            v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < kMxSegSteps; j++) {
                if (j < ns) {
                    const v4i lo = *reinterpret_cast<const v4i*>(slot + 128 * j);
                    const v4i hi = *reinterpret_cast<const v4i*>(slot + 128 * j + 64);
                    const uint32_t sc = sslot[4 * j];
                    const v4i wi = {(int)wv[j].x, (int)wv[j].y, (int)wv[j].z, (int)wv[j].w};
                    acc = mx_mfma<0>(wi, v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w}, acc, wsc[j], sc);
                }
            }
            part[(sl * NTG + nt) * 64 + lane] = acc;
        }
        lds_barrier();
        if (w < NTG) {   // wave w folds tile w's segments of this round in order
            const int nr = min(SL, nseg - rd * SL);
            for (int i = 0; i < nr; i++) {
                const v4f z = part[(i * NTG + w) * 64 + lane];
                y = (rd == 0 && i == 0) ? z : v4f{add_rn(y.x, z.x), add_rn(y.y, z.y), add_rn(y.z, z.z), add_rn(y.w, z.w)};
            }
        }
        lds_barrier();
    }
    if (w < NTG && r < live) mx_store<EPI>(out, ldo, r, 16 * (blockIdx.x * NTG + w) + 4 * p, y);
}

// ---------------------------------------------------------------------------- decode kernel, segments split
// e4m3 activations, M <= 16, over a balanced grid.  The projection's work is its (1024-input segment s, 16-row
// weight tile t) units, u = s T + t (segment-major); W workgroups take equal contiguous ranges, so a workgroup's
// units mostly share one segment (at most two when a range is no longer than T), and it copies only those segments'
// 16 activation rows into LDS (1 KB row DMAs) where the tile-major staged kernel copies all of K per pair of tiles.
// One wave per unit: the segment's weights into registers, the same MFMA chain from zero as every kernel, its fp32
// segment sums to the workspace `part` [nseg][T][64] (v4f per lane); mx_split_fold_kernel, launched next on the
// stream, adds each tile's segment sums left to right, as every kernel does, and stores.  (The sums handed between
// workgroups inside one launch measured slower: they must pass the XCDs' L2s, through write-through stores or a
// cache write-back per hand-over.)  With one segment (K <= 1024) the split kernel stores the outputs itself.
constexpr int kMxSplitWG = 256;                  // workgroups (CUs)
constexpr int kMxSplitWaves = 16;                // waves per workgroup at most (more units loop)

template <int EPI>
__global__ __launch_bounds__(1024) void mx_decode_split_kernel(const uint8_t* __restrict__ aq,
                                                               const uint8_t* __restrict__ as,
                                                               const uint8_t* __restrict__ wq,
                                                               const uint8_t* __restrict__ ws,
                                                               void* __restrict__ out, int64_t ldo,
                                                               const int32_t* __restrict__ n_rows, int M, int K,
                                                               int T, v4f* __restrict__ part) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* act = lds;                                  // [2][16][kDecRow]
    uint8_t* asl = lds + 2 * kDecActSlot;                // [2][16][32]
    kernel_args_now(aq, as, wq, ws, out, ldo, n_rows, M, K, T, part);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, NWV = blockDim.x >> 6;
    const int W = gridDim.x, v = blockIdx.x;
    const int KS = K / kMxStep, nseg = (KS + kMxSegSteps - 1) / kMxSegSteps;
    const int64_t U = (int64_t)nseg * T;
    const int u0 = (int)(U * v / W), u1 = (int)(U * (v + 1) / W);
    const int sA = u0 / T, nsl = (u1 - 1) / T - sA + 1;  // segments of the range (1 or 2: ranges of at most T units)
    const int p = lane >> 4, r = lane & 15;

    v4u wr[kMxSegSteps];
    uint32_t wsc[kMxSegSteps];
    auto load = [&](int u) {
        const int s = u / T, t = u - s * T;
        const int s0 = s * kMxSegSteps;
#pragma unroll
        for (int j = 0; j < kMxSegSteps; j++) {
            const int st = min(s0 + j, KS - 1);
            wr[j] = reinterpret_cast<const v4u*>(wq)[((int64_t)t * KS + st) * 64 + lane];
            wsc[j] = ws[((int64_t)t * KS + st) * 64 + lane];
        }
    };
    int u = u0 + wv;
    if (u < u1) load(u);                               // the weight requests first
    // the range's activation segments: 16 rows x 1 KB each (one DMA per row), their scale bytes (16 rows x 32)
    for (int c = wv; c < 16 * nsl; c += NWV) {
        const int sl = c >> 4, row = c & 15;
        const int s0 = (sA + sl) * kMxSegSteps, ns = min(kMxSegSteps, KS - s0);
        // a short last segment: lanes past its end re-read its last 16 bytes (never used)
        const uint8_t* src = aq + (int64_t)min(row, M - 1) * K + (int64_t)s0 * kMxStep + min(16 * lane, ns * kMxStep - 16);
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(act + sl * kDecActSlot + row * kDecRow),
                                         16, 0, 0);
    }
    for (int c = wv; c < 2 * nsl; c += NWV) {          // lane L covers row 8 h + L / 8, bytes 4 (L % 8) .. + 3
        const int sl = c >> 1, h = c & 1;
        const int s0 = (sA + sl) * kMxSegSteps, ns = min(kMxSegSteps, KS - s0);
        const int row = 8 * h + (lane >> 3);
        const uint8_t* src = as + (int64_t)min(row, M - 1) * (K / 32) + s0 * 4 + min(4 * (lane & 7), 4 * ns - 4);
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(asl + sl * kDecScaleSlot + h * 256),
                                         4, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    for (; u < u1; u += NWV) {
        const int s = u / T, t = u - s * T;
        const int sl = s - sA, ns = min(kMxSegSteps, KS - s * kMxSegSteps);
        const uint8_t* slot = act + sl * kDecActSlot + r * kDecRow + 16 * p;
        const uint8_t* sslot = asl + sl * kDecScaleSlot + r * 32 + p;
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < kMxSegSteps; j++) {
            if (j < ns) {
                const v4i lo = *reinterpret_cast<const v4i*>(slot + 128 * j);
                const v4i hi = *reinterpret_cast<const v4i*>(slot + 128 * j + 64);
                const uint32_t sc = sslot[4 * j];
                const v4i wi = {(int)wr[j].x, (int)wr[j].y, (int)wr[j].z, (int)wr[j].w};
                acc = mx_mfma<0>(wi, v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w}, acc, wsc[j], sc);
            }
        }
        if (u + NWV < u1) load(u + NWV);
        if (nseg > 1) {
            part[((int64_t)s * T + t) * 64 + lane] = acc;
        } else {
            const int live = n_rows ? min(M, __ldg(n_rows)) : M;
            if (r < live) mx_store<EPI>(out, ldo, r, 16 * t + 4 * p, acc);
        }
    }
}

// The split decode's second launch: one wave per 16-row tile adds its nseg segment sums left to right and stores.
template <int EPI>
__global__ __launch_bounds__(256) void mx_split_fold_kernel(const v4f* __restrict__ part, void* __restrict__ out,
                                                           int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                           int T, int nseg) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    v4f y = part[(int64_t)t * 64 + lane];
    for (int i0 = 1; i0 < nseg; i0 += 4) {
        v4f z[4];                                        // four segments' sums in flight at once
#pragma unroll
        for (int i = 0; i < 4; i++) z[i] = part[((int64_t)min(i0 + i, nseg - 1) * T + t) * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (i0 + i < nseg) y = v4f{add_rn(y.x, z[i].x), add_rn(y.y, z[i].y), add_rn(y.z, z[i].z), add_rn(y.w, z[i].w)};
    }
    const int live = n_rows ? min(M, __ldg(n_rows)) : M;
    const int p = lane >> 4, r = lane & 15;
    if (r < live) mx_store<EPI>(out, ldo, r, 16 * t + 4 * p, y);
}

int64_t mx_split_workspace_bytes(int64_t N, int64_t K) {     // 1 KB of segment sums per unit
    const int64_t T = N / 16, nseg = (K / kMxStep + kMxSegSteps - 1) / kMxSegSteps;
    return nseg > 1 ? nseg * T * 1024 : 16;
}

static size_t mx_decode_lds(int MT, int K) {
    const int nseg = (K / kMxStep + kMxSegSteps - 1) / kMxSegSteps;
    return (size_t)nseg * MT * 64 * sizeof(v4f);
}

}  // namespace prism

using namespace prism;

extern "C" int prism_mxfp4_pack(const float* w, int64_t ldw, uint8_t* q, uint8_t* s, int64_t N, int64_t K, int mode,
                                void* stream) {
    if (!w || !q || !s) return PRISM_ERR_ARG;
    if (N <= 0 || K <= 0 || N % 16 || K % kMxStep || ldw < K || ldw % 4 || N / 16 > 65535 || K / kMxStep > (1 << 30))
        return PRISM_ERR_SHAPE;
    if (mode < 0 || mode > 2) return PRISM_ERR_ARG;
    if (!PRISM_ALIGNED(w, 16) || !PRISM_ALIGNED(q, 16)) return PRISM_ERR_ALIGN;
    dim3 grid((unsigned)(K / kMxStep), (unsigned)(N / 16));
    hipStream_t st = (hipStream_t)stream;
    if (mode == 0) hipLaunchKernelGGL(mx_pack_kernel<0>, grid, dim3(64), 0, st, w, ldw, q, s, (int)K);
    else if (mode == 1) hipLaunchKernelGGL(mx_pack_kernel<1>, grid, dim3(64), 0, st, w, ldw, q, s, (int)K);
    else hipLaunchKernelGGL(mx_pack_kernel<2>, grid, dim3(64), 0, st, w, ldw, q, s, (int)K);
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_mxfp4_repack(const uint8_t* q_rows, const uint8_t* s_rows, uint8_t* q, uint8_t* s, int64_t N,
                                  int64_t K, void* stream) {
    if (!q_rows || !s_rows || !q || !s) return PRISM_ERR_ARG;
    if (N <= 0 || K <= 0 || N % 16 || K % kMxStep || N / 16 > 65535) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(q_rows, 16) || !PRISM_ALIGNED(q, 16)) return PRISM_ERR_ALIGN;
    dim3 grid((unsigned)(K / kMxStep), (unsigned)(N / 16));
    hipLaunchKernelGGL(mx_repack_kernel, grid, dim3(64), 0, (hipStream_t)stream, q_rows, s_rows, q, s, (int)K);
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_mxfp4_quant_act(const void* x, int x_f32, int64_t ldx, const float* inv, uint8_t* q, uint8_t* s,
                                     const int32_t* n_rows, int64_t M, int64_t K, int fmt, void* stream) {
    if (!x || !q || !s) return PRISM_ERR_ARG;
    if (fmt != PRISM_MX_E4M3 && fmt != PRISM_MX_E2M1 && fmt != PRISM_MX_E4M3_PANELS) return PRISM_ERR_ARG;
    if (M < 0 || K <= 0 || K % 32 || ldx < K || M > 65535) return PRISM_ERR_SHAPE;
    if (fmt == PRISM_MX_E4M3_PANELS && K % kMxStep) return PRISM_ERR_SHAPE;
    if ((x_f32 ? ldx % 4 : ldx % 8) || !PRISM_ALIGNED(x, 16) || !PRISM_ALIGNED(q, 16) ||
        (inv && !PRISM_ALIGNED(inv, 16)))
        return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    dim3 grid((unsigned)((K / 32 + 255) / 256), (unsigned)M);
    hipStream_t st = (hipStream_t)stream;
#define QA(AF, F) hipLaunchKernelGGL((mx_quant_act_kernel<AF, F>), grid, dim3(256), 0, st, x, ldx, inv, q, s, n_rows, \
                                     (int)M, (int)K)
    if (fmt == PRISM_MX_E4M3_PANELS) {
        if (x_f32) hipLaunchKernelGGL((mx_quant_act_kernel<0, true, true>), grid, dim3(256), 0, st, x, ldx, inv, q, s,
                                      n_rows, (int)M, (int)K);
        else hipLaunchKernelGGL((mx_quant_act_kernel<0, false, true>), grid, dim3(256), 0, st, x, ldx, inv, q, s,
                                n_rows, (int)M, (int)K);
    } else if (fmt == PRISM_MX_E4M3) { if (x_f32) QA(0, true); else QA(0, false); }
    else { if (x_f32) QA(4, true); else QA(4, false); }
#undef QA
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_mxfp4_gemm_ws(const uint8_t* aq, const uint8_t* as, int a_fmt, const uint8_t* wq,
                                   const uint8_t* ws, void* out, int64_t ldo, const int32_t* n_rows, int64_t M,
                                   int64_t N, int64_t K, int epi, int kernel, void* work, int64_t work_bytes,
                                   void* stream) {
    if (!aq || !as || !wq || !ws || !out) return PRISM_ERR_ARG;
    if (a_fmt != PRISM_MX_E4M3 && a_fmt != PRISM_MX_E2M1 && a_fmt != PRISM_MX_E4M3_PANELS) return PRISM_ERR_ARG;
    if (epi != 0 && epi != 1) return PRISM_ERR_ARG;
    if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % kMxStep || ldo < N || M > (1 << 24) || N / 16 > (1 << 24))
        return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(aq, 16) || !PRISM_ALIGNED(wq, 16) || ldo % 4 || !PRISM_ALIGNED(out, epi ? 16 : 8))
        return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    const int MT = (int)((M + 15) / 16);
    if (a_fmt == PRISM_MX_E4M3_PANELS) {                 // the direct-weight tile kernel only
        if (kernel == 1 || kernel == 2 || (int64_t)N * K / 2 >= (1LL << 31)) return PRISM_ERR_SHAPE;
        kernel = 0;
    }
    // the split decode: one 16-row block of e4m3 rows, its workspace, ranges of at most T units (two segments)
    const int64_t T = N / 16, nseg = (K / kMxStep + kMxSegSteps - 1) / kMxSegSteps, U = nseg * T;
    const int64_t need = mx_split_workspace_bytes(N, K);
    const bool split_ok = MT == 1 && a_fmt == PRISM_MX_E4M3 && work && need > 0 && work_bytes >= need &&
                          PRISM_ALIGNED(work, 16) && (U + kMxSplitWG - 1) / kMxSplitWG <= T && U < (1 << 30);
    if (kernel == 2 && !split_ok) return !work ? PRISM_ERR_ARG : !PRISM_ALIGNED(work, 16) ? PRISM_ERR_ALIGN : PRISM_ERR_SHAPE;
    // measured against the staged decode at 1-16 rows: 15.8-16.0 against 17.3-18.8 us at 17408 x 5120, 16.9
    // against 18.2-20.6 at 5120 x 17408, 21.5-21.7 against 23.5-25.6 at 27648 x 5120; slower below about 80 M weights
    // (its second launch costs about 2.5 us: 8.5 against 6.7-7.3 us at 5120^2, 14.0 against 11.4 at 8192^2)
    if (kernel < 0 && split_ok && N * K >= (80LL << 20)) kernel = 2;
    if (kernel < 0) kernel = (MT <= 4 && mx_decode_lds(MT, (int)K) <= 64 * 1024) ? 1 : 0;
    if (kernel == 2) {
        const int W = (int)std::min<int64_t>(kMxSplitWG, U);
        const int nw = (int)std::min<int64_t>(kMxSplitWaves, (U + W - 1) / W);
        const size_t lds = 2 * (size_t)(kDecActSlot + kDecScaleSlot);
        auto* part = static_cast<v4f*>(work);
#define DSP(E)                                                                                                       \
    do {                                                                                                             \
        hipLaunchKernelGGL((mx_decode_split_kernel<E>), dim3(W), dim3(64 * nw), lds, st, aq, as, wq, ws, out, ldo,   \
                           n_rows, (int)M, (int)K, (int)T, part);                                                    \
        if (nseg > 1)                                                                                                \
            hipLaunchKernelGGL((mx_split_fold_kernel<E>), dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, part, out, \
                               ldo, n_rows, (int)M, (int)T, (int)nseg);                                              \
    } while (0)
        if (epi) DSP(1); else DSP(0);
#undef DSP
    } else if (kernel == 1 && MT == 1 && a_fmt == PRISM_MX_E4M3) {
        const int nseg = (int)((K / kMxStep + kMxSegSteps - 1) / kMxSegSteps);
        const int ntg = (N % 32 == 0) ? 2 : 1;     // two weight tiles share each staged activation copy
        const int sl = min(nseg, 8);        // 8 segment lanes: 154 KB of LDS at NTG 2
        const size_t lds = mx_decode_staged_lds(ntg, sl);
        dim3 grid((unsigned)(N / (16 * ntg)));
#define DST(NTGV, E)                                                                                                 \
    do {                                                                                                             \
        allow_lds(mx_decode_staged_kernel<NTGV, E>, lds);                                                            \
        hipLaunchKernelGGL((mx_decode_staged_kernel<NTGV, E>), grid, dim3(64 * NTGV * sl), lds, st, aq, as, wq, ws,  \
                           out, ldo, n_rows, (int)M, (int)K, sl);                                                    \
    } while (0)
        if (ntg == 2) { if (epi) DST(2, 1); else DST(2, 0); }
        else { if (epi) DST(1, 1); else DST(1, 0); }
#undef DST
    } else if (kernel == 1) {
        if (MT > 4) return PRISM_ERR_SHAPE;
        const size_t lds = mx_decode_lds(MT, (int)K);
        if (lds > 160 * 1024) return PRISM_ERR_SHAPE;
        const int nseg = (int)((K / kMxStep + kMxSegSteps - 1) / kMxSegSteps);
        const int nw = min(nseg, MT == 1 ? 16 : 8);
        dim3 grid((unsigned)(N / 16));
#define DEC(MTV, AF, E)                                                                                              \
    do {                                                                                                             \
        allow_lds(mx_decode_kernel<MTV, AF, E>, lds);                                                                \
        hipLaunchKernelGGL((mx_decode_kernel<MTV, AF, E>), grid, dim3(64 * nw), lds, st, aq, as, wq, ws, out, ldo,   \
                           n_rows, (int)M, (int)K);                                                                  \
    } while (0)
#define DEC_MT(AF, E)                                                                                                \
    do {                                                                                                             \
        if (MT == 1) DEC(1, AF, E); else if (MT == 2) DEC(2, AF, E); else if (MT == 3) DEC(3, AF, E);                \
        else DEC(4, AF, E);                                                                                          \
    } while (0)
        if (a_fmt == PRISM_MX_E4M3) { if (epi) DEC_MT(0, 1); else DEC_MT(0, 0); }
        else { if (epi) DEC_MT(4, 1); else DEC_MT(4, 0); }
#undef DEC_MT
#undef DEC
    } else {
        // tile configuration: LDS stages, waves along M, waves along N, 16-row activation tiles per wave
#ifndef MXV_TILE
#define MXV_TILE 2, 1, 4, 4
#endif
#define MXT_(NS, WM, WN, AR) constexpr int kNS = NS, kWM = WM, kWN = WN, kAR = AR;
#define MXT(...) MXT_(__VA_ARGS__)
        MXT(MXV_TILE)
#undef MXT
#undef MXT_
        const int tiles_m = (int)((M + 16 * kAR * kWM - 1) / (16 * kAR * kWM)), tiles_n = (int)((N + 64 * kWN - 1) / (64 * kWN));
        dim3 grid((unsigned)(tiles_m * tiles_n));
#ifndef MX_WD
#define MX_WD 1
#endif
        if (MX_WD && N * K / 2 < (1LL << 31)) {            // the direct-weight form of the 64 x 256 tile
            constexpr int WT = MX_WD == 2 ? 8 : 4;           // weight tiles per wave
            const int tm = (int)((M + 63) / 64), tn = (int)((N + 64 * WT - 1) / (64 * WT));
#define TWD(AF, E, PN)                                                                                               \
    hipLaunchKernelGGL((mx_tile_wd_kernel<AF, E, WT, PN>), dim3((unsigned)(tm * tn)), dim3(256), 0, st, aq, as, wq,  \
                       ws, out, ldo, n_rows, (int)M, (int)N, (int)K, tm, tn)
            if (a_fmt == PRISM_MX_E4M3_PANELS) { if (epi) TWD(0, 1, true); else TWD(0, 0, true); }
            else if (a_fmt == PRISM_MX_E4M3) { if (epi) TWD(0, 1, false); else TWD(0, 0, false); }
            else { if (epi) TWD(4, 1, false); else TWD(4, 0, false); }
#undef TWD
            PRISM_LAUNCH_CHECK();
            return PRISM_OK;
        }
#define TILE(AF, E)                                                                                                  \
    do {                                                                                                             \
        const size_t lds = (size_t)kNS * MxStage<AF, kWM, kWN, kAR>::BYTES;                                          \
        allow_lds(mx_tile_kernel<AF, E, kNS, kWM, kWN, kAR>, lds);                                                   \
        hipLaunchKernelGGL((mx_tile_kernel<AF, E, kNS, kWM, kWN, kAR>), grid, dim3(64 * kWM * kWN), lds, st, aq, as, wq,  \
                           ws, out, ldo, n_rows, (int)M, (int)N, (int)K, tiles_m, tiles_n);                          \
    } while (0)
        if (a_fmt == PRISM_MX_E4M3) { if (epi) TILE(0, 1); else TILE(0, 0); }
        else { if (epi) TILE(4, 1); else TILE(4, 0); }
#undef TILE
    }
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_mxfp4_gemm(const uint8_t* aq, const uint8_t* as, int a_fmt, const uint8_t* wq,
                                const uint8_t* ws, void* out, int64_t ldo, const int32_t* n_rows, int64_t M,
                                int64_t N, int64_t K, int epi, int kernel, void* stream) {
    return prism_mxfp4_gemm_ws(aq, as, a_fmt, wq, ws, out, ldo, n_rows, M, N, K, epi, kernel, nullptr, 0, stream);
}

extern "C" int64_t prism_mxfp4_split_workspace_bytes(int64_t N, int64_t K) {
    if (N <= 0 || K <= 0 || N % 16 || K % kMxStep) return 0;
    return mx_split_workspace_bytes(N, K);
}
