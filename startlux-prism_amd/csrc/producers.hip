// Fused activation producers (gfx950): the kernels that sit between the engine's GEMMs and write their int8 inputs.
// Restates kernels/quant.py (StartLux-Prism):
//   norm_q8    :144-170, :418-431   y = rmsnorm(h) * w          -> int8 rows, one scale per row
//   swiglu_q8  :249-280, :472-478   y = silu(gate) * up * inv_s -> int8 rows, one scale per row
//   norm_g     :354-366, :395-397   y = rmsnorm(h) * w          -> W4A8 operands (_store_g, :314-330)
//   swiglu_g   :384-393, :403-406   y = silu(gate) * up         -> W4A8 operands
//   gated_norm_q8 :216-246, :460-469, gated_norm_g :349-365, :399-401
//                                   y = rmsnorm_head(o) * w * silu(z) (* inv_s) -> either back end
// One workgroup per row (256 threads; the SwiGLU and gated-norm kernels take 1024 for up to 64 rows, the decode sizes,
// which their results do not depend on); thread t owns the 8-input chunks t, t + TPB, ... and keeps them in registers
// between the row reductions and the stores, so a row is read once.
//
// Arithmetic (every step an IEEE fp32 operation, so the CPU oracle reproduces the bits):
//   rmsnorm: ss = sum of RN(h * h) in a fixed order - each thread adds its own inputs in increasing index, the 64
//            lanes of a wave combine by halving (lane l + lane l + 32, then + 16, ...), the four waves left to right;
//            r = RN(1 / RN(sqrt(RN(RN(ss / HID) + eps)))); y = RN(RN(h * r) * w).
//   gated:   per head of D values, ss = the chunk sums (8 values each, increasing index) combined by halving across
//            the D / 8 neighbouring lanes that hold the head (lane l + lane l ^ D/16, then ^ D/32, ...);
//            y = RN(RN(RN(o * r) * w[d]) * silu(z)), then RN(y * inv_s) for the q8 form.
//   silu:    RN(g / RN(1 + exp(-g))), with exp this library's own (prism_expf below).
//   quantization as the row quantizers: scale = RN(max(amax, 1e-10) / 127), q = rint(RN(y / scale)).
// The reference evaluates rsqrt, exp and '/' with NVIDIA's approximate instructions and sums in Triton's reduction
// order, neither of which has a specification; these kernels define the operations exactly instead.
#include <type_traits>

#include "common.h"

namespace prism {

constexpr int kPThreads = 256;

// e^x in fp32: x = n ln2 + r with n = rint(x log2 e) and r reduced by the two-constant method of Cody and Waite
// (ln2 = LN2_HI + LN2_LO, LN2_HI with 9 trailing zero bits so n LN2_HI is exact for |n| < 2^9), e^r by its Taylor
// series to degree 7 evaluated with fmas (|r| <= 0.3466: truncation below 2^-27 relative), then scaled by 2^n.
__device__ __forceinline__ float prism_expf(float x) {
    if (x > 88.72283935546875f) return __uint_as_float(0x7f800000u);
    if (x < -103.97208404541016f) return 0.f;
    const float n = rintf(mul_rn(x, 1.44269502162933349609375f));
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.428606765330187045e-06f, r);
    float p = 1.98412701e-04f;                  // 1/5040
    p = fmaf(p, r, 1.38888892e-03f);            // 1/720
    p = fmaf(p, r, 8.33333377e-03f);            // 1/120
    p = fmaf(p, r, 4.16666679e-02f);            // 1/24
    p = fmaf(p, r, 1.66666672e-01f);            // 1/6
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

__device__ __forceinline__ float silu_rn(float g) { return div_rn(g, add_rn(1.0f, prism_expf(-g))); }

__device__ __forceinline__ uint32_t pack4_i8(const float* f) {
    uint32_t r = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) r |= ((uint32_t)(int)f[j] & 0xffu) << (8 * j);
    return r;
}

// Row reductions over the workgroup: the maximum (exact in any order, so for any workgroup size TPB) and the
// fixed-order sum of the module comment (256 threads).
template <int TPB>
__device__ __forceinline__ float row_max(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < TPB / 64; i++) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float row_sum_fixed(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = add_rn(v, __shfl_xor(v, o, kWave));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = add_rn(add_rn(add_rn(red[0], red[1]), red[2]), red[3]);
    __syncthreads();
    return r;
}

// Back ends.  BACK 0: int8 row + one scale per row (q [M, K], s [M]).  BACK 1: the W4A8 operands with one scale
// per 256 inputs (xq [M, K], a [K/256, M], xs [K/256, M, 16]); BACK 2: the same with one scale per row (a [M]).
// TPB: the workgroup size (thread t owns chunks t, t + TPB, ...); every result is independent of it.
// live: the row is below n_rows (the workgroup computes either way and stores only then: reading n_rows before the
// row's loads would hold them back by a memory round trip).
template <int NCH, int BACK, int TPB = kPThreads>
__device__ __forceinline__ void store_back(float (&y)[NCH][8], float rmax, float* red, int64_t row, int out_row,
                                           int M, int K, int8_t* __restrict__ q, float* __restrict__ s,
                                           int8_t* __restrict__ xs, bool live) {
    const int nch = K / 8;
    if (BACK == 0 || BACK == 2) rmax = row_max<TPB>(rmax, red);
    if (!live) return;                       // uniform over the workgroup, after its last barrier
    v2u* qr = reinterpret_cast<v2u*>(q + (int64_t)out_row * K);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * TPB;
        float gmax = rmax;
        if (BACK == 1) {                     // the 32 chunks of a group of 256 are the lanes of a half-wave
            float m = 0.f;
            if (idx < nch) {
#pragma unroll
                for (int j = 0; j < 8; j++) m = fmaxf(m, fabsf(y[c][j]));
            }
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
            gmax = m;
        }
        const float scale = div_rn(fmaxf(gmax, 1e-10f), 127.0f), rs = div_rn(1.0f, scale);
        int sum = 0;
        if (idx < nch) {
            float r[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                r[j] = quant_rint(y[c][j], scale, rs);
                sum += (int)r[j];
            }
            qr[idx] = v2u{pack4_i8(r), pack4_i8(r + 4)};
        }
        if (BACK != 0) {
            sum = wave_sum_width(sum, 4);    // the 4 chunks of a sub-block of 32 are neighbouring lanes
            if (idx < nch) {
                const int b = idx / 32, j = (idx % 32) / 4;
                if ((idx % 4) == 0) {
                    int8_t* p = xs + ((int64_t)b * M + out_row) * 16;
                    p[j] = (int8_t)(sum & 63);
                    p[8 + j] = (int8_t)(sum >> 6);
                }
                if (BACK == 1 && (idx % 32) == 0) s[(int64_t)b * M + out_row] = scale;
            }
        }
    }
    if (threadIdx.x == 0) {
        if (BACK == 0) s[out_row] = div_rn(fmaxf(rmax, 1e-10f), 127.0f);
        if (BACK == 2) s[out_row] = div_rn(fmaxf(rmax, 1e-10f), 127.0f);
    }
    (void)row;
}

// ---------------------------------------------------------------------------------------------- deferred fold
// A residual add deferred by a split-K per-channel projection (prism_w8a8_pc_packed_gemm_split): the np int32 slots'
// sums of 8 inputs of row r from column c, tot = slot 0 + slot 1 + ... (exact), then h = RN(h + RN(RN(float(tot) sa)
// sw)) with sa = psa[r psa_sm] and sw = psw[c .. c + 7] (fp32, or fp16 when PSW16): the epilogue 1 of the unsplit
// projection, so the residual gets the same bits whichever way the projection ran (kernels/quant.py:129-141).
struct Fold {
    const int32_t* parts;
    int64_t part_stride, ldp;
    int np;
    const float* psa;
    int64_t psa_sm;
    const void* psw;
    int psw16;
};

__device__ __forceinline__ void fold8(float* hv, const Fold& f, int64_t r, int c) {
    int tot[8];
    const int32_t* p0 = f.parts + r * f.ldp + c;
    {
        const v4i a = *reinterpret_cast<const v4i*>(p0), b = *reinterpret_cast<const v4i*>(p0 + 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            tot[j] = a[j];
            tot[j + 4] = b[j];
        }
    }
    for (int p = 1; p < f.np; p++) {
        const int32_t* pp = p0 + p * f.part_stride;
        const v4i a = *reinterpret_cast<const v4i*>(pp), b = *reinterpret_cast<const v4i*>(pp + 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            tot[j] += a[j];
            tot[j + 4] += b[j];
        }
    }
    const float sa = f.psa[r * f.psa_sm];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float sw = f.psw16 ? f16_to_f32(static_cast<const uint16_t*>(f.psw)[c + j])
                                 : static_cast<const float*>(f.psw)[c + j];
        hv[j] = add_rn(hv[j], mul_rn(mul_rn((float)tot[j], sa), sw));
    }
}

// h fp32 [*, HID] (row stride ldh): one thread per 8 values of a live row.
__global__ __launch_bounds__(256) void fold_parts_kernel(float* __restrict__ h, int64_t ldh, Fold f,
                                                         const int32_t* __restrict__ n_rows, int HID) {
    const int64_t r = blockIdx.y;
    const int c = 8 * (blockIdx.x * 256 + threadIdx.x);
    if (r >= __ldg(n_rows) || c >= HID) return;
    v4f* hp = reinterpret_cast<v4f*>(h + r * ldh + c);
    const v4f a = hp[0], b = hp[1];
    float hv[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    fold8(hv, f, r, c);
    hp[0] = v4f{hv[0], hv[1], hv[2], hv[3]};
    hp[1] = v4f{hv[4], hv[5], hv[6], hv[7]};
}

// ---------------------------------------------------------------------------------------------- rmsnorm
// h fp32 [*, HID] (row stride ldh), w fp32 [HID]; output row i from input row rows[i] when rows is not null.  FOLD:
// first finish a deferred residual add in the row (fold8) and store the row back to h.
template <int NCH, int BACK, bool FOLD = false>
__global__ __launch_bounds__(kPThreads) void norm_prod_kernel(float* __restrict__ h, int64_t ldh,
                                                              const float* __restrict__ w,
                                                              const int32_t* __restrict__ rows, int8_t* __restrict__ q,
                                                              float* __restrict__ s, int8_t* __restrict__ xs,
                                                              const int32_t* __restrict__ n_rows, int M, int HID,
                                                              float eps, Fold f) {
    __shared__ float red[4];
    kernel_args_now(h, ldh, w, rows, q, s, xs, n_rows, M, HID, eps);
    const int i = blockIdx.x;
    // a gathered row's index is only meaningful below n_rows: that path tests the count first (a dependent load
    // follows anyway); without a gather every row index below M is a valid address and the count is read later
    if (rows && i >= __ldg(n_rows)) return;
    const int64_t src = rows ? (int64_t)__ldg(rows + i) : i;
    const int nch = HID / 8;
    v4f* hr = reinterpret_cast<v4f*>(h + src * ldh);
    const v4f* wr = reinterpret_cast<const v4f*>(w);
    float y[NCH][8];
    float ss = 0.f;
    // the row's and the weights' loads first, all of them, unconditionally (chunk indices clamped into the row): a
    // load inside a per-chunk branch would wait before the next chunk's went out
    v4f ha[NCH], hb[NCH], wa[NCH], wb[NCH];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = min((int)threadIdx.x + c * kPThreads, nch - 1);
        ha[c] = __builtin_nontemporal_load(hr + 2 * idx);
        hb[c] = __builtin_nontemporal_load(hr + 2 * idx + 1);
    }
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = min((int)threadIdx.x + c * kPThreads, nch - 1);
        wa[c] = wr[2 * idx];
        wb[c] = wr[2 * idx + 1];
    }
    const bool live = i < __ldg(n_rows);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * kPThreads;
        if (idx < nch) {
            const v4f a = ha[c], b = hb[c];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                y[c][j] = a[j];
                y[c][j + 4] = b[j];
            }
            if (FOLD && live) {
                fold8(y[c], f, src, 8 * idx);
                hr[2 * idx] = v4f{y[c][0], y[c][1], y[c][2], y[c][3]};
                hr[2 * idx + 1] = v4f{y[c][4], y[c][5], y[c][6], y[c][7]};
            }
#pragma unroll
            for (int j = 0; j < 8; j++) ss = add_rn(ss, mul_rn(y[c][j], y[c][j]));
        }
    }
    ss = row_sum_fixed(ss, red);
    const float r = div_rn(1.0f, sqrt_rn(add_rn(div_rn(ss, (float)HID), eps)));
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * kPThreads;
        if (idx < nch) {
            const v4f a = wa[c], b = wb[c];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                y[c][j] = mul_rn(mul_rn(y[c][j], r), a[j]);
                y[c][j + 4] = mul_rn(mul_rn(y[c][j + 4], r), b[j]);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(y[c][j]));
        }
    }
    store_back<NCH, BACK>(y, amax, red, src, i, M, HID, q, s, xs, live);
}

// ---------------------------------------------------------------------------------------------- SwiGLU
// gu [*, 2 FF] (bf16, or fp32 when GU32; row stride ldg): gate = columns 0 .. FF-1, up = FF .. 2 FF - 1; inv_s fp32
// [FF] or null.
template <int NCH, int BACK, bool GU32, int TPB>
__global__ __launch_bounds__(TPB) void swiglu_prod_kernel(const void* __restrict__ gu, int64_t ldg,
                                                                const float* __restrict__ inv_s,
                                                                int8_t* __restrict__ q, float* __restrict__ s,
                                                                int8_t* __restrict__ xs,
                                                                const int32_t* __restrict__ n_rows, int M, int FF) {
    __shared__ float red[TPB / 64];
    kernel_args_now(gu, ldg, inv_s, q, s, xs, n_rows, M, FF);
    const int i = blockIdx.x;
    const int nch = FF / 8;
    float y[NCH][8];
    float amax = 0.f;
    // every load first, unconditionally (chunk indices clamped into the row; see norm_prod_kernel)
    v4u raw[NCH][4];
    v4f isv[NCH][2];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = min((int)threadIdx.x + c * TPB, nch - 1);
        if (GU32) {
            const v4u* row = reinterpret_cast<const v4u*>(static_cast<const float*>(gu) + (int64_t)i * ldg);
            raw[c][0] = row[2 * idx];
            raw[c][1] = row[2 * idx + 1];
            raw[c][2] = row[FF / 4 + 2 * idx];
            raw[c][3] = row[FF / 4 + 2 * idx + 1];
        } else {
            const v4u* row = reinterpret_cast<const v4u*>(static_cast<const uint16_t*>(gu) + (int64_t)i * ldg);
            raw[c][0] = row[idx];
            raw[c][1] = row[FF / 8 + idx];
        }
        if (inv_s) {
            isv[c][0] = reinterpret_cast<const v4f*>(inv_s)[2 * idx];
            isv[c][1] = reinterpret_cast<const v4f*>(inv_s)[2 * idx + 1];
        }
    }
    const bool live = i < __ldg(n_rows);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * TPB;
        if (idx < nch) {
            float g[8], u[8];
            if (GU32) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    g[j] = __uint_as_float(raw[c][0][j]); g[j + 4] = __uint_as_float(raw[c][1][j]);
                    u[j] = __uint_as_float(raw[c][2][j]);
                    u[j + 4] = __uint_as_float(raw[c][3][j]);
                }
            } else {
                const v4u gv = raw[c][0], uv = raw[c][1];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    g[2 * j] = __uint_as_float(gv[j] << 16);
                    g[2 * j + 1] = __uint_as_float(gv[j] & 0xffff0000u);
                    u[2 * j] = __uint_as_float(uv[j] << 16);
                    u[2 * j + 1] = __uint_as_float(uv[j] & 0xffff0000u);
                }
            }
            float is[8];
            if (inv_s) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    is[j] = isv[c][0][j];
                    is[j + 4] = isv[c][1][j];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                float v = mul_rn(silu_rn(g[j]), u[j]);
                if (inv_s) v = mul_rn(v, is[j]);
                y[c][j] = v;
                amax = fmaxf(amax, fabsf(v));
            }
        }
    }
    store_back<NCH, BACK, TPB>(y, amax, red, i, i, M, FF, q, s, xs, live);
}

// ---------------------------------------------------------------------------------------------- gated RMSNorm
// o fp32 [*, HV D] (row stride ldo); z [*, ldz] (bf16, or fp32 when Z32): the row's gate values from column 0 (the
// caller offsets the projection's row); w fp32 [D]; inv_s fp32 [HV D] or null.  D / 8 is a power of two <= 64, so
// a head's chunks are neighbouring lanes of one wave.
template <int NCH, int BACK, bool Z32, int TPB>
__global__ __launch_bounds__(TPB) void gated_norm_prod_kernel(const float* __restrict__ o, int64_t ldo,
                                                                    const void* __restrict__ z, int64_t ldz,
                                                                    const float* __restrict__ w,
                                                                    const float* __restrict__ inv_s,
                                                                    int8_t* __restrict__ q, float* __restrict__ s,
                                                                    int8_t* __restrict__ xs,
                                                                    const int32_t* __restrict__ n_rows, int M, int HV,
                                                                    int D, float eps) {
    __shared__ float red[TPB / 64];
    kernel_args_now(o, ldo, z, ldz, w, inv_s, q, s, xs, n_rows, M, HV, D, eps);
    const int i = blockIdx.x;
    const int K = HV * D, nch = K / 8, cph = D / 8;
    const v4f* orow = reinterpret_cast<const v4f*>(o + (int64_t)i * ldo);
    float y[NCH][8];
    float amax = 0.f;
    // every load first, unconditionally (chunk indices clamped into the row; see norm_prod_kernel)
    v4f oa[NCH], ob[NCH], wv0[NCH], wv1[NCH], iv0[NCH], iv1[NCH];
    v4u zv[NCH][2];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = min((int)threadIdx.x + c * TPB, nch - 1);
        oa[c] = __builtin_nontemporal_load(orow + 2 * idx);
        ob[c] = __builtin_nontemporal_load(orow + 2 * idx + 1);
        const int d0 = (idx & (cph - 1)) * 8;
        wv0[c] = reinterpret_cast<const v4f*>(w + d0)[0];
        wv1[c] = reinterpret_cast<const v4f*>(w + d0)[1];
        if (Z32) {
            const v4u* zr = reinterpret_cast<const v4u*>(static_cast<const float*>(z) + (int64_t)i * ldz);
            zv[c][0] = zr[2 * idx];
            zv[c][1] = zr[2 * idx + 1];
        } else {
            zv[c][0] = reinterpret_cast<const v4u*>(static_cast<const uint16_t*>(z) + (int64_t)i * ldz)[idx];
        }
        if (inv_s) {
            iv0[c] = reinterpret_cast<const v4f*>(inv_s)[2 * idx];
            iv1[c] = reinterpret_cast<const v4f*>(inv_s)[2 * idx + 1];
        }
    }
    const bool live = i < __ldg(n_rows);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int idx = threadIdx.x + c * TPB;
        const bool in = idx < nch;
        float ss = 0.f;
        if (in) {
            const v4f a = oa[c], b = ob[c];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                y[c][j] = a[j];
                y[c][j + 4] = b[j];
            }
#pragma unroll
            for (int j = 0; j < 8; j++) ss = add_rn(ss, mul_rn(y[c][j], y[c][j]));
        }
        for (int off = cph >> 1; off > 0; off >>= 1) ss = add_rn(ss, __shfl_xor(ss, off, kWave));
        if (in) {
            const float r = div_rn(1.0f, sqrt_rn(add_rn(div_rn(ss, (float)D), eps)));
            const v4f w0 = wv0[c], w1 = wv1[c];
            float g[8];
            if (Z32) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    g[j] = __uint_as_float(zv[c][0][j]);
                    g[j + 4] = __uint_as_float(zv[c][1][j]);
                }
            } else {
                const v4u gv = zv[c][0];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    g[2 * j] = __uint_as_float(gv[j] << 16);
                    g[2 * j + 1] = __uint_as_float(gv[j] & 0xffff0000u);
                }
            }
            float is[8];
            if (inv_s) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    is[j] = iv0[c][j];
                    is[j + 4] = iv1[c][j];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float wj = j < 4 ? w0[j] : w1[j - 4];
                float v = mul_rn(mul_rn(mul_rn(y[c][j], r), wj), silu_rn(g[j]));
                if (inv_s) v = mul_rn(v, is[j]);
                y[c][j] = v;
                amax = fmaxf(amax, fabsf(v));
            }
        }
    }
    store_back<NCH, BACK, TPB>(y, amax, red, i, i, M, K, q, s, xs, live);
}

template <typename KN>
static int pick_nch(int K, KN&& launch, int tpb = kPThreads) {
    const int need = (K / 8 + tpb - 1) / tpb;
    if (need <= 1) return launch(std::integral_constant<int, 1>{});
    if (need <= 2) return launch(std::integral_constant<int, 2>{});
    if (need <= 3) return launch(std::integral_constant<int, 3>{});
    if (need <= 4) return launch(std::integral_constant<int, 4>{});
    if (need <= 6) return launch(std::integral_constant<int, 6>{});
    if (need <= 9) return launch(std::integral_constant<int, 9>{});
    if (need <= 12) return launch(std::integral_constant<int, 12>{});
    return launch(std::integral_constant<int, 16>{});
}

}  // namespace prism

using namespace prism;

static int norm_launch(float* h, int64_t ldh, const float* w, const int32_t* rows, int8_t* q, float* s, int8_t* xs,
                       const int32_t* n_rows, int64_t M, int64_t HID, float eps, int back, const Fold& f,
                       hipStream_t st) {
    if (!h || !w || !q || !s || !n_rows || (back != 0 && !xs)) return PRISM_ERR_ARG;
    if (back < 0 || back > 2) return PRISM_ERR_ARG;
    if (M < 0 || HID <= 0 || HID % 8 || ldh < HID || ldh % 8 || HID > 32768 || M > (1 << 30)) return PRISM_ERR_SHAPE;
    if (back != 0 && HID % 256) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(h, 16) || !PRISM_ALIGNED(w, 16) || !PRISM_ALIGNED(q, 8)) return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    const bool fold = f.np > 0;
    return pick_nch((int)HID, [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
#define NQ(B, F) hipLaunchKernelGGL((norm_prod_kernel<NC, B, F>), dim3((unsigned)M), dim3(kPThreads), 0, st, h, ldh, w, \
                                    rows, q, s, xs, n_rows, (int)M, (int)HID, eps, f)
        if (fold) { if (back == 0) NQ(0, true); else if (back == 1) NQ(1, true); else NQ(2, true); }
        else { if (back == 0) NQ(0, false); else if (back == 1) NQ(1, false); else NQ(2, false); }
#undef NQ
        return hipGetLastError() == hipSuccess ? 0 : (int)PRISM_ERR_LAUNCH;
    });
}

static int check_fold(const Fold& f, int64_t M, int64_t HID) {
    if (f.np < 1 || f.np > 64 || !f.parts || !f.psa || !f.psw) return PRISM_ERR_ARG;
    if (f.ldp < HID || (f.np > 1 && f.part_stride < M * f.ldp)) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(f.parts, 16) || f.ldp % 4 || f.part_stride % 4) return PRISM_ERR_ALIGN;
    return PRISM_OK;
}

// back: 0 int8 + row scale; 1 W4A8 operands, scale per 256; 2 W4A8 operands, one scale per row.
extern "C" int prism_norm_quant(const float* h, int64_t ldh, const float* w, const int32_t* rows, int8_t* q, float* s,
                                int8_t* xs, const int32_t* n_rows, int64_t M, int64_t HID, float eps, int back,
                                void* stream) {
    const Fold none{};
    return norm_launch(const_cast<float*>(h), ldh, w, rows, q, s, xs, n_rows, M, HID, eps, back, none,
                       (hipStream_t)stream);
}

extern "C" int prism_norm_quant_fold(float* h, int64_t ldh, const float* w, int8_t* q, float* s, int8_t* xs,
                                     const int32_t* n_rows, int64_t M, int64_t HID, float eps, int back,
                                     const int32_t* parts, int64_t part_stride, int64_t ldp, int np, const float* psa,
                                     int64_t psa_sm, const void* psw, int psw16, void* stream) {
    const Fold f{parts, part_stride, ldp, np, psa, psa_sm, psw, psw16};
    const int rc = check_fold(f, M, HID);
    if (rc != PRISM_OK) return rc;
    return norm_launch(h, ldh, w, nullptr, q, s, xs, n_rows, M, HID, eps, back, f, (hipStream_t)stream);
}

extern "C" int prism_fold_parts(float* h, int64_t ldh, const int32_t* parts, int64_t part_stride, int64_t ldp, int np,
                                const float* psa, int64_t psa_sm, const void* psw, int psw16, const int32_t* n_rows,
                                int64_t M, int64_t HID, void* stream) {
    if (!h || !n_rows) return PRISM_ERR_ARG;
    if (M < 0 || HID <= 0 || HID % 8 || ldh < HID || ldh % 4 || M > 65535 || HID > (1 << 24)) return PRISM_ERR_SHAPE;
    const Fold f{parts, part_stride, ldp, np, psa, psa_sm, psw, psw16};
    const int rc = check_fold(f, M, HID);
    if (rc != PRISM_OK) return rc;
    if (!PRISM_ALIGNED(h, 16)) return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    hipLaunchKernelGGL(fold_parts_kernel, dim3((unsigned)((HID / 8 + 255) / 256), (unsigned)M), dim3(256), 0,
                       (hipStream_t)stream, h, ldh, f, n_rows, (int)HID);
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_swiglu_quant(const void* gu, int gu_f32, int64_t ldg, const float* inv_s, int8_t* q, float* s,
                                  int8_t* xs, const int32_t* n_rows, int64_t M, int64_t FF, int back, void* stream) {
    if (!gu || !q || !s || !n_rows || (back != 0 && !xs)) return PRISM_ERR_ARG;
    if (back < 0 || back > 2) return PRISM_ERR_ARG;
    if (M < 0 || FF <= 0 || FF % 8 || ldg < 2 * FF || FF > 65536 || M > (1 << 30)) return PRISM_ERR_SHAPE;
    if (back != 0 && FF % 256) return PRISM_ERR_SHAPE;
    if ((gu_f32 ? ldg % 4 : ldg % 8) || !PRISM_ALIGNED(gu, 16) || !PRISM_ALIGNED(q, 8) ||
        (inv_s && !PRISM_ALIGNED(inv_s, 16)))
        return PRISM_ERR_ALIGN;
    if (gu_f32 && FF % 4) return PRISM_ERR_SHAPE;
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    // few rows (decode): 1024 threads per row; the results do not depend on the workgroup size
    const bool wide = M <= 64;
    return pick_nch((int)FF, [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
#define SW(B, G32, T) hipLaunchKernelGGL((swiglu_prod_kernel<NC, B, G32, T>), dim3((unsigned)M), dim3(T), 0, st, gu,  \
                                         ldg, inv_s, q, s, xs, n_rows, (int)M, (int)FF)
#define SWT(B, G32) do { if (wide) SW(B, G32, 1024); else SW(B, G32, kPThreads); } while (0)
        if (gu_f32) { if (back == 0) SWT(0, true); else if (back == 1) SWT(1, true); else SWT(2, true); }
        else { if (back == 0) SWT(0, false); else if (back == 1) SWT(1, false); else SWT(2, false); }
#undef SWT
#undef SW
        return hipGetLastError() == hipSuccess ? 0 : (int)PRISM_ERR_LAUNCH;
    }, wide ? 1024 : kPThreads);
}

// back as prism_norm_quant.  o: the GDN output rows, z: the gate values of the row (the projection row plus the
// caller's column offset), both with their row strides.
extern "C" int prism_gated_norm_quant(const float* o, int64_t ldo, const void* z, int z_f32, int64_t ldz,
                                      const float* w, const float* inv_s, int8_t* q, float* s, int8_t* xs,
                                      const int32_t* n_rows, int64_t M, int64_t HV, int64_t D, float eps, int back,
                                      void* stream) {
    if (!o || !z || !w || !q || !s || !n_rows || (back != 0 && !xs)) return PRISM_ERR_ARG;
    if (back < 0 || back > 2) return PRISM_ERR_ARG;
    if (M < 0 || HV <= 0 || D < 8 || D > 512 || (D & (D - 1)) || HV * D > 32768 || M > (1 << 30)) return PRISM_ERR_SHAPE;
    const int64_t K = HV * D;
    if (ldo < K || ldz < K || (back != 0 && K % 256)) return PRISM_ERR_SHAPE;
    if (ldo % 4 || (z_f32 ? ldz % 4 : ldz % 8) || !PRISM_ALIGNED(o, 16) || !PRISM_ALIGNED(z, 16) ||
        !PRISM_ALIGNED(w, 16) || !PRISM_ALIGNED(q, 8) || (inv_s && !PRISM_ALIGNED(inv_s, 16)))
        return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    const bool wide = M <= 64;                       // as prism_swiglu_quant
    return pick_nch((int)K, [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
#define GN(B, Z, T) hipLaunchKernelGGL((gated_norm_prod_kernel<NC, B, Z, T>), dim3((unsigned)M), dim3(T), 0, st, o,  \
                                       ldo, z, ldz, w, inv_s, q, s, xs, n_rows, (int)M, (int)HV, (int)D, eps)
#define GNT(B, Z) do { if (wide) GN(B, Z, 1024); else GN(B, Z, kPThreads); } while (0)
        if (z_f32) { if (back == 0) GNT(0, true); else if (back == 1) GNT(1, true); else GNT(2, true); }
        else { if (back == 0) GNT(0, false); else if (back == 1) GNT(1, false); else GNT(2, false); }
#undef GNT
#undef GN
        return hipGetLastError() == hipSuccess ? 0 : (int)PRISM_ERR_LAUNCH;
    }, wide ? 1024 : kPThreads);
}
