/*
 * prism_oracle.c -- CPU restatement of StartLux-Prism's quantized linear-layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are compared against; it is never part of
 * the product path.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Every function cites the reference file:line whose arithmetic it restates (paths relative to the
 * StartLux-Prism source tree).  Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off: no fused
 * multiply-adds except where the reference asks for one with an explicit fma).
 *
 * Conventions shared with the GPU library:
 *   bf16 / fp16 values travel as uint16_t bit patterns; conversions to them round to nearest even.
 *   "live" rows: rows >= live are neither computed nor written (kernels/w8a8.py:44-46, 77-80).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------------------------- float formats */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

EXPORT float orc_bf16_to_float(uint16_t h) { return u2f((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even; NaN stays a quiet NaN (torch's .to(torch.bfloat16)). */
EXPORT uint16_t orc_float_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

EXPORT float orc_half_to_float(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    if (e == 0x1f) return u2f(s | 0x7f800000u | (m << 13));
    if (e == 0) {                                   /* zero or subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * 0x1p-24f;
        return s ? -v : v;
    }
    return u2f(s | ((e + 112) << 23) | (m << 13));
}

/* fp32 -> fp16, round to nearest even, overflow to inf (numpy / torch .half()). */
EXPORT uint16_t orc_float_to_half(float f) {
    uint32_t u = f2u(f), s = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(s | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u);        /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                         /* below 2^-14: subnormal half */
        /* value = a_f; half subnormal unit 2^-24: q = rint(a_f * 2^24) (exact scaling, one rounding) */
        float v = u2f(a) * 0x1p24f;
        return (uint16_t)(s | (uint32_t)rintf(v));
    }
    uint32_t e = (a >> 23) - 112, m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13), rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(s | h);
}

static inline int nthreads_or(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* ----------------------------------------------------------------------------------------------- Q8_0 */
/*
 * Q8_0 quantizer: gguf_weights.py:121-133 (KQuant.as_q8) -- per 32 values dh = fp16(amax / 127),
 * inv = 1 / float(dh) (0 when dh == 0), q = clamp(round(w * inv), -127, 127), round half to even.
 * w fp32 [N, K] -> qs int8 [N, K], d fp16 [N, K / 32].
 */
EXPORT void orc_q8_0_quantize(const float* w, int64_t N, int64_t K, int8_t* qs, uint16_t* d, int nthreads) {
    int64_t G = K / 32;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t n = 0; n < N; n++) {
        for (int64_t g = 0; g < G; g++) {
            const float* x = w + n * K + g * 32;
            float amax = 0.f;
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
            uint16_t dh = orc_float_to_half(amax / 127.0f);
            float df = orc_half_to_float(dh);
            float inv = df > 0.f ? 1.0f / df : 0.f;
            for (int i = 0; i < 32; i++) {
                float q = rintf(x[i] * inv);
                q = q > 127.f ? 127.f : (q < -127.f ? -127.f : q);
                qs[n * K + g * 32 + i] = (int8_t)q;
            }
            d[n * G + g] = dh;
        }
    }
}

/*
 * Per-token int8 activation quantization: kernels/quant.py:287-309 (_rows_q8_kernel; MODE 0):
 * y = x * inv_s (inv_s NULL: y = x), scale = max(amax(|y|), 1e-10) / 127, q = rint(y / scale).
 * Both divisions are IEEE (correctly rounded), the convention of kernels/quant.py:320-321 and w4a8.py:151.
 * x bf16 [M, K] with row stride ldx -> q int8 [M, K], s fp32 [M].  Rows >= live are untouched.
 */
EXPORT void orc_quant_rows_i8(const uint16_t* x, int64_t ldx, const float* inv_s, int64_t M, int64_t K,
                              int64_t live, int8_t* q, float* s, int nthreads) {
    (void)M;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t m = 0; m < live; m++) {
        float amax = 0.f;
        for (int64_t k = 0; k < K; k++) {
            float y = orc_bf16_to_float(x[m * ldx + k]);
            if (inv_s) y = y * inv_s[k];
            amax = fmaxf(amax, fabsf(y));
        }
        float scale = fmaxf(amax, 1e-10f) / 127.0f;
        for (int64_t k = 0; k < K; k++) {
            float y = orc_bf16_to_float(x[m * ldx + k]);
            if (inv_s) y = y * inv_s[k];
            q[m * K + k] = (int8_t)rintf(y / scale);
        }
        s[m] = scale;
    }
}

/*
 * Per-(row, group) int8 quantization: kernels/w8a8.py:101-112 (_quant_rows_kernel) and quant_rows (:264-271):
 * per gk inputs scale = max(amax, 1e-10) / 127, q = rint(x / scale).  x bf16 [M, K] -> q [M, K], s fp32 [M, K/gk].
 */
EXPORT void orc_quant_rows_groups(const uint16_t* x, int64_t M, int64_t K, int64_t gk, int64_t live, int8_t* q,
                                  float* s, int nthreads) {
    (void)M;
    int64_t G = K / gk;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t m = 0; m < live; m++) {
        for (int64_t g = 0; g < G; g++) {
            float amax = 0.f;
            for (int64_t k = g * gk; k < (g + 1) * gk; k++) amax = fmaxf(amax, fabsf(orc_bf16_to_float(x[m * K + k])));
            float scale = fmaxf(amax, 1e-10f) / 127.0f;
            for (int64_t k = g * gk; k < (g + 1) * gk; k++)
                q[m * K + k] = (int8_t)rintf(orc_bf16_to_float(x[m * K + k]) / scale);
            s[m * G + g] = scale;
        }
    }
}

static inline int32_t dot_i8(const int8_t* a, const int8_t* b, int64_t n) {
    int32_t acc = 0;
    for (int64_t i = 0; i < n; i++) acc += (int32_t)a[i] * (int32_t)b[i];
    return acc;
}

/* The int32 dot product of every (row, column, group): P[m, n, g] = sum_{k in g} a[m, k] w[n, k]
 * (kernels/w8a8.py:66-73, tl.dot int8 -> int32).  For tests on small shapes. */
EXPORT void orc_w8a8_block_sums(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K, int64_t gk,
                                int32_t* P) {
    int64_t G = K / gk;
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++)
            for (int64_t g = 0; g < G; g++) P[(m * N + n) * G + g] = dot_i8(a + m * K + g * gk, w + n * K + g * gk, gk);
}

/*
 * W8A8 GEMM with per-group scales along K: kernels/w8a8.py:64-85 (_w8a8_kernel, EPI 0 and 1).
 *   per group g in increasing order: P = sum_{k in g} a w (int32, exact);
 *                                    y = RN(y + RN(RN(float(P) * sa[m, g]) * sw[n, g]))     (:74-76)
 *   epi 0: out bf16 = RN_bf16(y) (:78-80);  epi 1: out fp32 = RN(out + y) (:81-85).
 * a int8 [M, K]; a_s fp32 with element (m, g) at a_s[m * as_sm + g * as_sg] (as_sg = 0: one scale per token);
 * w int8 [N, K]; w_s per (n, g) at w_s[n * (K/gk) + g], fp16 bits when ws_fp16 else fp32
 * (Q8_0's fp16 block scale as fp32 is exact: w8a8.py:277-278).  out row stride ldo (elements).
 */
EXPORT void orc_w8a8_gemm(const int8_t* a, const float* a_s, int64_t as_sm, int64_t as_sg, const int8_t* w,
                          const void* w_s, int ws_fp16, int64_t M, int64_t N, int64_t K, int64_t gk, int epi,
                          void* out, int64_t ldo, int64_t live, int nthreads) {
    (void)M;
    int64_t G = K / gk;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(dynamic, 1)
    for (int64_t m = 0; m < live; m++) {
        for (int64_t n = 0; n < N; n++) {
            float y = 0.f;
            for (int64_t g = 0; g < G; g++) {
                int32_t p = dot_i8(a + m * K + g * gk, w + n * K + g * gk, gk);
                float sa = a_s[m * as_sm + g * as_sg];
                float sw = ws_fp16 ? orc_half_to_float(((const uint16_t*)w_s)[n * G + g]) : ((const float*)w_s)[n * G + g];
                float t = (float)p * sa;
                t = t * sw;
                y = y + t;
            }
            if (epi == 0)
                ((uint16_t*)out)[m * ldo + n] = orc_float_to_bf16(y);
            else {
                float* o = (float*)out + m * ldo + n;
                *o = *o + y;
            }
        }
    }
}

/*
 * The reassociated form of orc_w8a8_gemm for one activation scale per token (this build's "reassoc" kernel choice,
 * not the reference's order): the per-token scale factors out of the block sum, so per block g in increasing g
 * y = fmaf(float(P), sw, y) (one rounding), then y = RN(y sa[m]), then the same epilogues.  P is the same exact int32
 * block sum; only the fp32 rounding sequence differs from kernels/w8a8.py:64-85.
 */
EXPORT void orc_w8a8_gemm_reassoc(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* w, const void* w_s,
                                  int ws_fp16, int64_t N, int64_t K, int64_t gk, int epi, void* out, int64_t ldo,
                                  int64_t live, int nthreads) {
    int64_t G = K / gk;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(dynamic, 1)
    for (int64_t m = 0; m < live; m++) {
        for (int64_t n = 0; n < N; n++) {
            float y = 0.f;
            for (int64_t g = 0; g < G; g++) {
                int32_t p = dot_i8(a + m * K + g * gk, w + n * K + g * gk, gk);
                float sw = ws_fp16 ? orc_half_to_float(((const uint16_t*)w_s)[n * G + g]) : ((const float*)w_s)[n * G + g];
                y = fmaf((float)p, sw, y);
            }
            y = y * a_s[m * as_sm];
            if (epi == 0)
                ((uint16_t*)out)[m * ldo + n] = orc_float_to_bf16(y);
            else {
                float* o = (float*)out + m * ldo + n;
                *o = *o + y;
            }
        }
    }
}

/*
 * The residual add deferred by a split-K per-channel projection (kernels/quant.py:129-141 _fold_parts, run by norm_q8
 * :160-166 and fold :435-457): tot = the sum over the np slots of parts[p][r][c] (int32: the splits' sums add up to
 * the unsplit product's exact sum), then h[r][c] = RN(h + RN(RN(float(tot) psa[r]) psw[c])), the epilogue 1 of the
 * unsplit product (orc_w8a8_gemm with gk = K, epi 1).  parts: slot stride part_stride, row stride ldp (elements);
 * psa row r at psa[r * psa_sm]; psw fp32, fp16 bits when psw16.  Rows >= live untouched.
 */
EXPORT void orc_fold_parts(float* h, int64_t ldh, const int32_t* parts, int64_t part_stride, int64_t ldp, int np,
                           const float* psa, int64_t psa_sm, const void* psw, int psw16, int64_t live, int64_t HID) {
    for (int64_t r = 0; r < live; r++)
        for (int64_t c = 0; c < HID; c++) {
            int64_t tot = 0;
            for (int p = 0; p < np; p++) tot += parts[p * part_stride + r * ldp + c];
            float sw = psw16 ? orc_half_to_float(((const uint16_t*)psw)[c]) : ((const float*)psw)[c];
            float t = (float)(int32_t)tot * psa[r * psa_sm];
            t = t * sw;
            h[r * ldh + c] = h[r * ldh + c] + t;
        }
}

/* ----------------------------------------------------------------------------------------------- Q4_K */
/*
 * A Q4_K quantizer of this build's own (the reference only reads Q4_K from files: gguf_weights.py:100-133).
 * Per 256-value super-block: per sub-block j of 32, lo_j = min(0, min x), hi_j = max x, scale_j = (hi_j - lo_j)/15,
 * min_j = -lo_j; d = fp16(max scale_j / 63), dmin = fp16(max min_j / 63); sc_j = clamp(rint(scale_j / d), 0, 63),
 * m_j = clamp(rint(min_j / dmin), 0, 63); q = clamp(rint((x + dmin m_j) / (d sc_j)), 0, 15).
 * Output: GGUF block_q4_K bytes [N, K/256, 144]: d, dmin (fp16 LE), scales[12] in ggml's 6-bit packing
 * (inverse of get_scale_min_k4, gguf_weights.py:56-60), qs[128] (per 32 bytes: low nibbles sub-block 2c, high
 * nibbles 2c + 1: gguf_weights.py:63-70).
 */
EXPORT void orc_q4k_quantize(const float* w, int64_t N, int64_t K, uint8_t* blocks, int nthreads) {
    int64_t NB = K / 256;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t n = 0; n < N; n++) {
        for (int64_t b = 0; b < NB; b++) {
            const float* x = w + n * K + b * 256;
            uint8_t* o = blocks + (n * NB + b) * 144;
            float scale[8], mn[8], smax = 0.f, mmax = 0.f;
            for (int j = 0; j < 8; j++) {
                float lo = 0.f, hi = -INFINITY;
                for (int i = 0; i < 32; i++) { lo = fminf(lo, x[32 * j + i]); hi = fmaxf(hi, x[32 * j + i]); }
                if (hi < lo) hi = lo;
                scale[j] = (hi - lo) / 15.f;
                mn[j] = -lo;
                smax = fmaxf(smax, scale[j]);
                mmax = fmaxf(mmax, mn[j]);
            }
            uint16_t dh = orc_float_to_half(smax / 63.f), dmh = orc_float_to_half(mmax / 63.f);
            float d = orc_half_to_float(dh), dmin = orc_half_to_float(dmh);
            uint8_t sc[8], m[8];
            for (int j = 0; j < 8; j++) {
                float s = d > 0.f ? rintf(scale[j] / d) : 0.f, t = dmin > 0.f ? rintf(mn[j] / dmin) : 0.f;
                sc[j] = (uint8_t)(s < 0.f ? 0.f : (s > 63.f ? 63.f : s));
                m[j] = (uint8_t)(t < 0.f ? 0.f : (t > 63.f ? 63.f : t));
            }
            o[0] = dh & 0xff; o[1] = dh >> 8; o[2] = dmh & 0xff; o[3] = dmh >> 8;
            uint8_t* s12 = o + 4;
            for (int j = 0; j < 4; j++) {
                s12[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
                s12[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
                s12[j + 8] = (uint8_t)((sc[j + 4] & 0xf) | ((m[j + 4] & 0xf) << 4));
            }
            uint8_t qv[256];
            for (int j = 0; j < 8; j++) {
                float step = d * (float)sc[j], off = dmin * (float)m[j];
                for (int i = 0; i < 32; i++) {
                    float q = step > 0.f ? rintf((x[32 * j + i] + off) / step) : 0.f;
                    qv[32 * j + i] = (uint8_t)(q < 0.f ? 0.f : (q > 15.f ? 15.f : q));
                }
            }
            for (int c = 0; c < 4; c++)
                for (int t = 0; t < 32; t++) o[16 + 32 * c + t] = (uint8_t)(qv[64 * c + t] | (qv[64 * c + 32 + t] << 4));
        }
    }
}

/* get_scale_min_k4: gguf_weights.py:56-60. */
static void scale_min_k4(const uint8_t* s, uint8_t* sc, uint8_t* mn) {
    for (int j = 0; j < 4; j++) {
        sc[j] = s[j] & 63;
        mn[j] = s[j + 4] & 63;
        sc[j + 4] = (uint8_t)((s[j + 8] & 0xf) | ((s[j] >> 6) << 4));
        mn[j + 4] = (uint8_t)((s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4));
    }
}

/* Q4_K dequantization: gguf_weights.py:63-70 (_dq_q4_k), y = (d sc) q - (dmin m), products and difference in fp32. */
EXPORT void orc_q4k_dequant(const uint8_t* blocks, int64_t N, int64_t K, float* w) {
    int64_t NB = K / 256;
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < NB; b++) {
            const uint8_t* o = blocks + (n * NB + b) * 144;
            float d = orc_half_to_float((uint16_t)(o[0] | (o[1] << 8))), dmin = orc_half_to_float((uint16_t)(o[2] | (o[3] << 8)));
            uint8_t sc[8], mn[8];
            scale_min_k4(o + 4, sc, mn);
            for (int j = 0; j < 8; j++) {
                float a = d * (float)sc[j], c = dmin * (float)mn[j];
                for (int t = 0; t < 32; t++) {
                    uint8_t byte = o[16 + 32 * (j / 2) + t];
                    float q = (float)((j & 1) ? (byte >> 4) : (byte & 0xf));
                    w[n * K + b * 256 + 32 * j + t] = a * q - c;
                }
            }
        }
}

/*
 * Q4_K -> the W4 layout the GEMM reads: kernels/w4a8.py:44-81 (W4, repack).
 *   q uint8 [N, K/2]: per 32 inputs 16 bytes, byte t = q[t] | q[t + 16] << 4 (values in k order);
 *   sc, mn uint8 [K/256, N, 8]; d, dm fp32 [K/256, N] (super-block-major).
 */
EXPORT void orc_q4k_repack(const uint8_t* blocks, int64_t N, int64_t K, uint8_t* q, uint8_t* sc, uint8_t* mn,
                           float* d, float* dm) {
    int64_t NB = K / 256;
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < NB; b++) {
            const uint8_t* o = blocks + (n * NB + b) * 144;
            d[b * N + n] = orc_half_to_float((uint16_t)(o[0] | (o[1] << 8)));
            dm[b * N + n] = orc_half_to_float((uint16_t)(o[2] | (o[3] << 8)));
            scale_min_k4(o + 4, sc + (b * N + n) * 8, mn + (b * N + n) * 8);
            for (int j = 0; j < 8; j++) {
                uint8_t v[32];
                for (int t = 0; t < 32; t++) {
                    uint8_t byte = o[16 + 32 * (j / 2) + t];
                    v[t] = (j & 1) ? (byte >> 4) : (byte & 0xf);
                }
                for (int t = 0; t < 16; t++) q[n * (K / 2) + b * 128 + j * 16 + t] = (uint8_t)(v[t] | (v[t + 16] << 4));
            }
        }
}

/*
 * W4A8 activation producer: kernels/w4a8.py:144-155 (quantize_ref) = kernels/quant.py:314-330 (_store_g).
 * x fp32 [M, K] (the bf16 input, widened); per `group` inputs (256 in the reference; K for one scale per token)
 * a = max(amax, 1e-10) / 127 (true division), xq = rint(x / a) (true division); per 32 inputs the int32 sum S of
 * xq, stored as eight S & 63 then eight S >> 6 per 256 inputs.
 * Outputs: xq int8 [M, K]; a fp32 [K/group, M]; xs int8 [K/256, M, 16].  Rows >= live untouched.
 */
EXPORT void orc_quant_rows_g(const float* x, int64_t M, int64_t K, int64_t group, int64_t live, int8_t* xq, float* a,
                             int8_t* xs, int nthreads) {
    int64_t G = K / group, NB = K / 256;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t m = 0; m < live; m++) {
        for (int64_t g = 0; g < G; g++) {
            float amax = 0.f;
            for (int64_t k = g * group; k < (g + 1) * group; k++) amax = fmaxf(amax, fabsf(x[m * K + k]));
            float sc = fmaxf(amax, 1e-10f) / 127.0f;
            for (int64_t k = g * group; k < (g + 1) * group; k++) xq[m * K + k] = (int8_t)rintf(x[m * K + k] / sc);
            a[g * M + m] = sc;
        }
        for (int64_t b = 0; b < NB; b++)
            for (int j = 0; j < 8; j++) {
                int32_t S = 0;
                for (int t = 0; t < 32; t++) S += xq[m * K + b * 256 + 32 * j + t];
                xs[(b * M + m) * 16 + j] = (int8_t)(S & 63);
                xs[(b * M + m) * 16 + 8 + j] = (int8_t)(S >> 6);
            }
    }
}

/*
 * W4A8 GEMM on Q4_K: kernels/w4a8.py:14-22 (arithmetic) and :177-199 (gemm_ref), per super-block b in order:
 *   acc  = sum_g sc[b,n,g] * (xq . q)_g            int32, exact
 *   mins = sum_g mn[b,n,g] * S[m, 8b + g]           int32, exact (S = (xs & 63 part) + 64 * (xs >> 6 part), :158-161)
 *   t = RN(d[b,n] * float(acc));  t = fma(-dm[b,n], float(mins), t);  y = fma(a[b,m], t, y)
 * then epi 0: bf16(y); epi 1: out = RN(out + y).  fma32 (:164-174) is IEEE fma: C fmaf.
 * a fp32: element (b, m) at a[b * a_sb + m] (a_sb = 0: one scale per token).
 * acc_out / mins_out (nullable) receive the int32 super-block sums [M, N, K/256] for bit-exactness tests.
 */
EXPORT void orc_w4a8_gemm(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs, const uint8_t* q,
                          const uint8_t* sc, const uint8_t* mn, const float* d, const float* dm, int64_t M, int64_t N,
                          int64_t K, int epi, void* out, int64_t ldo, int64_t live, int32_t* acc_out,
                          int32_t* mins_out, int nthreads) {
    int64_t NB = K / 256;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(dynamic, 1)
    for (int64_t m = 0; m < live; m++) {
        int8_t qv[256];
        for (int64_t n = 0; n < N; n++) {
            float y = 0.f;
            for (int64_t b = 0; b < NB; b++) {
                const uint8_t* qb = q + n * (K / 2) + b * 128;
                for (int j = 0; j < 8; j++)
                    for (int t = 0; t < 16; t++) {
                        qv[32 * j + t] = (int8_t)(qb[16 * j + t] & 0xf);
                        qv[32 * j + 16 + t] = (int8_t)(qb[16 * j + t] >> 4);
                    }
                int32_t acc = 0, mins = 0;
                const int8_t* xb = xs + (b * M + m) * 16;
                for (int j = 0; j < 8; j++) {
                    acc += (int32_t)sc[(b * N + n) * 8 + j] * dot_i8(xq + m * K + b * 256 + 32 * j, qv + 32 * j, 32);
                    int32_t S = (int32_t)xb[j] + 64 * (int32_t)xb[8 + j];
                    mins += (int32_t)mn[(b * N + n) * 8 + j] * S;
                }
                if (acc_out) acc_out[(m * N + n) * NB + b] = acc;
                if (mins_out) mins_out[(m * N + n) * NB + b] = mins;
                float t = d[b * N + n] * (float)acc;
                t = fmaf(-dm[b * N + n], (float)mins, t);
                y = fmaf(a[b * a_sb + m], t, y);
            }
            if (epi == 0)
                ((uint16_t*)out)[m * ldo + n] = orc_float_to_bf16(y);
            else {
                float* o = (float*)out + m * ldo + n;
                *o = *o + y;
            }
        }
    }
}

/* ----------------------------------------------------------------------------------------------- Q6_K */
/*
 * GGUF block_q6_K (210 bytes per 256 values; ggml's layout as gguf_weights.py:85-97 _dq_q6_k reads it): ql[128]
 * low 4 bits, qh[64] high 2 bits, scales int8[16] (one per 16 values), d fp16.  Per half h of 128 values and
 * l < 32, with Q = q + 32 in 0..63 of values v = 128 h + l + 32 i (i = 0..3):
 *   ql[64 h + l] = Q0 & 15 | (Q2 & 15) << 4,  ql[64 h + 32 + l] = Q1 & 15 | (Q3 & 15) << 4,
 *   qh[32 h + l] = Q0 >> 4 | (Q1 >> 4) << 2 | (Q2 >> 4) << 4 | (Q3 >> 4) << 6.
 */
static int q6k_value(const uint8_t* o, int v) {
    const int h = v / 128, r = v % 128, i = r / 32, l = r % 32;
    const uint8_t lq = o[64 * h + 32 * (i & 1) + l];
    const int lo = (i < 2) ? (lq & 15) : (lq >> 4);
    const int hi = (o[128 + 32 * h + l] >> (2 * i)) & 3;
    return (lo | (hi << 4)) - 32;
}

/*
 * A Q6_K quantizer of this build's own (the reference only reads Q6_K from files).  Per sub-block j of 16:
 * scale_j = max|x| / 31; d = fp16(max scale_j / 127); sc_j = clamp(rint(scale_j / d), -128, 127);
 * q = clamp(rint(x / (d sc_j)), -32, 31).
 */
EXPORT void orc_q6k_quantize(const float* w, int64_t N, int64_t K, uint8_t* blocks, int nthreads) {
    const int64_t NB = K / 256;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < NB; b++) {
            const float* x = w + n * K + b * 256;
            uint8_t* o = blocks + (n * NB + b) * 210;
            float scale[16], smax = 0.f;
            for (int j = 0; j < 16; j++) {
                float a = 0.f;
                for (int t = 0; t < 16; t++) a = fmaxf(a, fabsf(x[16 * j + t]));
                scale[j] = a / 31.f;
                smax = fmaxf(smax, scale[j]);
            }
            const uint16_t dh = orc_float_to_half(smax / 127.f);
            const float d = orc_half_to_float(dh);
            int8_t sc[16];
            int Q[256];
            for (int j = 0; j < 16; j++) {
                float t = d > 0.f ? rintf(scale[j] / d) : 0.f;
                sc[j] = (int8_t)(t < -128.f ? -128.f : (t > 127.f ? 127.f : t));
                const float step = d * (float)sc[j];
                for (int u = 0; u < 16; u++) {
                    float q = step != 0.f ? rintf(x[16 * j + u] / step) : 0.f;
                    q = q < -32.f ? -32.f : (q > 31.f ? 31.f : q);
                    Q[16 * j + u] = (int)q + 32;
                }
            }
            for (int h = 0; h < 2; h++)
                for (int l = 0; l < 32; l++) {
                    const int* P = Q + 128 * h + l;
                    o[64 * h + l] = (uint8_t)((P[0] & 15) | ((P[64] & 15) << 4));
                    o[64 * h + 32 + l] = (uint8_t)((P[32] & 15) | ((P[96] & 15) << 4));
                    o[128 + 32 * h + l] = (uint8_t)((P[0] >> 4) | ((P[32] >> 4) << 2) | ((P[64] >> 4) << 4) | ((P[96] >> 4) << 6));
                }
            for (int j = 0; j < 16; j++) o[192 + j] = (uint8_t)sc[j];
            o[208] = dh & 0xff;
            o[209] = dh >> 8;
        }
}

/* Q6_K dequantization: gguf_weights.py:85-97 (_dq_q6_k), y = RN(d sc) (q - 32) in fp32. */
EXPORT void orc_q6k_dequant(const uint8_t* blocks, int64_t N, int64_t K, float* w) {
    const int64_t NB = K / 256;
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < NB; b++) {
            const uint8_t* o = blocks + (n * NB + b) * 210;
            const float d = orc_half_to_float((uint16_t)(o[208] | (o[209] << 8)));
            for (int v = 0; v < 256; v++) {
                const float ds = d * (float)(int8_t)o[192 + v / 16];
                w[n * K + b * 256 + v] = ds * (float)q6k_value(o, v);
            }
        }
}

/*
 * Q6_K -> the W4 layout of kernels/w4a8.py:82-90 (repack): q int8 [N, K] (values - 32, k order), sc int8
 * [K/256, N, 16], d fp32 [K/256, N].
 */
EXPORT void orc_q6k_repack(const uint8_t* blocks, int64_t N, int64_t K, int8_t* q, int8_t* sc, float* d) {
    const int64_t NB = K / 256;
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < NB; b++) {
            const uint8_t* o = blocks + (n * NB + b) * 210;
            for (int v = 0; v < 256; v++) q[n * K + b * 256 + v] = (int8_t)q6k_value(o, v);
            for (int j = 0; j < 16; j++) sc[(b * N + n) * 16 + j] = (int8_t)o[192 + j];
            d[b * N + n] = orc_half_to_float((uint16_t)(o[208] | (o[209] << 8)));
        }
}

/*
 * W4A8 GEMM on Q6_K: kernels/w4a8.py:19-20 (arithmetic) and :193-197 (gemm_ref), per super-block b in order:
 *   acc = sum_h sc[b,n,h] * (xq . q)_h    int32, exact (16 sub-blocks of 16)
 *   y = fma(a[b,m], RN(d[b,n] * float(acc)), y)
 * then epi 0 bf16(y), epi 1 out = RN(out + y).  acc_out (nullable): the int32 super-block sums [M, N, K/256].
 */
EXPORT void orc_w4a8_gemm_q6k(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* q, const int8_t* sc,
                              const float* d, int64_t M, int64_t N, int64_t K, int epi, void* out, int64_t ldo,
                              int64_t live, int32_t* acc_out, int nthreads) {
    const int64_t NB = K / 256;
    (void)M;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(dynamic, 1)
    for (int64_t m = 0; m < live; m++)
        for (int64_t n = 0; n < N; n++) {
            float y = 0.f;
            for (int64_t b = 0; b < NB; b++) {
                int32_t acc = 0;
                for (int h = 0; h < 16; h++)
                    acc += (int32_t)sc[(b * N + n) * 16 + h] *
                           dot_i8(xq + m * K + b * 256 + 16 * h, q + n * K + b * 256 + 16 * h, 16);
                if (acc_out) acc_out[(m * N + n) * NB + b] = acc;
                const float t = d[b * N + n] * (float)acc;
                y = fmaf(a[b * a_sb + m], t, y);
            }
            if (epi == 0)
                ((uint16_t*)out)[m * ldo + n] = orc_float_to_bf16(y);
            else {
                float* o = (float*)out + m * ldo + n;
                *o = *o + y;
            }
        }
}

EXPORT double orc_fmaf(float a, float b, float c) { return (double)fmaf(a, b, c); }

/* ------------------------------------------------------------------------------------------------ MXFP4 */
/* Formats (kernels/mxfp4.py:1-6, tests/quant_sim.py:40-81): e2m1 codes 0..7 = {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3
 * the sign; e4m3 (OCP float8_e4m3fn, bias 7, max 448, no infinities); e8m0 scale byte b = 2^(b - 127). */
static const float MX_E2M1[8] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};

EXPORT float orc_e2m1_value(int code) { float v = MX_E2M1[code & 7]; return (code & 8) ? -v : v; }

EXPORT float orc_e4m3_value(int code) {
    int e = (code >> 3) & 15, m = code & 7;
    if (e == 15 && m == 7) return NAN;
    float v = e ? ldexpf(1.f + m / 8.f, e - 7) : ldexpf((float)m, -9);
    return (code & 0x80) ? -v : v;
}

/* |x| / scale -> e2m1 magnitude code.  ties == 0: the engine's strict thresholds, midpoints round toward zero
 * (kernels/mxfp4.py:40-54 for weights, :110-121 for activations; tests/quant_sim.py:43-48 bucketizes the same way).
 * ties == 1: round to nearest, ties to the even code, saturating at 6 (the OCP MX conversion the C4 workload
 * specifies). */
static inline int mx_e2m1_mag(float a, int ties) {
    if (ties == 0)
        return (a > .25f) + (a > .75f) + (a > 1.25f) + (a > 1.75f) + (a > 2.5f) + (a > 3.5f) + (a > 5.f);
    return (a > .25f) + (a >= .75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) + (a > 5.f);
}

/* floor(log2(v)) and ceil(log2(v)) of a positive normal fp32 value, exactly (from its exponent bits). */
static inline int ilog2_floor(float v) { int e; float m = frexpf(v, &e); (void)m; return e - 1; }
static inline int ilog2_ceil(float v) { int e; float m = frexpf(v, &e); return m == .5f ? e - 1 : e; }

/* fp32 -> e4m3 code, round to nearest even, |v| <= 448 assumed (callers clamp first, as tests/quant_sim.py:81
 * clamps before .to(torch.float8_e4m3fn)).  The sign bit follows the input's (so -0 and tiny negatives -> 0x80). */
EXPORT int orc_e4m3_code(float v) {
    int s = signbit(v) ? 0x80 : 0;
    float a = fabsf(v);
    if (a < 0x1p-6f) return s | (int)rintf(a * 512.f);       /* subnormal step 2^-9; 2^-6 itself -> code 8 */
    int E = ilog2_floor(a);
    int m = (int)rintf(ldexpf(a, 3 - E));                     /* 8..16, exact scaling then one rounding */
    return s | ((E + 6) * 8 + m);
}

/* One 32-block: the e8m0 exponent and the 32 codes (low nibble first for e2m1).  mode 0 "max" and 1 "mse"
 * follow kernels/mxfp4.py:57-86 (pack); mode 2 "ocp" follows tests/quant_sim.py:66-72 (2^(floor(log2 amax) - 2))
 * with round-to-nearest-even codes. */
static int mx_block_e2m1(const float* w, int mode, uint8_t* codes) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(w[i]));
    int e;
    if (mode == 2) {
        e = ilog2_floor(fmaxf(amax, 1e-30f)) - 2;
    } else {
        e = ilog2_ceil(fmaxf(amax, 1e-30f) / 6.0f);
        if (e > 127) e = 127;
        if (e < -127) e = -127;
        if (mode == 1) {
            /* the power of two among e and e - 1 with the smaller squared error; numpy's float32 sum over the
             * 32 values (pairwise: eight strided partial sums, then a fixed tree) */
            int cand[2] = {e, e - 1 < -127 ? -127 : e - 1};
            float err[2];
            for (int c = 0; c < 2; c++) {
                float s = ldexpf(1.f, cand[c]), r[8] = {0};
                for (int i = 0; i < 32; i++) {
                    float a = fabsf(w[i]) / s;
                    int q = mx_e2m1_mag(a, 0);
                    float v = MX_E2M1[q] * s;
                    if (w[i] < 0 && q) v = -v;
                    float d = v - w[i];
                    r[i % 8] = (i < 8) ? d * d : r[i % 8] + d * d;
                }
                err[c] = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
            }
            if (err[1] < err[0]) e = cand[1];
        }
    }
    float s = ldexpf(1.f, e);
    for (int i = 0; i < 32; i++) {
        float a = fabsf(w[i]) / s;
        int q = mx_e2m1_mag(mode == 2 ? fminf(a, 6.f) : a, mode == 2);
        if (w[i] < 0 && q) q |= 8;
        codes[i] = (uint8_t)q;
    }
    return e;
}

/* Weights fp32 [N, K] -> q uint8 [N, K/2] (low nibble first), s uint8 [N, K/32] (e + 127).
 * kernels/mxfp4.py:57-86 (modes 0, 1); tests/quant_sim.py:66-72 (mode 2). */
EXPORT void orc_mx_pack(const float* w, int64_t N, int64_t K, int mode, uint8_t* q, uint8_t* s, int nthreads) {
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < K / 32; b++) {
            uint8_t c[32];
            int e = mx_block_e2m1(w + n * K + b * 32, mode, c);
            s[n * (K / 32) + b] = (uint8_t)(e + 127);
            for (int i = 0; i < 16; i++) q[n * (K / 2) + b * 16 + i] = (uint8_t)(c[2 * i] | (c[2 * i + 1] << 4));
        }
}

/* Activations fp32 [M, K] (bf16 inputs widened exactly), optionally times inv[K] (fp32 multiply,
 * kernels/mxfp4.py:153-154):
 *   fmt 4 (e2m1): kernels/mxfp4.py:124-146 (_quant_kernel): e = clip(ceil(log2(max(amax, 1e-30) / 6)), +-127),
 *                 codes by strict thresholds, sign bit set for every negative input (also when the code is 0);
 *                 q [M, K/2];
 *   fmt 0 (e4m3): tests/quant_sim.py:75-81 (mxfp8): e = floor(log2(max(amax, 1e-30))) - 8, codes
 *                 e4m3(clamp(x / 2^e, +-448)) rounded to nearest even; q [M, K].
 * s [M, K/32] = e + 127.  Rows >= live are not written. */
EXPORT void orc_mx_quant_act(const float* x, const float* inv, int64_t M, int64_t K, int fmt, int64_t live,
                             uint8_t* q, uint8_t* s, int nthreads) {
    const int64_t rows = live < M ? live : M;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t m = 0; m < rows; m++)
        for (int64_t b = 0; b < K / 32; b++) {
            float v[32], amax = 0.f;
            for (int i = 0; i < 32; i++) {
                v[i] = x[m * K + b * 32 + i];
                if (inv) v[i] = v[i] * inv[b * 32 + i];
                amax = fmaxf(amax, fabsf(v[i]));
            }
            int e;
            if (fmt == 0) {
                e = ilog2_floor(fmaxf(amax, 1e-30f)) - 8;
                float sc = ldexpf(1.f, e);
                for (int i = 0; i < 32; i++) {
                    float a = v[i] / sc;
                    a = fminf(fmaxf(a, -448.f), 448.f);
                    q[m * K + b * 32 + i] = (uint8_t)orc_e4m3_code(a);
                }
            } else {
                e = ilog2_ceil(fmaxf(amax, 1e-30f) / 6.0f);
                if (e > 127) e = 127;
                if (e < -127) e = -127;
                float sc = ldexpf(1.f, e);
                uint8_t c[32];
                for (int i = 0; i < 32; i++) c[i] = (uint8_t)(mx_e2m1_mag(fabsf(v[i]) / sc, 0) | (v[i] < 0 ? 8 : 0));
                for (int i = 0; i < 16; i++) q[m * (K / 2) + b * 16 + i] = (uint8_t)(c[2 * i] | (c[2 * i + 1] << 4));
            }
            s[m * (K / 32) + b] = (uint8_t)(e + 127);
        }
}

/* y[m, n] = sum_k a(m, k) 2^(sa(m, k/32) - 127) w(n, k) 2^(sw(n, k/32) - 127), in float64 (every product of two
 * such values is exact in float64; the sum's relative error is ~1e-16).  The fp32-accumulating GEMM of
 * kernels/mxfp4.py:260-289 and its test (tests/test_mxfp4.py:56-60: the dequantised product) are compared with
 * this value within a stated bound.  a: fmt 0 -> e4m3 [M, K], fmt 4 -> e2m1 [M, K/2]; w: e2m1 [N, K/2]. */
EXPORT void orc_mx_gemm(const uint8_t* aq, const uint8_t* as, int fmt, const uint8_t* wq, const uint8_t* ws,
                        int64_t M, int64_t N, int64_t K, double* y, double* yabs, int nthreads) {
    float e4[256];
    for (int c = 0; c < 256; c++) e4[c] = orc_e4m3_value(c);
    double* wv = (double*)malloc(sizeof(double) * N * K);
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t k = 0; k < K; k++)
            wv[n * K + k] = ldexp((double)orc_e2m1_value((wq[n * (K / 2) + k / 2] >> (4 * (k & 1))) & 15),
                                  (int)ws[n * (K / 32) + k / 32] - 127);
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t m = 0; m < M; m++) {
        double* av = (double*)malloc(sizeof(double) * K);
        for (int64_t k = 0; k < K; k++) {
            float c = fmt == 0 ? e4[aq[m * K + k]]
                               : orc_e2m1_value((aq[m * (K / 2) + k / 2] >> (4 * (k & 1))) & 15);
            av[k] = ldexp((double)c, (int)as[m * (K / 32) + k / 32] - 127);
        }
        for (int64_t n = 0; n < N; n++) {
            const double* w = wv + n * K;
            double acc = 0.0, accabs = 0.0;
            for (int64_t k = 0; k < K; k++) {
                acc += av[k] * w[k];
                accabs += fabs(av[k] * w[k]);
            }
            y[m * N + n] = acc;
            if (yabs) yabs[m * N + n] = accabs;
        }
        free(av);
    }
    free(wv);
}

/* ------------------------------------------------------------------------------------------ fused producers */
/* kernels/quant.py:144-170 (norm_q8), :249-280 (swiglu_q8), :354-366 / :384-393 (norm_g, swiglu_g), storing as
 * :287-309 (one scale per row) or _store_g :314-330 (per 256 inputs, or one per row, plus split per-32 sums).
 * The reference evaluates rsqrt, exp and '/' with NVIDIA's approximate instructions in Triton's reduction order; this
 * build defines them exactly (the GPU library does the same steps):
 *   exp(x):  n = rint(RN(x log2 e)), r = fma(-n, LN2_HI, x), r = fma(-n, LN2_LO, r) (Cody-Waite), Taylor series of
 *            e^r to degree 7 by Horner with fma, times 2^n (ldexp);
 *   rmsnorm: the sum of RN(h*h) over a row in the order of a 256-thread workgroup - thread t adds inputs
 *            8 (t + 256 c) + j (c, then j increasing), the 64 threads of each wave combine by halving, the four wave
 *            sums left to right; r = RN(1 / RN(sqrt(RN(RN(ss / HID) + eps)))), y = RN(RN(h r) w);
 *   silu:    RN(g / RN(1 + exp(-g))), y = RN(RN(silu(g) u) inv_s). */
EXPORT float orc_expf(float x) {
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.97208404541016f) return 0.f;
    const float n = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.428606765330187045e-06f, r);
    float p = 1.98412701e-04f;
    p = fmaf(p, r, 1.38888892e-03f);
    p = fmaf(p, r, 8.33333377e-03f);
    p = fmaf(p, r, 4.16666679e-02f);
    p = fmaf(p, r, 1.66666672e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* the workgroup's fixed-order sum of squares of y[0..K) */
EXPORT float orc_sumsq_fixed(const float* y, int64_t K) {
    float part[256];
    const int64_t nch = K / 8;
    for (int t = 0; t < 256; t++) {
        float acc = 0.f;
        for (int64_t idx = t; idx < nch; idx += 256)
            for (int j = 0; j < 8; j++) {
                const float v = y[idx * 8 + j];
                acc = acc + v * v;
            }
        part[t] = acc;
    }
    float wsum[4];
    for (int w = 0; w < 4; w++) {
        float a[64];
        for (int l = 0; l < 64; l++) a[l] = part[64 * w + l];
        for (int o = 32; o > 0; o >>= 1)
            for (int l = 0; l < o; l++) a[l] = a[l] + a[l + o];
        wsum[w] = a[0];
    }
    return ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
}

/* y [K] -> back 0: q int8 [K] at row, s[row]; back 1: q, a [K/256, M] at (b, row), xs [K/256, M, 16]; back 2: one
 * scale per row in a[row]. */
static void store_back_row(const float* y, int64_t K, int back, int64_t M, int64_t row, int8_t* q, float* s,
                           int8_t* xs) {
    const int64_t G = back == 1 ? 256 : K;
    for (int64_t g0 = 0; g0 < K; g0 += G) {
        float amax = 0.f;
        for (int64_t k = g0; k < g0 + G; k++) amax = fmaxf(amax, fabsf(y[k]));
        const float scale = fmaxf(amax, 1e-10f) / 127.0f;
        for (int64_t k = g0; k < g0 + G; k++) q[row * K + k] = (int8_t)(int)rintf(y[k] / scale);
        if (back == 1) s[(g0 / 256) * M + row] = scale;
        else s[row] = scale;
    }
    if (back != 0)
        for (int64_t sb = 0; sb < K / 32; sb++) {
            int sum = 0;
            for (int k = 0; k < 32; k++) sum += q[row * K + sb * 32 + k];
            xs[((sb / 8) * M + row) * 16 + sb % 8] = (int8_t)(sum & 63);
            xs[((sb / 8) * M + row) * 16 + 8 + sb % 8] = (int8_t)(sum >> 6);
        }
}

EXPORT void orc_norm_quant(const float* h, int64_t HID, const float* w, const int32_t* rows, int64_t M, float eps,
                           int back, int64_t live, int8_t* q, float* s, int8_t* xs, int nthreads) {
    const int64_t n = live < M ? live : M;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const float* hr = h + (rows ? (int64_t)rows[i] : i) * HID;
        float* y = (float*)malloc(sizeof(float) * HID);
        const float ss = orc_sumsq_fixed(hr, HID);
        const float r = 1.0f / sqrtf(ss / (float)HID + eps);
        for (int64_t k = 0; k < HID; k++) y[k] = (hr[k] * r) * w[k];
        store_back_row(y, HID, back, M, i, q, s, xs);
        free(y);
    }
}

/* The fixed-order sum of squares of one head of D values (the GPU kernel's order): each 8-value chunk summed in
 * increasing index, then the D / 8 chunk sums combined by halving (chunk c + chunk c + D/16, then + D/32, ...). */
EXPORT float orc_head_sumsq(const float* y, int64_t D) {
    float a[64];
    const int64_t n = D / 8;
    for (int64_t c = 0; c < n; c++) {
        float acc = 0.f;
        for (int j = 0; j < 8; j++) acc = acc + y[c * 8 + j] * y[c * 8 + j];
        a[c] = acc;
    }
    for (int64_t o = n / 2; o > 0; o >>= 1)
        for (int64_t l = 0; l < o; l++) a[l] = a[l] + a[l + o];
    return a[0];
}

/* Gated RMSNorm per head (StartLux-Prism kernels/quant.py:216-246 _gated_norm_q8_kernel, :349-365 _gated_norm_g_kernel):
 * o fp32 [M, HV D], z fp32 [M, ldz] (bf16 inputs widened exactly; the HV D gate values from column 0), w fp32 [D],
 * inv_s fp32 [HV D] or NULL.  y = RN(RN(RN(o r) w) silu(z)) (then RN(y inv_s)) with r per head, as norm_quant. */
EXPORT void orc_gated_norm_quant(const float* o, const float* z, int64_t ldz, const float* w, const float* inv_s,
                                 int64_t M, int64_t HV, int64_t D, float eps, int back, int64_t live, int8_t* q,
                                 float* s, int8_t* xs, int nthreads) {
    const int64_t n = live < M ? live : M, K = HV * D;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        float* y = (float*)malloc(sizeof(float) * K);
        for (int64_t hh = 0; hh < HV; hh++) {
            const float* oh = o + i * K + hh * D;
            const float ss = orc_head_sumsq(oh, D);
            const float r = 1.0f / sqrtf(ss / (float)D + eps);
            for (int64_t d = 0; d < D; d++) {
                const float g = z[i * ldz + hh * D + d];
                float v = ((oh[d] * r) * w[d]) * (g / (1.0f + orc_expf(-g)));
                if (inv_s) v = v * inv_s[hh * D + d];
                y[hh * D + d] = v;
            }
        }
        store_back_row(y, K, back, M, i, q, s, xs);
        free(y);
    }
}

/* gu fp32 [M, 2 FF] (bf16 inputs widened exactly) */
EXPORT void orc_swiglu_quant(const float* gu, int64_t FF, const float* inv_s, int64_t M, int back, int64_t live,
                             int8_t* q, float* s, int8_t* xs, int nthreads) {
    const int64_t n = live < M ? live : M;
#pragma omp parallel for num_threads(nthreads_or(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        float* y = (float*)malloc(sizeof(float) * FF);
        for (int64_t k = 0; k < FF; k++) {
            const float g = gu[i * 2 * FF + k], u = gu[i * 2 * FF + FF + k];
            float v = (g / (1.0f + orc_expf(-g))) * u;
            if (inv_s) v = v * inv_s[k];
            y[k] = v;
        }
        store_back_row(y, FF, back, M, i, q, s, xs);
        free(y);
    }
}
