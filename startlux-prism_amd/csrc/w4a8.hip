// W4A8 GEMM on Q4_K weights (gfx950): int8 activations x 4-bit k-quant weights on int8 MFMA.
//
// Arithmetic (StartLux-Prism kernels/w4a8.py:14-22, gemm_ref :177-199), per output (m, n), super-blocks b of 256
// inputs in increasing b:
//   acc  = sum_g sc[n,b,g] (xq . q)_g        int32, exact (the scales enter the MFMA's weight operand, two_plane)
//   mins = sum_g mn[n,b,g] S[m, 8b + g]       int32, exact (S: the activation sums per 32 inputs)
//   t = RN(d[n,b] float(acc));  t = fma(-dmin[n,b], float(mins), t);  y = fma(a[b,m], t, y)
// then bf16(y) (epi 0) or out = RN(out + y) (epi 1).  y's chain over b is kept in super-block order by every kernel.
//
// Device layout (prism_q4k_pack, made once at load from the GGUF block_q4_K bytes, as the reference's repack is:
// kernels/w4a8.py:70-94): a byte permutation of the GGUF blocks, 144 bytes per row and super-block.
//   qv   uint8 [N/16][K/256][2][64][16]: per (16-row tile nt, super-block b) 2 KB.  Half h, lane slot l (row
//        r = l % 16, q = l / 16), byte j: pair p = 2 h + j / 8 of sub-blocks, t = j % 8, k0 = 64 p + 16 q + t (input
//        index in the super-block), the byte is v[k0] | v[k0 + 8] << 4 for row 16 nt + r.  A lane's 8 bytes of pair
//        p unpack with two masks into the 16-byte MFMA operand for inputs 64 p + 16 q .. + 15 of the super-block,
//        the activation operand being those 16 bytes as they lie in the row (one 16-byte read).
//   meta uint8 [N/16][K/256][16][16]: per row the GGUF block's first 16 bytes: d, dmin (fp16) and the 12 bytes of
//        6-bit scales and mins (ggml get_scale_min_k4 order, gguf_weights.py:56-60).
// Activations: xq int8 [M, K] row-major; a fp32, (b, m) at a[b a_sb + m] (a_sb = 0: one scale per token);
// xs int8 [K/256, M, 16]: per super-block the eight S & 63 then the eight S >> 6 (kernels/quant.py:314-330).
#include "common.h"
#include "w4a8_bal.h"
#include "w4a8_common.h"
#include "w4a8_prefill.h"

#ifndef Q4S_TG2_ROWS
#define Q4S_TG2_ROWS 5
#endif

namespace prism {

// ---------------------------------------------------------------------------------------------- pack
// One thread per (nt, b, h, l): gathers 4 sub-blocks x 4 bytes from the GGUF block of row 16 nt + l % 16.
__global__ __launch_bounds__(256) void q4k_pack_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ qv,
                                                       uint8_t* __restrict__ meta, int N, int K) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int NB = K / 256;
    const int64_t total = (int64_t)(N / 16) * NB * 128;
    if (e >= total) return;
    const int l = (int)(e & 63), h = (int)((e >> 6) & 1);
    const int64_t c = e >> 7;                          // (nt, b)
    const int b = (int)(c % NB), nt = (int)(c / NB);
    const int r = l & 15, q = l >> 4;
    const uint8_t* blk = raw + ((int64_t)(16 * nt + r) * NB + b) * 144;
    const uint8_t* qs = blk + 16;                      // 128 bytes: 32-byte group c holds sub-block 2 c (low
    uint32_t o[4] = {0, 0, 0, 0};                      // nibbles) and 2 c + 1 (high nibbles)
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int k = 128 * h + 64 * (j >> 3) + 16 * q + (j & 7);     // this byte: values k and k + 8
        const uint32_t v0 = (qs[32 * (k >> 6) + (k & 31)] >> (4 * ((k >> 5) & 1))) & 0xf;
        const uint32_t v1 = (qs[32 * ((k + 8) >> 6) + ((k + 8) & 31)] >> (4 * (((k + 8) >> 5) & 1))) & 0xf;
        o[j >> 2] |= (v0 | (v1 << 4)) << (8 * (j & 3));
    }
    reinterpret_cast<v4u*>(qv)[e] = v4u{o[0], o[1], o[2], o[3]};
    if (h == 0 && q == 0) {                            // blocks are 144 bytes: 16-byte aligned, copy by words
        const uint32_t* s32 = reinterpret_cast<const uint32_t*>(blk);
        reinterpret_cast<v4u*>(meta)[c * 16 + r] = v4u{s32[0], s32[1], s32[2], s32[3]};
    }
}

// Q6_K value v (0..255) of a block_q6_K (ggml's layout, gguf_weights.py:85-97): low 4 bits from ql, high 2 from qh,
// minus 32.
__device__ __forceinline__ int q6k_val(const uint8_t* blk, int v) {
    const int h = v >> 7, i = (v >> 5) & 3, l = v & 31;
    const uint32_t lq = blk[64 * h + 32 * (i & 1) + l];
    const uint32_t lo = (i < 2) ? (lq & 15) : (lq >> 4);
    const uint32_t hi = (blk[128 + 32 * h + l] >> (2 * i)) & 3;
    return (int)(lo | (hi << 4)) - 32;
}

// One thread per (nt, b, j, l): the 16 bytes of lane l = 16 q + r, chunk j of the Q6_K device layout.
__global__ __launch_bounds__(256) void q6k_pack_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ qv,
                                                       uint8_t* __restrict__ meta, int N, int K) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int NB = K / 256;
    const int64_t total = (int64_t)(N / 16) * NB * 256;
    if (e >= total) return;
    const int l = (int)(e & 63), j = (int)((e >> 6) & 3);
    const int64_t c = e >> 8;                          // (nt, b)
    const int b = (int)(c % NB), nt = (int)(c / NB);
    const int r = l & 15, q = l >> 4;
    const uint8_t* blk = raw + ((int64_t)(16 * nt + r) * NB + b) * 210;
    uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 16; t++) {
        const int k = 32 * (2 * j + (t >> 3)) + 8 * q + (t & 7);
        o[t >> 2] |= ((uint32_t)q6k_val(blk, k) & 0xffu) << (8 * (t & 3));
    }
    reinterpret_cast<v4u*>(qv)[e] = v4u{o[0], o[1], o[2], o[3]};
    if (j == 0 && q == 0) {                            // 210-byte blocks: copy by bytes
        uint8_t* m = meta + c * Q6_META;
#pragma unroll
        for (int t = 0; t < 16; t++) m[16 * r + t] = blk[192 + t];
        m[256 + 2 * r] = blk[208];
        m[256 + 2 * r + 1] = blk[209];
    }
}

// ---------------------------------------------------------------------------------------------- Q6_K decode
// Q6_K (prism_q6k_pack).  A workgroup owns TG adjacent 16-row tiles, NW waves each, and every activation row
// (M <= 16), staged once for its TG tiles.  Round r covers R super-blocks; wave w of a tile computes super-blocks
// r R + w CB .. + CB - 1.  Per round the per-wave global loads
// are the weight chunks (4 KB per super-block: four dwordx4 per lane, requested D - 1 rounds ahead).  The round's
// scales (unpacked once per row and super-block by a staging thread), activation rows and activation scales are
// fetched with 16-byte loads a round ahead and staged in one of two LDS buffers.  Each super-block's term t of each
// output goes to one of two LDS term buffers; the owner thread of each output folds round r - 1's terms,
// y = fma(a[b, m], t, y) in super-block order, while round r is computed; one barrier per round.
template <int NW, int R, int MX, int D, int TG, int EPI>
__global__ __launch_bounds__(NW * TG * 64, 2) void w4a8_q6k_decode_kernel(const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ a, int64_t a_sb,
                                                                  const uint8_t* __restrict__ qv,
                                                                  const uint8_t* __restrict__ meta,
                                                                  void* __restrict__ out, int64_t ldo,
                                                                  const int32_t* __restrict__ n_rows, int M, int N,
                                                                  int K) {
    constexpr int NT = NW * TG * 64;
    constexpr int CB = R / NW;                     // super-blocks per wave per round
    static_assert(CB >= 1 && CB * NW == R, "R must be a multiple of NW");
    static_assert(MX <= 16 && TG * R * 16 <= NT && R * MX <= NT, "one staging thread per (tile, row, super-block)");
    constexpr int RB = R * 256;                    // activation bytes per row per round
    constexpr int LDA = RB + 16;
    constexpr int CPR = RB / 16;
    constexpr int XPT = (MX * CPR + NT - 1) / NT;
    constexpr int WCH = 4;                         // 16-byte weight chunks per lane and super-block
    extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
    // LDS (q6k_decode_lds): terms, per window the second scale and the first minus the second, d, activations and
    // activation scales
    float* terms = reinterpret_cast<float*>(dsm);                 // [TG][2][R][M][16]
    int* sca = reinterpret_cast<int*>(terms + TG * 2 * R * M * 16);  // [TG][2][R][8][16] [window][row]
    int* scb = sca + TG * 2 * R * 128;                            // [TG][2][R][8][16]
    float* dl = reinterpret_cast<float*>(scb + TG * 2 * R * 128);  // [TG][2][R][16]
    int8_t* xl = reinterpret_cast<int8_t*>(dl + TG * 2 * R * 16);  // [2][M][LDA]
    float* al = reinterpret_cast<float*>(xl + 2 * M * LDA);       // [3][R][M] activation scales: read by the fold of
                                                                  // round r - 1 while round r + 1 is staged
    const int tstride = R * M * 16, xstride = M * LDA;

    kernel_args_now(xq, a, a_sb, qv, meta, out, ldo, n_rows, M, N, K);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wt = tid >> 6, tg = wt / NW, wv = wt - tg * NW;      // wave wv of tile tg
    const int nt0 = blockIdx.x * TG;
    const int live = min(M, __ldg(n_rows));
    const int NB = K / 256;
    const int nr = (NB + R - 1) / R;
    const int lm = lane & 15, q = lane >> 4;
    const int xch = M * CPR;

    const v4u* cw = reinterpret_cast<const v4u*>(qv) + (int64_t)(nt0 + tg) * NB * 64 * WCH + lane;
    const uint8_t* cm6 = meta + (int64_t)nt0 * NB * Q6_META;

    struct Staged {
        v4u m;        // thread < 16 R TG: tile tid / 16 R, super-block tid / 16 % R, row tid % 16: its 16 scales
        uint32_t dh;  // the row's fp16 d
        float as;     // thread < R M: activation scale of (super-block tid / M, row tid % M)
        v4i x[XPT];
    };
    auto stage_load = [&](int r, Staged& sg) {
        const int b0 = r * R;
        const int c = min(tid, 16 * R * TG - 1), cg = c / (16 * R), cl = c - cg * 16 * R;
        const uint8_t* mp = cm6 + ((int64_t)cg * NB + min(b0 + cl / 16, NB - 1)) * Q6_META;
        sg.m = reinterpret_cast<const v4u*>(mp)[c & 15];
        sg.dh = reinterpret_cast<const uint16_t*>(mp + 256)[c & 15];
        const int e = min(tid, R * M - 1);
        const int bb = min(b0 + e / M, NB - 1), mm = e % M;
        sg.as = a[(int64_t)bb * a_sb + mm];
        const int64_t k0 = (int64_t)r * RB;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int cc = min(tid + i * NT, xch - 1);
            const int64_t kk = min(k0 + (cc % CPR) * 16, (int64_t)K - 16);
            sg.x[i] = *reinterpret_cast<const v4i*>(xq + (int64_t)(cc / CPR) * K + kk);
        }
    };
    auto stage_store = [&](const Staged& sg, int rr) {
        const int buf = rr & 1;
        if (tid < 16 * R * TG) {
            const int sg_t = tid / (16 * R), lb = (tid >> 4) % R, row = tid & 15;
            int* pa = sca + ((sg_t * 2 + buf) * R + lb) * 128 + row;
            int* pb = scb + ((sg_t * 2 + buf) * R + lb) * 128 + row;
#pragma unroll
            for (int w = 0; w < 8; w++) {
                const int s0 = sbyte(sg.m, 2 * w), s1 = sbyte(sg.m, 2 * w + 1);
                pa[16 * w] = s1;
                pb[16 * w] = s0 - s1;
            }
            dl[((sg_t * 2 + buf) * R + lb) * 16 + row] = f16_to_f32(sg.dh);
        }
        if (tid < R * M) al[(rr % 3) * R * M + tid] = sg.as;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int cc = tid + i * NT;
            if (cc < xch) *reinterpret_cast<v4i*>(&xl[buf * xstride + (cc / CPR) * LDA + (cc % CPR) * 16]) = sg.x[i];
        }
    };
    auto load_w = [&](int r, v4u (*w)[WCH]) {
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int64_t b = min(r * R + wv * CB + i, NB - 1);
#pragma unroll
            for (int j = 0; j < WCH; j++) w[i][j] = __builtin_nontemporal_load(cw + b * 64 * WCH + 64 * j);
        }
    };
    auto compute = [&](int r, v4u (*w)[WCH], int buf) {
        float* tb = terms + (tg * 2 + (r & 1)) * tstride;
        const int mrow = min(lm, M - 1);
        const int8_t* xrow = xl + buf * xstride + mrow * LDA;
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int lb = wv * CB + i;
            if (r * R + lb < NB) {
                // per 32-input window: P over both sub-blocks, Pl over the first (activations of lanes q >= 2,
                // which hold the second, zeroed): acc += sc1 P + (sc0 - sc1) Pl
                const int* pa = sca + ((tg * 2 + buf) * R + lb) * 128 + 4 * q;
                const int* pb = scb + ((tg * 2 + buf) * R + lb) * 128 + 4 * q;
                v4i acc = {0, 0, 0, 0};
                const v4i zero = {0, 0, 0, 0};
#pragma unroll
                for (int wn = 0; wn < 8; wn++) {
                    const v4u& c16 = w[i][wn >> 1];
                    const int64_t wf = (int64_t)c16[2 * (wn & 1)] | ((int64_t)c16[2 * (wn & 1) + 1] << 32);
                    const int64_t af = *reinterpret_cast<const int64_t*>(xrow + lb * 256 + 32 * wn + 8 * q);
                    const v4i P = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf, af, zero, 0, 0, 0);
                    const v4i Pl = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf, q < 2 ? af : 0, zero, 0, 0, 0);
                    const v4i A = *reinterpret_cast<const v4i*>(pa + 16 * wn), B = *reinterpret_cast<const v4i*>(pb + 16 * wn);
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[e] += __mul24(A[e], P[e]) + __mul24(B[e], Pl[e]);
                }
                const v4f d = *reinterpret_cast<const v4f*>(&dl[((tg * 2 + buf) * R + lb) * 16 + 4 * q]);
                v4f t;
#pragma unroll
                for (int e = 0; e < 4; e++) t[e] = mul_rn(d[e], (float)acc[e]);
                if (lm < M) *reinterpret_cast<v4f*>(&tb[(lb * M + lm) * 16 + 4 * q]) = t;
            }
        }
    };
    float y = 0.f;
    // output fo of tile fg (m = fo / 16, n = 16 (nt0 + fg) + fo % 16): thread tid < TG M 16
    const int fg = tid / (M * 16), fo = tid - fg * M * 16;
    auto fold = [&](int r) {
        if (fg < TG) {
            const float* tb = terms + (fg * 2 + (r & 1)) * tstride;
            const float* ap = al + (r % 3) * R * M + (fo >> 4);
            const int nb = min(R, NB - r * R);
            float acc = y;
            for (int j = 0; j < nb; j++) acc = fmaf(ap[j * M], tb[j * M * 16 + fo], acc);
            y = acc;
        }
    };

    v4u wr[D][CB][WCH];
    Staged sg;
#pragma unroll
    for (int d = 0; d < D - 1; d++) load_w(d, wr[d]);
    stage_load(0, sg);
    stage_store(sg, 0);
    stage_load(1, sg);
    lds_barrier();
    for (int r0 = 0; r0 < nr; r0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int r = r0 + d;
            load_w(r + D - 1, wr[(d + D - 1) % D]);        // past the end: the last chunk again (a cache hit)
            stage_store(sg, r + 1);
            stage_load(r + 2, sg);
            if (r < nr) compute(r, wr[d], r & 1);
            if (r >= 1 && r <= nr) fold(r - 1);
            lds_barrier();
        }
    }
    if (nr % D == 0) fold(nr - 1);
    const int m = fo >> 4, n = 16 * (nt0 + fg) + (fo & 15);
    if (fg < TG && m < live) {
        if (EPI == 0) {
            reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = (uint16_t)f32_to_bf16(y);
        } else {
            float* op = reinterpret_cast<float*>(out) + (int64_t)m * ldo + n;
            *op = add_rn(*op, y);
        }
    }
}

static size_t q6k_decode_lds(int R, int M, int TG) {
    return TG * (2 * (size_t)R * M * 16 * 4 + 2 * 2 * (size_t)R * 128 * 4 + 2 * (size_t)R * 16 * 4) +
           2 * (size_t)M * (R * 256 + 16) + 3 * (size_t)R * M * 4;
}

// ---------------------------------------------------------------------------------------------- Q4_K stream decode
// Up to 16 activation rows; one workgroup per TG adjacent 16-row weight tiles and all of K.  Wave w computes
// super-blocks w, w + NW, ... of every tile with PD of them in flight in a register ring, each holding what its lane
// needs from memory: per tile the 2 KB of weights (two 16-byte slots) and the 16 meta bytes of the lane's weight row,
// and once for the TG tiles the lane's activation row (four 16-byte pieces) and its split activation sums.  A
// super-block's term t of each output (the two-plane MFMA sums, the mins on the MFMA, q4k_term) goes to LDS
// [tile][b][m][n]; after one barrier each output's thread adds the terms in super-block order, y = fma(a[b, m], t, y),
// as the reference's sequential chain does.  Two tiles per wave halve the activation requests, which at 16 rows are
// twice the weight bytes (every tile reads every activation row).
template <int NW, int PD, int TG, int EPI>
__global__ __launch_bounds__(NW * 64) void w4a8_q4k_stream_kernel(const int8_t* __restrict__ xq,
                                                                 const float* __restrict__ a, int64_t a_sb,
                                                                 const int8_t* __restrict__ xs,
                                                                 const uint8_t* __restrict__ qv,
                                                                 const uint8_t* __restrict__ meta,
                                                                 void* __restrict__ out, int64_t ldo,
                                                                 const int32_t* __restrict__ n_rows, int M, int K) {
    extern __shared__ __attribute__((aligned(16))) float tl[];          // [TG][NB][M][16]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nt0 = blockIdx.x * TG;
    const int NB = K / 256;
    const int lm = lane & 15, q = lane >> 4;
    const int m = min(lm, M - 1);

    const v4u* cw = reinterpret_cast<const v4u*>(qv) + (int64_t)nt0 * NB * 128 + lane;
    kernel_args_now(xq, a, a_sb, xs, qv, meta, out, ldo, n_rows, M, K);
    const v4u* cm = reinterpret_cast<const v4u*>(meta) + (int64_t)nt0 * NB * 16 + lm;
    const int8_t* cx = xq + (int64_t)m * K + 16 * q;
    struct SB {
        v4u w[TG][2];
        v4u mt[TG];
        v4i x[4];
        v4i s;
    };
    auto load = [&](int i, SB& c) {
        const int b = min(wv + NW * i, NB - 1);
#pragma unroll
        for (int g = 0; g < TG; g++) {
            c.w[g][0] = __builtin_nontemporal_load(cw + ((int64_t)g * NB + b) * 128);
            c.w[g][1] = __builtin_nontemporal_load(cw + ((int64_t)g * NB + b) * 128 + 64);
            c.mt[g] = cm[((int64_t)g * NB + b) * 16];
        }
#pragma unroll
        for (int p = 0; p < 4; p++) c.x[p] = *reinterpret_cast<const v4i*>(cx + (int64_t)b * 256 + 64 * p);
        c.s = *reinterpret_cast<const v4i*>(xs + ((int64_t)b * M + m) * 16);
    };
    auto term = [&](int i, const SB& c) {
        const int b = wv + NW * i;
        const int64_t slo = q == 0 ? ((int64_t)(uint32_t)c.s[0] | ((int64_t)(uint32_t)c.s[1] << 32)) : 0;
        const int64_t shi = q == 0 ? ((int64_t)(uint32_t)c.s[2] | ((int64_t)(uint32_t)c.s[3] << 32)) : 0;
#pragma unroll
        for (int g = 0; g < TG; g++) {
            // this lane's weight row lm of tile g: d, dmin and its four sub-blocks' split scales
            const float d = f16_to_f32(c.mt[g][0] & 0xffffu), dm = f16_to_f32(c.mt[g][0] >> 16);
            uint32_t sp[4];
            q4k_lane_splits(c.mt[g], q >> 1, sp);
            v4i alo = {0, 0, 0, 0}, ahi = {0, 0, 0, 0};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                v4i wl, wh;
                two_plane(c.w[g][p >> 1][2 * (p & 1)], c.w[g][p >> 1][2 * (p & 1) + 1], sp[p], wl, wh);
                alo = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl, c.x[p], alo, 0, 0, 0);
                ahi = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh, c.x[p], ahi, 0, 0, 0);
            }
            const int64_t mn8 = q == 0 ? q4k_mins8(c.mt[g]) : 0;
            const v4i mins = mins_mfma(mn8, slo, shi);
            v4f t;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float de = __shfl(d, 4 * q + e, kWave), dme = __shfl(dm, 4 * q + e, kWave);   // row 4 q + e
                t[e] = q4k_term(de, dme, alo[e] + 8 * ahi[e], mins[e]);
            }
            if (lm < M && b < NB) *reinterpret_cast<v4f*>(&tl[(((int64_t)g * NB + b) * M + lm) * 16 + 4 * q]) = t;
        }
    };
    const int cnt = wv < NB ? (NB - wv + NW - 1) / NW : 0;
    SB ring[PD];
#pragma unroll
    for (int d = 0; d < PD; d++) load(d, ring[d]);
    const int full = cnt / PD * PD;
    for (int i0 = 0; i0 < full; i0 += PD) {
#pragma unroll
        for (int d = 0; d < PD; d++) {
            term(i0 + d, ring[d]);
            load(i0 + d + PD, ring[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < PD; d++)
        if (full + d < cnt) term(full + d, ring[d]);
    __syncthreads();
    // the live-row count only here (read earlier, its load would precede the first weight requests)
    const int live = min(M, __ldg(n_rows));
    for (int fo = tid; fo < TG * M * 16; fo += NW * 64) {
        const int g = fo / (M * 16), f = fo - g * M * 16;
        const int mo = f >> 4, n = 16 * (nt0 + g) + (f & 15);
        if (mo >= live) continue;
        float y = 0.f;
        for (int b = 0; b < NB; b++)
            y = fmaf(a[(int64_t)b * a_sb + mo], tl[(((int64_t)g * NB + b) * M + mo) * 16 + (f & 15)], y);
        if (EPI == 0) {
            reinterpret_cast<uint16_t*>(out)[(int64_t)mo * ldo + n] = (uint16_t)f32_to_bf16(y);
        } else {
            float* op = reinterpret_cast<float*>(out) + (int64_t)mo * ldo + n;
            *op = add_rn(*op, y);
        }
    }
}

// ---------------------------------------------------------------------------------------------- Q6_K stream decode
// The Q4_K stream kernel's structure on Q6_K weights (prism_q6k_pack): per super-block a lane holds the tile's 4 KB
// of weights (four 16-byte slots), the 16 int8 scales of its four output rows 4 q .. 4 q + 3, their fp16 d, and the
// eight 8-byte activation pieces of its row.  Per 32-input window, P over both sub-blocks and Pl over the first
// (activations of lanes q >= 2, which hold the second, zeroed): acc += sc1 P + (sc0 - sc1) Pl, exact; then
// t = RN(d float(acc)) to LDS, and the ordered fold y = fma(a[b, m], t, y) after one barrier.  About three times the
// staged kernel's loads per weight byte: faster only for some shapes at a few rows, so the dispatch table picks it
// ("stream") where it measured faster.
template <int NW, int PD, int EPI>
__global__ __launch_bounds__(NW * 64) void w4a8_q6k_stream_kernel(const int8_t* __restrict__ xq,
                                                                 const float* __restrict__ a, int64_t a_sb,
                                                                 const uint8_t* __restrict__ qv,
                                                                 const uint8_t* __restrict__ meta,
                                                                 void* __restrict__ out, int64_t ldo,
                                                                 const int32_t* __restrict__ n_rows, int M, int K) {
    extern __shared__ __attribute__((aligned(16))) float tl[];          // [NB][M][16]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nt = blockIdx.x;
    const int live = min(M, __ldg(n_rows));
    const int NB = K / 256;
    const int lm = lane & 15, q = lane >> 4;
    const int m = min(lm, M - 1);

    const v4u* cw = reinterpret_cast<const v4u*>(qv) + (int64_t)nt * NB * 256 + lane;
    kernel_args_now(xq, a, a_sb, qv, meta, out, ldo, n_rows, M, K);
    const uint8_t* cm = meta + (int64_t)nt * NB * Q6_META;
    const int8_t* cx = xq + (int64_t)m * K + 8 * q;
    struct SB {
        v4u w[4];
        v4u sc[4];
        v2u dh;
        v2u x[8];
    };
    auto load = [&](int i, SB& c) {
        const int b = min(wv + NW * i, NB - 1);
#pragma unroll
        for (int j = 0; j < 4; j++) c.w[j] = __builtin_nontemporal_load(cw + (int64_t)b * 256 + 64 * j);
        const uint8_t* mp = cm + (int64_t)b * Q6_META;
#pragma unroll
        for (int e = 0; e < 4; e++) c.sc[e] = reinterpret_cast<const v4u*>(mp)[4 * q + e];
        c.dh = *reinterpret_cast<const v2u*>(mp + 256 + 8 * q);
#pragma unroll
        for (int wn = 0; wn < 8; wn++) c.x[wn] = *reinterpret_cast<const v2u*>(cx + (int64_t)b * 256 + 32 * wn);
    };
    auto term = [&](int i, const SB& c) {
        const int b = wv + NW * i;
        const v4i zero = {0, 0, 0, 0};
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int wn = 0; wn < 8; wn++) {
            const v4u& c16 = c.w[wn >> 1];
            const int64_t wf = (int64_t)c16[2 * (wn & 1)] | ((int64_t)c16[2 * (wn & 1) + 1] << 32);
            const int64_t af = (int64_t)(uint32_t)c.x[wn][0] | ((int64_t)c.x[wn][1] << 32);
            const v4i P = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf, af, zero, 0, 0, 0);
            const v4i Pl = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf, q < 2 ? af : 0, zero, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int s0 = sbyte(c.sc[e], 2 * wn), s1 = sbyte(c.sc[e], 2 * wn + 1);
                acc[e] += __mul24(s1, P[e]) + __mul24(s0 - s1, Pl[e]);
            }
        }
        v4f t;
#pragma unroll
        for (int e = 0; e < 4; e++)
            t[e] = mul_rn(f16_to_f32((e & 1) ? (c.dh[e >> 1] >> 16) : (c.dh[e >> 1] & 0xffffu)), (float)acc[e]);
        if (lm < M && b < NB) *reinterpret_cast<v4f*>(&tl[((int64_t)b * M + lm) * 16 + 4 * q]) = t;
    };
    const int cnt = wv < NB ? (NB - wv + NW - 1) / NW : 0;
    SB ring[PD];
#pragma unroll
    for (int d = 0; d < PD; d++) load(d, ring[d]);
    const int full = cnt / PD * PD;
    for (int i0 = 0; i0 < full; i0 += PD) {
#pragma unroll
        for (int d = 0; d < PD; d++) {
            term(i0 + d, ring[d]);
            load(i0 + d + PD, ring[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < PD; d++)
        if (full + d < cnt) term(full + d, ring[d]);
    __syncthreads();
    for (int fo = tid; fo < M * 16; fo += NW * 64) {
        const int mo = fo >> 4, n = 16 * nt + (fo & 15);
        if (mo >= live) continue;
        float y = 0.f;
        for (int b = 0; b < NB; b++) y = fmaf(a[(int64_t)b * a_sb + mo], tl[((int64_t)b * M + mo) * 16 + (fo & 15)], y);
        if (EPI == 0) {
            reinterpret_cast<uint16_t*>(out)[(int64_t)mo * ldo + n] = (uint16_t)f32_to_bf16(y);
        } else {
            float* op = reinterpret_cast<float*>(out) + (int64_t)mo * ldo + n;
            *op = add_rn(*op, y);
        }
    }
}

// ---------------------------------------------------------------------------------------------- prefill tile
// 128 (n) x 64 (m) output tile per 256-thread workgroup: 4 waves, each 32 n x 64 m (2 x 4 MFMA tiles of 16 x 16),
// one super-block per stage, two stage buffers in LDS.  The stage's weight chunks (8 row tiles x 2 KB) and activation
// rows (64 x 256 B) arrive by LDS-DMA into the free buffer while the other is computed; the tile's meta (unpacked
// once per row by a staging thread), activation sums and scales go through registers.  One barrier per stage.
// Activation row r holds its 16-byte chunk c at slot c ^ (r & 15): the 16 rows a 16-lane read spans fall in distinct
// banks.  Each wave keeps its outputs' fp32 sums y over super-blocks.
constexpr int QBN = 128, QBM = 64;

template <int EPI>
__global__ __launch_bounds__(256, 2) void w4a8_tile_kernel(const int8_t* __restrict__ xq, const float* __restrict__ a,
                                                           int64_t a_sb, const int8_t* __restrict__ xs,
                                                           const uint8_t* __restrict__ qv,
                                                           const uint8_t* __restrict__ meta, void* __restrict__ out,
                                                           int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                           int N, int K, int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][8 * 2048];  // 8 row tiles x (2 halves x 64 lanes x 16 B)
    __shared__ __attribute__((aligned(16))) int8_t As[2][QBM * 256];  // swizzled activation rows
    __shared__ uint32_t scl[2][8][QBN];                               // split scales, [sub-block][weight row]
    __shared__ __attribute__((aligned(8))) uint8_t mnb[2][QBN][8];  // the 8 mins of each weight row, as bytes
    __shared__ float dl[2][QBN], dml[2][QBN];
    __shared__ __attribute__((aligned(16))) int8_t xsb[2][QBM][16]; // per activation row: S & 63 x 8, S >> 6 x 8
    __shared__ float al[2][QBM];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int lm = lane & 15, q = lane >> 4;
    // tile order as the W8A8 kernels: XCD-contiguous ranges, groups of 8 tile-rows of M
    int pm, pn;
    {
        const int total = tiles_m * tiles_n;
        int t = blockIdx.x;
        if ((total & 7) == 0) t = (t & 7) * (total >> 3) + (t >> 3);
        const int per_group = 8 * tiles_n, first_m = (t / per_group) * 8, gm = min(tiles_m - first_m, 8);
        pm = first_m + (t % per_group) % gm;
        pn = (t % per_group) / gm;
    }
    const int m0 = pm * QBM, n0 = pn * QBN;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int NB = K / 256, ntiles = N / 16;

    // DMA sources, chunk c = tid + 256 i: weight chunk c of the stage's 8 x 128, activation row c / 16, slot c % 16
    const uint8_t* wsrc[4];
    const int8_t* xsrc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = tid + 256 * i;
        wsrc[i] = qv + ((int64_t)min(n0 / 16 + (c >> 7), ntiles - 1) * NB * 128 + (c & 127)) * 16;
        const int r = c >> 4;
        xsrc[i] = xq + (int64_t)min(m0 + r, M - 1) * K + (((c & 15) ^ (r & 15)) * 16);
    }
    auto dma = [&](int b, int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int base = (256 * i + 64 * wv) * 16;                // this wave's 64 chunks
            dma16(wsrc[i] + (int64_t)b * 2048, &Bs[buf][base]);
            dma16(xsrc[i] + (int64_t)b * 256, &As[buf][base]);
        }
    };
    // meta: 128 rows x 16 B (threads < 128); sums and scale: one activation row each (threads < 64)
    const v4u* msrc = reinterpret_cast<const v4u*>(meta) + (int64_t)min(n0 / 16 + (tid >> 4), ntiles - 1) * NB * 16 + (tid & 15);
    const int srow = min(m0 + (tid & 63), M - 1);
    v4u rm;
    v4i rs;
    float ra;
    auto gmeta = [&](int b) {
        rm = msrc[(int64_t)b * 16];
        rs = *reinterpret_cast<const v4i*>(xs + ((int64_t)b * M + srow) * 16);
        ra = a[(int64_t)b * a_sb + srow];
    };
    auto smeta = [&](int buf) {
        if (tid < 128) {
            float d, dm;
            int sc[8], mn[8];
            row_meta(rm, d, dm, sc, mn);
#pragma unroll
            for (int g = 0; g < 8; g++) scl[buf][g][tid] = split_scale(sc[g]);
            *reinterpret_cast<v2u*>(&mnb[buf][tid][0]) =
                v2u{(uint32_t)(mn[0] | (mn[1] << 8) | (mn[2] << 16) | (mn[3] << 24)),
                    (uint32_t)(mn[4] | (mn[5] << 8) | (mn[6] << 16) | (mn[7] << 24))};
            dl[buf][tid] = d;
            dml[buf][tid] = dm;
        }
        if (tid < 64) {
            *reinterpret_cast<v4i*>(&xsb[buf][tid][0]) = rs;
            al[buf][tid] = ra;
        }
    };

    // wave wv: n rows 32 wv .. 32 wv + 31 (tiles 2 wv, 2 wv + 1), all 64 m (4 tiles)
    float y[2][4][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) y[i][j][e] = 0.f;

    gmeta(0);
    dma(0, 0);
    smeta(0);
    vm_wait<0>();
    lds_barrier();
    for (int b = 0; b < NB; b++) {
        const int cb = b & 1;
        if (b + 1 < NB) {
            gmeta(b + 1);
            dma(b + 1, cb ^ 1);
        }
        // acc = sum_g sc[n, g] P_g, two MFMA chains over the 4 sub-block pairs (two_plane): acc = lo + 8 hi
        v4i alo[2][4], ahi[2][4];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) alo[i][j] = ahi[i][j] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            v4u wq[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                wq[i] = *reinterpret_cast<const v4u*>(&Bs[cb][(2 * wv + i) * 2048 + hh * 1024 + lane * 16]);
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                const int p = 2 * hh + pp, g = 2 * p + (q >> 1);
                v4i wl[2], wh[2], af[4];
#pragma unroll
                for (int i = 0; i < 2; i++)
                    two_plane(wq[i][2 * pp], wq[i][2 * pp + 1], scl[cb][g][32 * wv + 16 * i + lm], wl[i], wh[i]);
#pragma unroll
                for (int j = 0; j < 4; j++)
                    af[j] = *reinterpret_cast<const v4i*>(&As[cb][(16 * j + lm) * 256 + (((4 * p + q) ^ lm) * 16)]);
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        alo[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl[i], af[j], alo[i][j], 0, 0, 0);
                        ahi[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh[i], af[j], ahi[i][j], 0, 0, 0);
                    }
            }
        }
        int64_t mnf[2], slo[4], shi[4];
#pragma unroll
        for (int i = 0; i < 2; i++)
            mnf[i] = q == 0 ? *reinterpret_cast<const int64_t*>(&mnb[cb][32 * wv + 16 * i + lm][0]) : 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            slo[j] = q == 0 ? *reinterpret_cast<const int64_t*>(&xsb[cb][16 * j + lm][0]) : 0;
            shi[j] = q == 0 ? *reinterpret_cast<const int64_t*>(&xsb[cb][16 * j + lm][8]) : 0;
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const v4f d = *reinterpret_cast<const v4f*>(&dl[cb][32 * wv + 16 * i + 4 * q]);
            const v4f dm = *reinterpret_cast<const v4f*>(&dml[cb][32 * wv + 16 * i + 4 * q]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const v4i mins = mins_mfma(mnf[i], slo[j], shi[j]);
                const float am = al[cb][16 * j + lm];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    y[i][j][e] = fmaf(am, q4k_term(d[e], dm[e], alo[i][j][e] + 8 * ahi[i][j][e], mins[e]), y[i][j][e]);
            }
        }
        if (b + 1 < NB) smeta(cb ^ 1);
        vm_wait<0>();
        lds_barrier();
    }
    // D element (i, j, e): n = n0 + 32 wv + 16 i + 4 q + e, m = m0 + 16 j + lm
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int m = m0 + 16 * j + lm;
            const int nb = n0 + 32 * wv + 16 * i + 4 * q;
            if (m < live && nb < N) {
                if (EPI == 0) {
                    uint32_t lo = f32_to_bf16(y[i][j][0]) | (f32_to_bf16(y[i][j][1]) << 16);
                    uint32_t hi = f32_to_bf16(y[i][j][2]) | (f32_to_bf16(y[i][j][3]) << 16);
                    uint16_t* o = reinterpret_cast<uint16_t*>(out) + (int64_t)m * ldo + nb;
                    if ((((uintptr_t)o) & 7) == 0) {
                        *reinterpret_cast<v2u*>(o) = v2u{lo, hi};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; e++) o[e] = (uint16_t)f32_to_bf16(y[i][j][e]);
                    }
                } else {
                    float* o = reinterpret_cast<float*>(out) + (int64_t)m * ldo + nb;
#pragma unroll
                    for (int e = 0; e < 4; e++) o[e] = add_rn(o[e], y[i][j][e]);
                }
            }
        }
}

// ---------------------------------------------------------------------------------------------- Q6_K prefill tile
constexpr int Q6BN = 64;

// The Q6_K prefill tile on v_mfma_i32_32x32x16_i8, whose 16 inputs are one Q6_K sub-block: no masked second MFMA.
// 64 (m) x 64 (n) per 256-thread workgroup; wave wv owns the 32 x 32 block (m rows 32 (wv & 1) .., n rows
// 32 (wv >> 1) ..).  A stage is half a super-block (8 sub-blocks): the 4 row tiles' 2 KB of packed weights and the 64
// activation rows' 128 bytes by LDS-DMA, double-buffered, 33 KB of LDS per workgroup so that four fit a CU (four
// waves per SIMD hide the MFMA-to-VALU chain).  The activations are the A operand and the weights the B operand, so
// lane l's 16 sums are all of weight row n = l % 32 (activation rows 8 i + 4 (l / 32) + e, e < 4): its sub-block scale
// is one int per sub-block, and acc += sc_h P_h is one v_mad_i32_i24 per sum and sub-block (exact: |P_h| < 2^16).
// The B operand of sub-block h is gathered from the packed chunks: lane l's 8 bytes are inputs 16 h + 8 (l / 32) ..
// + 7 of row n, which the pack keeps in chunk h / 4, lane slot 16 (2 (h & 1) + l / 32) + n % 16, half (h / 2) & 1.
// The super-block's d, scales and activation scales come through registers into LDS once per super-block.
template <int EPI>
__global__ __launch_bounds__(256, 4) void w4a8_q6k_tile32_kernel(const int8_t* __restrict__ xq,
                                                                 const float* __restrict__ a, int64_t a_sb,
                                                                 const uint8_t* __restrict__ qv,
                                                                 const uint8_t* __restrict__ meta,
                                                                 void* __restrict__ out, int64_t ldo,
                                                                 const int32_t* __restrict__ n_rows, int M, int N,
                                                                 int K, int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][4 * 2048];   // 4 row tiles x (2 chunks x 64 lanes x 16 B)
    __shared__ __attribute__((aligned(16))) int8_t As[2][QBM * 128];   // activation rows, 8 swizzled granules each
    __shared__ __attribute__((aligned(16))) v4u scs[2][Q6BN];          // per weight row: its 16 int8 scales
    __shared__ __attribute__((aligned(16))) float dl[2][Q6BN];
    __shared__ __attribute__((aligned(16))) float al[2][QBM];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int pm, pn;
    {
        const int total = tiles_m * tiles_n;
        int t = blockIdx.x;
        if ((total & 7) == 0) t = (t & 7) * (total >> 3) + (t >> 3);
        const int per_group = 8 * tiles_n, first_m = (t / per_group) * 8, gm = min(tiles_m - first_m, 8);
        pm = first_m + (t % per_group) % gm;
        pn = (t % per_group) / gm;
    }
    const int m0 = pm * QBM, n0 = pn * Q6BN;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int NB = K / 256, ntiles = N / 16, NS = 2 * NB;

    // stage s = (super-block s / 2, half s % 2): thread c = tid + 256 i (i < 2) copies weight tile c / 128's
    // 16 bytes (c % 128) of the half's 2 KB, and activation row c / 8's granule (c % 8) ^ (row % 8)
    const uint8_t* wsrc[2];
    const int8_t* xsrc[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int c = tid + 256 * i;
        wsrc[i] = qv + ((int64_t)min(n0 / 16 + (c >> 7), ntiles - 1) * NB * 256 + (c & 127)) * 16;
        const int r = c >> 3;
        xsrc[i] = xq + (int64_t)min(m0 + r, M - 1) * K + (((c & 7) ^ (r & 7)) * 16);
    }
    auto dma = [&](int st, int buf) {
        const int64_t wo = (int64_t)(st >> 1) * 4096 + (st & 1) * 2048, xo = (int64_t)st * 128;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int base = (256 * i + 64 * wv) * 16;
            dma16(wsrc[i] + wo, &Bs[buf][base]);
            dma16(xsrc[i] + xo, &As[buf][base]);
        }
    };
    // threads < 64: weight row tid's scales and d, activation row tid's scale
    const uint8_t* msrc = meta + (int64_t)min(n0 / 16 + (tid >> 4), ntiles - 1) * NB * Q6_META;
    const int srow = min(m0 + (tid & 63), M - 1);
    v4u rm;
    uint32_t rd;
    float ra;
    auto gmeta = [&](int b) {
        if (tid < 64) {
            const uint8_t* mp = msrc + (int64_t)b * Q6_META;
            rm = reinterpret_cast<const v4u*>(mp)[tid & 15];
            rd = reinterpret_cast<const uint16_t*>(mp + 256)[tid & 15];
            ra = a[(int64_t)b * a_sb + srow];
        }
    };
    auto smeta = [&](int buf) {
        if (tid < 64) {
            scs[buf][tid] = rm;
            dl[buf][tid] = f16_to_f32(rd);
            al[buf][tid] = ra;
        }
    };

    const int mb = wv & 1, nbk = wv >> 1;
    const int col = lane & 31, kh = lane >> 5;
    const int nr = 32 * nbk + col;                                     // this lane's weight row in the tile
    const int mr = 32 * mb + col;                                      // this lane's A-operand activation row
    const int bofs = (nr >> 4) * 2048 + (16 * kh + (nr & 15)) * 16;    // + chunk, slot pair and half per sub-block
    const int aofs = mr * 128 + 8 * kh;

    float y[16];
#pragma unroll
    for (int e = 0; e < 16; e++) y[e] = 0.f;
    v16i acc;

    gmeta(0);
    dma(0, 0);
    smeta(0);
    vm_wait<0>();
    lds_barrier();
    for (int st = 0; st < NS; st++) {
        const int cb = st & 1, b = st >> 1, mbuf = b & 1;
        if (st + 1 < NS) dma(st + 1, cb ^ 1);
        if (cb == 1 && b + 1 < NB) gmeta(b + 1);
        if (cb == 0) {
#pragma unroll
            for (int e = 0; e < 16; e++) acc[e] = 0;
        }
        const v4u scv = scs[mbuf][nr];
        const uint32_t sw0 = cb ? scv[2] : scv[0], sw1 = cb ? scv[3] : scv[1];   // this half's 8 scales
        const uint8_t* bp = &Bs[cb][bofs];
        const int8_t* ap = &As[cb][aofs];
        const v16i zero = {};
#pragma unroll
        for (int h = 0; h < 8; h++) {
            // local sub-block h: chunk h / 4 of the half, lane slot pair h & 1, half (h / 2) & 1
            const int64_t bf = *reinterpret_cast<const int64_t*>(bp + (h >> 2) * 1024 + (h & 1) * 512 +
                                                                 ((h >> 1) & 1) * 8);
            const int64_t af = *reinterpret_cast<const int64_t*>(ap + ((h ^ (mr & 7)) * 16));
            const v16i P = __builtin_amdgcn_mfma_i32_32x32x16_i8(af, bf, zero, 0, 0, 0);
            const int sc = (int)(int8_t)((h < 4 ? sw0 : sw1) >> (8 * (h & 3)));
#pragma unroll
            for (int e = 0; e < 16; e++) acc[e] += __mul24(sc, P[e]);
        }
        if (cb == 1) {
            const float d = dl[mbuf][nr];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const v4f am = *reinterpret_cast<const v4f*>(&al[mbuf][32 * mb + 8 * i + 4 * kh]);
#pragma unroll
                for (int e = 0; e < 4; e++) y[4 * i + e] = fmaf(am[e], mul_rn(d, (float)acc[4 * i + e]), y[4 * i + e]);
            }
            if (b + 1 < NB) smeta(mbuf ^ 1);
        }
        vm_wait<0>();
        lds_barrier();
    }
    // register 4 i + e: m = m0 + 32 mb + 8 i + 4 kh + e, n = n0 + nr
    const int n = n0 + nr;
    if (n < N) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + 32 * mb + 8 * i + 4 * kh + e;
                if (m < live) {
                    if (EPI == 0) {
                        reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = (uint16_t)f32_to_bf16(y[4 * i + e]);
                    } else {
                        float* o = reinterpret_cast<float*>(out) + (int64_t)m * ldo + n;
                        *o = add_rn(*o, y[4 * i + e]);
                    }
                }
            }
    }
}

}  // namespace prism

using namespace prism;

extern "C" int prism_q4k_pack(const uint8_t* raw, uint8_t* qv, uint8_t* meta, int64_t N, int64_t K, void* stream) {
    if (!raw || !qv || !meta) return PRISM_ERR_ARG;
    if (N <= 0 || K <= 0 || N % 16 || K % 256 || N > (1 << 30) || K > (1 << 30)) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(raw, 16) || !PRISM_ALIGNED(qv, 16) || !PRISM_ALIGNED(meta, 16)) return PRISM_ERR_ALIGN;
    const int64_t total = N / 16 * (K / 256) * 128;
    hipLaunchKernelGGL(q4k_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, raw,
                       qv, meta, (int)N, (int)K);
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_w4a8_q4k_gemm(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs,
                                   const uint8_t* qv, const uint8_t* meta, void* out, int64_t ldo,
                                   const int32_t* n_rows, int64_t M, int64_t N, int64_t K, int epi, int kernel,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
    if (!xq || !a || !xs || !qv || !meta || !out || !n_rows) return PRISM_ERR_ARG;
    if (epi != 0 && epi != 1) return PRISM_ERR_ARG;
    if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 256 || ldo < N || M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
        return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(xq, 16) || !PRISM_ALIGNED(xs, 16) || !PRISM_ALIGNED(qv, 16) || !PRISM_ALIGNED(meta, 16))
        return PRISM_ERR_ALIGN;
    if (kernel < -1 || kernel > 2) return PRISM_ERR_ARG;
    const bool can_bal = q4k_bal_fits(M, N, K) && workspace && workspace_bytes >= q4k_bal_workspace_bytes(N);
    // by default up to 4 rows: the balanced kernel for long projections of fewer than two 16-row tiles per CU (where
    // a tile per workgroup leaves CUs with one tile more than others: 5120 x 17408 at 1 row 15.1 us against 18.4 us),
    // given its workspace; the per-tile kernel otherwise (13824 x 5120: 11.4 against 15.4 us; 5120^2 at 1-4 rows
    // 7.5-8.0 against 8.2-8.8 us) and from 5 rows, where it takes two tiles per workgroup (5120^2 at 16 rows 8.9
    // against 9.9 us); the tile kernel beyond 16 rows.  The MI355X table overrides this per shape.
    if (kernel == -1) kernel = M >= 1 && M <= 16 ? (can_bal && N / 16 < 512 && K >= 8192 && M <= 4 ? 2 : 1) : 0;
    if (kernel == 1 && M > 16) return PRISM_ERR_ARG;
    if (kernel == 2 && !can_bal) return M > 16 || !q4k_bal_fits(M, N, K) ? PRISM_ERR_SHAPE : PRISM_ERR_ARG;
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    if (kernel == 2) {
        const int rc = q4k_bal_launch(xq, a, a_sb, xs, qv, meta, out, ldo, n_rows, M, N, K, epi, workspace,
                                      workspace_bytes, st);
        if (rc != PRISM_OK) return rc;
        PRISM_LAUNCH_CHECK();
        return PRISM_OK;
    }
    const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
    if (kernel == 1) {
        // Q4_K decode: the stream kernel, 8 waves for long K or narrow projections (few workgroups), else 4
        const size_t lds = (size_t)(K / 256) * M * 16 * 4;
        if (lds > 160 * 1024) kernel = 0;                 // the terms of every super-block do not fit: tile kernel
    }
    if (kernel == 1) {
        const bool wide = K >= 6144 || N <= 2048;
        // two tiles per wave (one activation load for both) from 5 rows, below 1024 tiles (at 17408 x 5120 half as
        // many workgroups lost 1-1.3 us up to 8 rows and tied at 16; C3's 13824 x 5120 at 16 rows: 16.6 -> 14.4 us,
        // 5120 x 17408: 26.8 -> 20.7 us)
        const int tg = (M >= Q4S_TG2_ROWS && N % 32 == 0 && N / 16 < 1024 &&
                        (size_t)(K / 256) * M * 16 * 4 * 2 <= 160 * 1024) ? 2 : 1;
        const size_t lds = (size_t)tg * (K / 256) * M * 16 * 4;
#define W4S(NW, TG, E) do {                                                                                        \
        allow_lds(w4a8_q4k_stream_kernel<NW, 2, TG, E>, lds);                                                     \
        hipLaunchKernelGGL((w4a8_q4k_stream_kernel<NW, 2, TG, E>), dim3(Ni / (16 * TG)), dim3(64 * NW), lds, st, xq, \
                           a, a_sb, xs, qv, meta, out, ldo, n_rows, Mi, Ki);                                       \
    } while (0)
#define W4S_TG(NW, E) do { if (tg == 2) W4S(NW, 2, E); else W4S(NW, 1, E); } while (0)
        if (wide) { if (epi == 0) W4S_TG(8, 0); else W4S_TG(8, 1); }
        else { if (epi == 0) W4S_TG(4, 0); else W4S_TG(4, 1); }
#undef W4S_TG
#undef W4S
    } else if ((int64_t)(N / 16) * (K / 256) * 2048 < ((int64_t)1 << 31) && M * K < ((int64_t)1 << 31)) {
        // the 128 x 128 tile kernel (w4a8_prefill.hip), whose stage offsets are 32-bit
        q4k_tile_launch(xq, a, a_sb, xs, qv, meta, out, ldo, n_rows, Mi, Ni, Ki, epi, st);
    } else {
        // operands of 2 GB or more: the 128 x 64 tile kernel above
        const int tiles_m = (Mi + QBM - 1) / QBM, tiles_n = (Ni + QBN - 1) / QBN;
        if (epi == 0)
            hipLaunchKernelGGL((w4a8_tile_kernel<0>), dim3(tiles_m * tiles_n), dim3(256), 0, st, xq, a, a_sb, xs, qv,
                               meta, out, ldo, n_rows, Mi, Ni, Ki, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL((w4a8_tile_kernel<1>), dim3(tiles_m * tiles_n), dim3(256), 0, st, xq, a, a_sb, xs, qv,
                               meta, out, ldo, n_rows, Mi, Ni, Ki, tiles_m, tiles_n);
    }
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_q6k_pack(const uint8_t* raw, uint8_t* qv, uint8_t* meta, int64_t N, int64_t K, void* stream) {
    if (!raw || !qv || !meta) return PRISM_ERR_ARG;
    if (N <= 0 || K <= 0 || N % 16 || K % 256 || N > (1 << 30) || K > (1 << 30)) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(qv, 16) || !PRISM_ALIGNED(meta, 16)) return PRISM_ERR_ALIGN;
    const int64_t total = N / 16 * (K / 256) * 256;
    hipLaunchKernelGGL(q6k_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, raw,
                       qv, meta, (int)N, (int)K);
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_w4a8_q6k_gemm(const int8_t* xq, const float* a, int64_t a_sb, const uint8_t* qv,
                                   const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int64_t M,
                                   int64_t N, int64_t K, int epi, int kernel, void* stream) {
    if (!xq || !a || !qv || !meta || !out || !n_rows) return PRISM_ERR_ARG;
    if (epi != 0 && epi != 1) return PRISM_ERR_ARG;
    if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 256 || ldo < N || M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
        return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(xq, 16) || !PRISM_ALIGNED(qv, 16) || !PRISM_ALIGNED(meta, 16)) return PRISM_ERR_ALIGN;
    if (kernel < -1 || kernel > 2) return PRISM_ERR_ARG;
    if (kernel == -1) kernel = M <= 16 ? 1 : 0;
    if (kernel >= 1 && M > 16) return PRISM_ERR_ARG;
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
    if (kernel == 2 && (size_t)(K / 256) * M * 16 * 4 > 160 * 1024) kernel = 1;   // terms beyond the LDS: staged
    if (kernel == 2) {
        const size_t lds = (size_t)(K / 256) * M * 16 * 4;
#define Q6S(E) do {                                                                                                \
        allow_lds(w4a8_q6k_stream_kernel<4, 2, E>, lds);                                                          \
        hipLaunchKernelGGL((w4a8_q6k_stream_kernel<4, 2, E>), dim3(Ni / 16), dim3(256), lds, st, xq, a, a_sb, qv,   \
                           meta, out, ldo, n_rows, Mi, Ki);                                                        \
    } while (0)
        if (epi == 0) Q6S(0); else Q6S(1);
#undef Q6S
    } else if (kernel == 1) {
#define Q6DEC(NW, R, MX, D, TG, E)                                                                                  \
    do {                                                                                                           \
        const size_t lds = q6k_decode_lds(R, Mi, TG);                                                               \
        allow_lds(w4a8_q6k_decode_kernel<NW, R, MX, D, TG, E>, lds);                                                \
        hipLaunchKernelGGL((w4a8_q6k_decode_kernel<NW, R, MX, D, TG, E>), dim3(Ni / (16 * TG)), dim3(NW * TG * 64),  \
                           lds, st, xq, a, a_sb, qv, meta, out, ldo, n_rows, Mi, Ni, Ki);                          \
    } while (0)
// decode configurations (waves per tile, super-blocks per round, rows, rounds of weights in flight, tiles per
// workgroup), measured on MI355X at the 27B's shapes (M <= 4, M <= 16); overridable at build time.  At 5-8 rows two
// tiles share each staged activation copy where N allows (C3's 13824 x 5120: 25.1 / 23.9 -> 23.5 / 23.1 us at 5 / 8
// rows; at 16 rows 0.3-0.8 us slower: this kernel's own VALU, not the activation copy, bounds it there)
#ifndef W6V_SMALL
#define W6V_SMALL 4, 4, 4, 2, 1
#endif
#ifndef W6V_BIG
#define W6V_BIG 4, 4, 16, 2, 1
#endif
#ifndef W6V_BIG2
#define W6V_BIG2 4, 4, 16, 2, 2
#endif
#define Q6DEC_(...) Q6DEC(__VA_ARGS__)
        if (M <= 4) {
            if (epi == 0) Q6DEC_(W6V_SMALL, 0); else Q6DEC_(W6V_SMALL, 1);
        } else if (M <= 8 && N % 32 == 0 && N / 16 < 1024) {
            if (epi == 0) Q6DEC_(W6V_BIG2, 0); else Q6DEC_(W6V_BIG2, 1);
        } else {
            if (epi == 0) Q6DEC_(W6V_BIG, 0); else Q6DEC_(W6V_BIG, 1);
        }
#undef Q6DEC_
#undef Q6DEC
    } else if ((int64_t)(N / 16) * (K / 256) * 4096 < ((int64_t)1 << 31) && M * K < ((int64_t)1 << 31)) {
        // the 128 x 128 two-plane tile kernel (w4a8_prefill.hip), whose stage offsets are 32-bit
        q6k_tile_launch(xq, a, a_sb, qv, meta, out, ldo, n_rows, Mi, Ni, Ki, epi, st);
    } else {
        // operands of 2 GB or more: the 32 x 32 x 16 tile kernel above
        const int tiles_m = (Mi + QBM - 1) / QBM, tiles_n = (Ni + Q6BN - 1) / Q6BN;
        if (epi == 0)
            hipLaunchKernelGGL((w4a8_q6k_tile32_kernel<0>), dim3(tiles_m * tiles_n), dim3(256), 0, st, xq, a, a_sb,
                               qv, meta, out, ldo, n_rows, Mi, Ni, Ki, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL((w4a8_q6k_tile32_kernel<1>), dim3(tiles_m * tiles_n), dim3(256), 0, st, xq, a, a_sb,
                               qv, meta, out, ldo, n_rows, Mi, Ni, Ki, tiles_m, tiles_n);
    }
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}
