// W8A8 GEMM with per-group scales along K on gfx950 int8 MFMA: Q8_0 weights (gk = 32: the file's int8 values and
// fp16 block scales) and the per-channel form (gk = K).
//
// Arithmetic (StartLux-Prism kernels/w8a8.py:64-85, _w8a8_kernel), for every output (m, n), groups g in increasing
// order:   P = sum_{k in g} a[m,k] w[n,k]                    int32, exact (MFMA i32 accumulation)
//          y = RN(y + RN(RN(float(P) * sa[m,g]) * sw[n,g]))  fp32, each step rounded once, y starting at +0
// epi 0 stores RN_bf16(y); epi 1 stores RN(out + y).  Every kernel keeps this order for every element, so all
// kernels, tile shapes and batch sizes give the same bits (batch invariance).
//
// Because the fp32 sum over groups is ordered, K is never split across waves that add partial fp32 sums; where a
// kernel spreads K over waves (the decode kernel) the per-group terms go through LDS and one owner lane adds them in
// order.
//
// Two kernels:
//   tile    BM x BN = 128 x 128 per 256-thread workgroup (2 x 2 waves of 64 x 64), v_mfma_i32_32x32x32_i8 (K = 32 is
//           exactly one Q8_0 block), A/B tiles of 4 blocks staged through LDS with register prefetch.  Prefill.
//   decode  M <= 64, gk = 32.  A workgroup owns 16 weight rows and every activation row; its four waves take
//           interleaved runs of C blocks of K per round (v_mfma_i32_16x16x32_i8, weights as the A operand, read
//           straight from HBM with 8-byte loads), write the per-block terms to LDS, and after a barrier each output's
//           owner thread adds the round's terms in block order.  HBM-bound on the weight stream.
#include "common.h"

namespace prism {

// ============================================================================================== decode kernel
// A workgroup of NW waves owns 16 weight rows (n0 .. n0 + 15) and every activation row (M <= 64).  K is walked in
// rounds of R blocks (32 R bytes per row).  Round r:
//   1. the round's weight rows, activation rows and weight scales, requested during round r - 1 with
//      row-contiguous 16-byte loads (a wave instruction reads 1 KB of a row), are written to LDS, and round r + 1's
//      loads are issued;
//   2. wave w computes blocks w CB .. w CB + CB - 1 of the round with v_mfma_i32_16x16x32_i8 (weights as the A
//      operand: lane l reads row l % 16, bytes 8 (l / 16) .. +8 of the block from LDS; activations as B), turns each
//      block's int32 sums into the term RN(RN(float(P) sa) sw) and writes the terms of live rows to one of two LDS
//      term buffers, [block][m][n];
//   3. meanwhile the owner thread of each output adds round r - 1's terms, from the other buffer, in block order
//      (the reference's sequential fp32 sum over groups), so the ordered sum is off the MFMA path.
template <int NW, int R, int MT, int D, bool AS_GROUP, bool WS16, int EPI>
__global__ __launch_bounds__(NW * 64) void w8a8_decode_kernel(const int8_t* __restrict__ a,
                                                              const float* __restrict__ a_s, int64_t as_sm,
                                                              int64_t as_sg, const int8_t* __restrict__ w,
                                                              const void* __restrict__ w_s, void* __restrict__ out,
                                                              int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                              int N, int K) {
    constexpr int NT = NW * 64;
    constexpr int CB = R / NW;                     // blocks per wave per round
    static_assert(CB >= 1 && CB * NW == R, "R must be a multiple of NW");
    constexpr int RB = R * 32;                     // bytes per row per round
    constexpr int LD = RB + 16;                    // padded LDS row
    constexpr int CPR = RB / 16;                   // 16-byte chunks per row per round
    constexpr int WPT = (16 * CPR + NT - 1) / NT;
    constexpr int APT = (MT * 16 * CPR + NT - 1) / NT;
    constexpr int SWV = (16 * R + NT - 1) / NT;
    extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
    int8_t* Wl = dsm;                                                   // [16][LD]
    int8_t* Al = Wl + 16 * LD;                                          // [M][LD]
    float* sws = reinterpret_cast<float*>(Al + ((M * LD + 15) & ~15));  // [R][16]
    float* terms = sws + R * 16;                                        // [2][R][M][16]
    const int tstride = R * M * 16;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n0 = blockIdx.x * 16;
    const int live = min(M, __ldg(n_rows));
    const int G = K / 32;
    const int lm = lane & 15, kq = (lane >> 4) * 8;
    const int ach = M * CPR;

    float sa[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) sa[mt] = AS_GROUP ? 0.f : a_s[(int64_t)min(mt * 16 + lm, M - 1) * as_sm];

    struct Stage {
        v4i w[WPT];
        v4i a[APT];
        uint32_t sw[SWV];     // raw scale bits (fp16 or fp32), widened when written to LDS
    };
    // Loads are unconditional (indices clamped in range, surplus threads reload a valid chunk): no branch around
    // them, so the compiler's wait counts stay exact and a round's loads stay in flight across the barriers.
    auto load = [&](int rb, Stage& st) {
        const int64_t k0 = (int64_t)rb * 32;
#pragma unroll
        for (int i = 0; i < WPT; i++) {
            const int c = min(tid + i * NT, 16 * CPR - 1);
            const int row = c / CPR;
            const int64_t kk = min(k0 + (c % CPR) * 16, (int64_t)K - 16);
            st.w[i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + (int64_t)(n0 + row) * K + kk));
        }
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int c = min(tid + i * NT, ach - 1);
            const int row = c / CPR;
            const int64_t kk = min(k0 + (c % CPR) * 16, (int64_t)K - 16);
            st.a[i] = *reinterpret_cast<const v4i*>(a + (int64_t)row * K + kk);
        }
#pragma unroll
        for (int i = 0; i < SWV; i++) {
            const int e = min(tid + i * NT, 16 * R - 1);
            const int row = e / R, blk = min(rb + e % R, G - 1);
            const int64_t off = (int64_t)(n0 + row) * G + blk;
            st.sw[i] = WS16 ? (uint32_t)reinterpret_cast<const uint16_t*>(w_s)[off]
                            : reinterpret_cast<const uint32_t*>(w_s)[off];
        }
    };
    // chunks past the end of K were loaded from its last 16 bytes; they land past the round's last block
    auto store = [&](const Stage& st) {
#pragma unroll
        for (int i = 0; i < WPT; i++) {
            const int c = tid + i * NT;
            if (c < 16 * CPR) *reinterpret_cast<v4i*>(&Wl[(c / CPR) * LD + (c % CPR) * 16]) = st.w[i];
        }
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int c = tid + i * NT;
            if (c < ach) *reinterpret_cast<v4i*>(&Al[(c / CPR) * LD + (c % CPR) * 16]) = st.a[i];
        }
#pragma unroll
        for (int i = 0; i < SWV; i++) {
            const int e = tid + i * NT;
            if (e < 16 * R) sws[(e % R) * 16 + e / R] = WS16 ? f16_to_f32(st.sw[i]) : __uint_as_float(st.sw[i]);
        }
    };
    auto compute = [&](int rb, float* tb) {
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int lb = wv * CB + i, blk = rb + lb;
            if (blk < G) {
                const int64_t wf = *reinterpret_cast<const int64_t*>(&Wl[lm * LD + lb * 32 + kq]);
                const v4f sw4 = *reinterpret_cast<const v4f*>(&sws[lb * 16 + (lane >> 4) * 4]);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const int m = mt * 16 + lm;
                    const int64_t af = *reinterpret_cast<const int64_t*>(&Al[min(m, M - 1) * LD + lb * 32 + kq]);
                    const v4i zero = {0, 0, 0, 0};
                    const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf, af, zero, 0, 0, 0);
                    float s = sa[mt];
                    if (AS_GROUP) s = a_s[(int64_t)min(m, M - 1) * as_sm + (int64_t)blk * as_sg];
                    v4f t;
#pragma unroll
                    for (int r = 0; r < 4; r++) t[r] = mul_rn(mul_rn((float)acc[r], s), sw4[r]);
                    if (m < M) *reinterpret_cast<v4f*>(&tb[(lb * M + m) * 16 + (lane >> 4) * 4]) = t;
                }
            }
        }
    };
    // output o = tid + NT j: m = o / 16, n = n0 + o % 16
    constexpr int OPT = (64 * 16 + NT - 1) / NT;
    float y[OPT];
#pragma unroll
    for (int j = 0; j < OPT; j++) y[j] = 0.f;
    auto fold = [&](int rb, const float* tb) {
        const int nb = min(R, G - rb);
#pragma unroll
        for (int jo = 0; jo < OPT; jo++) {
            const int o = tid + jo * NT;
            if (o < M * 16) {
                const float* tp = tb + o;
                const int st = M * 16;
                float acc = y[jo];
                int j = 0;
                for (; j + 16 <= nb; j += 16) {
                    float v[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) v[u] = tp[(j + u) * st];
#pragma unroll
                    for (int u = 0; u < 16; u++) acc = add_rn(acc, v[u]);
                }
                for (; j < nb; j++) acc = add_rn(acc, tp[j * st]);
                y[jo] = acc;
            }
        }
    };

    // D-deep register ring: round r + D - 1 is requested before round r's data are waited for.  Loads and LDS
    // stores run for every slot (past the end they reload the last chunk of K); only the math is guarded.
    Stage st[D];
#pragma unroll
    for (int d = 0; d < D - 1; d++) load(d * R, st[d]);
    const int nr = (G + R - 1) / R;
    for (int r0 = 0; r0 < nr; r0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int r = r0 + d, rb = r * R;
            load(rb + (D - 1) * R, st[(d + D - 1) % D]);
            store(st[d]);
            lds_barrier();
            if (r < nr) {
                compute(rb, terms + (r & 1) * tstride);
                if (r > 0) fold(rb - R, terms + ((r - 1) & 1) * tstride);
            }
            lds_barrier();
        }
    }
    const int last = ((G - 1) / R) * R;
    fold(last, terms + ((last / R) & 1) * tstride);
#pragma unroll
    for (int jo = 0; jo < OPT; jo++) {
        const int o = tid + jo * NT;
        const int m = o >> 4, n = n0 + (o & 15);
        if (o < M * 16 && m < live) {
            if (EPI == 0) {
                reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = (uint16_t)f32_to_bf16(y[jo]);
            } else {
                float* op = reinterpret_cast<float*>(out) + (int64_t)m * ldo + n;
                *op = add_rn(*op, y[jo]);
            }
        }
    }
}

static size_t decode_lds(int R, int M) {
    const size_t LD = (size_t)R * 32 + 16;
    return 16 * LD + ((M * LD + 15) & ~(size_t)15) + (size_t)R * 16 * 4 + 2 * (size_t)R * M * 64;
}

// ============================================================================================== tile kernel
constexpr int TBM = 128, TBN = 128, TBK = 128;     // bytes of K per stage = 4 blocks
constexpr int TLD = TBK + 16;                       // padded LDS row (bytes)

template <bool AS_GROUP, bool WS16, int EPI>
__global__ __launch_bounds__(256, 1) void w8a8_tile_kernel(const int8_t* __restrict__ a, const float* __restrict__ a_s,
                                                           int64_t as_sm, int64_t as_sg,
                                                           const int8_t* __restrict__ w, const void* __restrict__ w_s,
                                                           void* __restrict__ out, int64_t ldo,
                                                           const int32_t* __restrict__ n_rows, int M, int N, int K,
                                                           int GB, int tiles_m) {
    __shared__ __attribute__((aligned(16))) int8_t As[TBM * TLD];
    __shared__ __attribute__((aligned(16))) int8_t Bs[TBN * TLD];
    __shared__ float sws[4][TBN];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv >> 1, wn = wv & 1;
    const int pid = blockIdx.x;
    const int pm = pid % tiles_m, pn = pid / tiles_m;
    const int m0 = pm * TBM, n0 = pn * TBN;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int G = K / 32;          // blocks
    const int NG = G / GB;         // groups

    // ---- global -> register staging: 4 chunks of 16 bytes per thread per operand
    v4i ra[4], rb[4];
    float rs[2];
    auto gload = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + i * 256, row = c >> 3, col = (c & 7) * 16;
            const bool kin = kb * 32 + col < K;
            const int am = m0 + row, bn = n0 + row;
            ra[i] = (am < M && kin) ? *reinterpret_cast<const v4i*>(a + (int64_t)am * K + kb * 32 + col) : v4i{0, 0, 0, 0};
            rb[i] = (bn < N && kin) ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + (int64_t)bn * K + kb * 32 + col))
                                    : v4i{0, 0, 0, 0};
        }
        if (GB == 1) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int e = tid + i * 256, row = e >> 2, blk = e & 3;
                const int n = n0 + row, g = kb + blk;
                float v = 0.f;
                if (n < N && g < G) {
                    const int64_t off = (int64_t)n * NG + g;
                    v = WS16 ? f16_to_f32(reinterpret_cast<const uint16_t*>(w_s)[off]) : reinterpret_cast<const float*>(w_s)[off];
                }
                rs[i] = v;
            }
        }
    };
    auto sstore = [&]() {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + i * 256, row = c >> 3, col = (c & 7) * 16;
            *reinterpret_cast<v4i*>(&As[row * TLD + col]) = ra[i];
            *reinterpret_cast<v4i*>(&Bs[row * TLD + col]) = rb[i];
        }
        if (GB == 1) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int e = tid + i * 256;
                sws[e & 3][e >> 2] = rs[i];
            }
        }
    };

    // D layout of v_mfma_i32_32x32x32_i8: lane l, register r -> column l % 32, row 8 (r / 4) + 4 (l / 32) + r % 4
    const int lrow = 4 * (lane >> 5);
    float sa[2][16];
    if (!AS_GROUP) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + mt * 32 + 8 * (r >> 2) + lrow + (r & 3);
                sa[mt][r] = m < M ? a_s[(int64_t)m * as_sm] : 0.f;
            }
    }
    float y[2][2][16];
    v16i acc[2][2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                y[mt][nt][r] = 0.f;
                acc[mt][nt][r] = 0;
            }

    const int arow0 = (wm * 64 + (lane & 31)) * TLD + (lane >> 5) * 16;
    const int brow0 = (wn * 64 + (lane & 31)) * TLD + (lane >> 5) * 16;
    gload(0);
    for (int kb = 0; kb < G; kb += 4) {
        __syncthreads();
        sstore();
        __syncthreads();
        if (kb + 4 < G) gload(kb + 4);
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
            const int blk = kb + bi;
            if (blk < G) {
                v4i fa[2], fb[2];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    fa[t] = *reinterpret_cast<const v4i*>(&As[arow0 + t * 32 * TLD + bi * 32]);
                    fb[t] = *reinterpret_cast<const v4i*>(&Bs[brow0 + t * 32 * TLD + bi * 32]);
                }
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int nt = 0; nt < 2; nt++)
                        acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[mt], fb[nt], acc[mt][nt], 0, 0, 0);
                if ((blk + 1) % GB == 0) {
                    const int g = blk / GB;
#pragma unroll
                    for (int nt = 0; nt < 2; nt++) {
                        const int nl = wn * 64 + nt * 32 + (lane & 31);
                        float sw;
                        if (GB == 1) {
                            sw = sws[bi][nl];
                        } else {
                            const int n = n0 + nl;
                            const int64_t off = (int64_t)n * NG + g;
                            sw = n < N ? (WS16 ? f16_to_f32(reinterpret_cast<const uint16_t*>(w_s)[off])
                                               : reinterpret_cast<const float*>(w_s)[off])
                                       : 0.f;
                        }
#pragma unroll
                        for (int mt = 0; mt < 2; mt++) {
#pragma unroll
                            for (int r = 0; r < 16; r++) {
                                float s = sa[mt][r];
                                if (AS_GROUP) {
                                    const int m = m0 + wm * 64 + mt * 32 + 8 * (r >> 2) + lrow + (r & 3);
                                    s = m < M ? a_s[(int64_t)m * as_sm + (int64_t)g * as_sg] : 0.f;
                                }
                                y[mt][nt][r] = add_rn(y[mt][nt][r], mul_rn(mul_rn((float)acc[mt][nt][r], s), sw));
                                acc[mt][nt][r] = 0;
                            }
                        }
                    }
                }
            }
        }
    }
    // ---- epilogue: rows < live, columns < N
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int n = n0 + wn * 64 + nt * 32 + (lane & 31);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + mt * 32 + 8 * (r >> 2) + lrow + (r & 3);
                if (m < live) {
                    if (EPI == 0) {
                        reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = (uint16_t)f32_to_bf16(y[mt][nt][r]);
                    } else {
                        float* o = reinterpret_cast<float*>(out) + (int64_t)m * ldo + n;
                        *o = add_rn(*o, y[mt][nt][r]);
                    }
                }
            }
        }
}

// ============================================================================================== Q8_0 tile kernel
// The prefill path for gk = 32 with one activation scale per token and K % 128 == 0: one
// v_mfma_i32_32x32x32_i8 per (32 x 32 tile, block) with a zero accumulator input, so each block's int32 sums come
// out of the MFMA ready for the epilogue and nothing is carried between blocks but the fp32 sums y.  The exact
// per-block epilogue (cvt, two multiplies, add: 4 VALU ops per output and block) is the bound of this kernel.
//
// Tile order: the hardware hands workgroup i to XCD i % 8.  Logical tile t = (i % 8) * (tiles / 8) + i / 8 gives
// each XCD a contiguous range of tiles, walked in groups of 8 tile-rows (m fastest), so the workgroups that run
// together on one XCD share 8 activation tiles and 8 weight tiles through that XCD's L2.
template <bool WS16, int EPI>
__global__ __launch_bounds__(256, 2) void w8a8_q8_tile_kernel(const int8_t* __restrict__ a,
                                                              const float* __restrict__ a_s, int64_t as_sm,
                                                              const int8_t* __restrict__ w,
                                                              const void* __restrict__ w_s, void* __restrict__ out,
                                                              int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                              int N, int K, int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(16))) int8_t As[TBM * TLD];
    __shared__ __attribute__((aligned(16))) int8_t Bs[TBN * TLD];
    __shared__ float sws[4][TBN];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv >> 1, wn = wv & 1;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * TBM, n0 = pn * TBN;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int G = K / 32;

    // loaders: chunk i of this thread is row lr + 32 i, bytes lc .. lc + 15 of the stage (rows clamped in range:
    // a clamped row is loaded but never stored)
    const int lr = tid >> 3, lc = (tid & 7) * 16;
    const int8_t* ap[4];
    const int8_t* bp[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        ap[i] = a + (int64_t)min(m0 + lr + 32 * i, M - 1) * K + lc;
        bp[i] = w + (int64_t)min(n0 + lr + 32 * i, N - 1) * K + lc;
    }
    // weight scales: element e = tid + 256 i -> row e / 4, block e % 4 of the stage
    const int64_t sw_off0 = (int64_t)min(n0 + (tid >> 2), N - 1) * G + (tid & 3);
    const int64_t sw_off1 = (int64_t)min(n0 + 64 + (tid >> 2), N - 1) * G + (tid & 3);
    auto ldsw = [&](int64_t off) -> float {
        return WS16 ? f16_to_f32(reinterpret_cast<const uint16_t*>(w_s)[off]) : reinterpret_cast<const float*>(w_s)[off];
    };

    v4i ra[4], rb[4];
    float rs0, rs1;
    auto gload = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            ra[i] = *reinterpret_cast<const v4i*>(ap[i] + kb * 32);
            rb[i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(bp[i] + kb * 32));
        }
        rs0 = ldsw(sw_off0 + kb);
        rs1 = ldsw(sw_off1 + kb);
    };

    const int lrow = 4 * (lane >> 5);
    float sa[2][16];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = min(m0 + wm * 64 + mt * 32 + 8 * (r >> 2) + lrow + (r & 3), M - 1);
            sa[mt][r] = a_s[(int64_t)m * as_sm];
        }
    float y[2][2][16];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int r = 0; r < 16; r++) y[mt][nt][r] = 0.f;

    const int arow0 = (wm * 64 + (lane & 31)) * TLD + (lane >> 5) * 16;
    const int brow0 = (wn * 64 + (lane & 31)) * TLD + (lane >> 5) * 16;
    const int swc = wn * 64 + (lane & 31);
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    gload(0);
    for (int kb = 0; kb < G; kb += 4) {
        lds_barrier();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *reinterpret_cast<v4i*>(&As[(lr + 32 * i) * TLD + lc]) = ra[i];
            *reinterpret_cast<v4i*>(&Bs[(lr + 32 * i) * TLD + lc]) = rb[i];
        }
        sws[tid & 3][tid >> 2] = rs0;
        sws[tid & 3][64 + (tid >> 2)] = rs1;
        lds_barrier();
        if (kb + 4 < G) gload(kb + 4);
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
            v4i fa[2], fb[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                fa[t] = *reinterpret_cast<const v4i*>(&As[arow0 + t * 32 * TLD + bi * 32]);
                fb[t] = *reinterpret_cast<const v4i*>(&Bs[brow0 + t * 32 * TLD + bi * 32]);
            }
            const float sw[2] = {sws[bi][swc], sws[bi][swc + 32]};
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const v16i acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[mt], fb[nt], zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        y[mt][nt][r] = add_rn(y[mt][nt][r], mul_rn(mul_rn((float)acc[r], sa[mt][r]), sw[nt]));
                }
        }
    }
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int n = n0 + wn * 64 + nt * 32 + (lane & 31);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + mt * 32 + 8 * (r >> 2) + lrow + (r & 3);
                if (m < live) {
                    if (EPI == 0) {
                        reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = (uint16_t)f32_to_bf16(y[mt][nt][r]);
                    } else {
                        float* o = reinterpret_cast<float*>(out) + (int64_t)m * ldo + n;
                        *o = add_rn(*o, y[mt][nt][r]);
                    }
                }
            }
        }
}

// ============================================================================================== launch
int launch_w8a8_pc(int kernel, bool wpack, const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* w,
                   const void* w_s, bool ws16, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K,
                   int epi, hipStream_t st, int split, int64_t zstride);

template <bool AS_GROUP, bool WS16, int EPI>
static int launch_w8a8(int kernel, const int8_t* a, const float* a_s, int64_t as_sm, int64_t as_sg, const int8_t* w,
                       const void* w_s, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int gk,
                       hipStream_t st) {
    // per channel (one group): the int8 MFMA GEMMs with an epilogue (w8a8_pc.hip)
    if (gk == K && K % 64 == 0 && ldo % 4 == 0 && PRISM_ALIGNED(out, EPI ? 16 : 8))
        return launch_w8a8_pc(kernel, false, a, a_s, as_sm, w, w_s, WS16, out, ldo, n_rows, M, N, K, EPI, st, 1, 0);
    if (kernel == 1) {
        dim3 grid(N / 16);
#define DEC(NW, R, MT, D)                                                                                         \
    hipLaunchKernelGGL((w8a8_decode_kernel<NW, R, MT, D, AS_GROUP, WS16, EPI>), grid, dim3(NW * 64),                \
                       decode_lds(R, M), st, a, a_s, as_sm, as_sg, w, w_s, out, ldo, n_rows, M, N, K)
        if (M <= 16) DEC(16, 32, 1, 6);
        else if (M <= 32) DEC(8, 8, 2, 8);
        else if (M <= 48) DEC(8, 8, 3, 8);
        else DEC(8, 8, 4, 8);
#undef DEC
    } else {
        const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
        dim3 grid(tiles_m * tiles_n), block(256);
        if (!AS_GROUP && gk == 32 && K % TBK == 0)
            hipLaunchKernelGGL((w8a8_q8_tile_kernel<WS16, EPI>), grid, block, 0, st, a, a_s, as_sm, w, w_s, out, ldo,
                               n_rows, M, N, K, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL((w8a8_tile_kernel<AS_GROUP, WS16, EPI>), grid, block, 0, st, a, a_s, as_sm, as_sg, w,
                               w_s, out, ldo, n_rows, M, N, K, gk / 32, tiles_m);
    }
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

}  // namespace prism

using namespace prism;

extern "C" int prism_w8a8_gemm(const int8_t* a, const float* a_s, int64_t as_sm, int64_t as_sg, const int8_t* w,
                               const void* w_s, int ws_fp16, void* out, int64_t ldo, const int32_t* n_rows, int64_t M,
                               int64_t N, int64_t K, int64_t gk, int epi, int kernel, void* stream) {
    if (!a || !a_s || !w || !w_s || !out || !n_rows) return PRISM_ERR_ARG;
    if (epi != 0 && epi != 1) return PRISM_ERR_ARG;
    if (M < 0 || N <= 0 || K <= 0 || K % 32 || N % 16 || gk <= 0 || gk % 32 || K % gk || ldo < N) return PRISM_ERR_SHAPE;
    if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) return PRISM_ERR_SHAPE;
    if ((int64_t)gk * 128 * 128 >= ((int64_t)1 << 31)) return PRISM_ERR_SHAPE;   // int32 group sums stay exact
    if (!PRISM_ALIGNED(a, 16) || !PRISM_ALIGNED(w, 16)) return PRISM_ERR_ALIGN;
    if (kernel < -1 || kernel > 1) return PRISM_ERR_ARG;
    // per channel on the int8 MFMA kernels: one group, 64-input stages, vector epilogue stores
    const bool pc = gk == K && K % 64 == 0 && ldo % 4 == 0 && PRISM_ALIGNED(out, epi ? 16 : 8);
    if (kernel == -1) kernel = ((gk == 32 || pc) && M <= 64) ? 1 : 0;
    if (kernel == 1 && ((gk != 32 && !pc) || (!pc && M > 64) || M > 65535 * 64)) return PRISM_ERR_ARG;
    if (M == 0) return PRISM_OK;
    const bool asg = as_sg != 0, ws16 = ws_fp16 != 0;
    hipStream_t st = (hipStream_t)stream;
#define L(AG, W16, E) return launch_w8a8<AG, W16, E>(kernel, a, a_s, as_sm, as_sg, w, w_s, out, ldo, n_rows, (int)M, \
                                                    (int)N, (int)K, (int)gk, st)
    if (asg) {
        if (ws16) { if (epi == 0) L(true, true, 0); else L(true, true, 1); }
        else { if (epi == 0) L(true, false, 0); else L(true, false, 1); }
    } else {
        if (ws16) { if (epi == 0) L(false, true, 0); else L(false, true, 1); }
        else { if (epi == 0) L(false, false, 0); else L(false, false, 1); }
    }
#undef L
}
