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
// MT: activation tiles of 16 rows (M <= 16 MT); C: blocks per wave per round (4 C blocks per round).
template <int MT, int C, bool AS_GROUP, bool WS16, int EPI>
__global__ __launch_bounds__(256) void w8a8_decode_kernel(const int8_t* __restrict__ a, const float* __restrict__ a_s,
                                                          int64_t as_sm, int64_t as_sg,
                                                          const int8_t* __restrict__ w, const void* __restrict__ w_s,
                                                          void* __restrict__ out, int64_t ldo,
                                                          const int32_t* __restrict__ n_rows, int M, int N, int K) {
    constexpr int R = 4 * C;                       // blocks per round
    __shared__ v4f terms[R][MT * 16][4];           // [block][m][n / 4]: 16 n per row as 4 float4
    __shared__ float sws[R][16];                   // the round's weight scales, fp32, [block][n]

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n0 = blockIdx.x * 16;
    const int live = min(M, __ldg(n_rows));
    const int G = K / 32;

    // MFMA lanes: A = weights, row n0 + lane % 16, bytes [8 (lane / 16), +8) of each 32-byte block;
    //             B = activations, row (column of D) mt * 16 + lane % 16, the same bytes.
    const int8_t* wrow = w + (int64_t)(n0 + (lane & 15)) * K + (lane >> 4) * 8;
    const int kq = (lane >> 4) * 8;
    float sa[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = mt * 16 + (lane & 15);
        sa[mt] = (!AS_GROUP && m < M) ? a_s[(int64_t)m * as_sm] : 0.f;
    }

    // sw staging: 16 rows x R blocks, (16 R) / 256 values per thread
    constexpr int SWV = (16 * R + 255) / 256;
    auto load_sw = [&](int rb, float* reg) {
#pragma unroll
        for (int i = 0; i < SWV; i++) {
            const int e = tid + i * 256;
            const int row = e / R, blk = e % R;
            float v = 0.f;
            if (e < 16 * R && rb + blk < G) {
                const int64_t off = (int64_t)(n0 + row) * G + rb + blk;
                v = WS16 ? f16_to_f32(reinterpret_cast<const uint16_t*>(w_s)[off])
                         : reinterpret_cast<const float*>(w_s)[off];
            }
            reg[i] = v;
        }
    };
    auto store_sw = [&](const float* reg) {
#pragma unroll
        for (int i = 0; i < SWV; i++) {
            const int e = tid + i * 256;
            if (e < 16 * R) sws[e % R][e / R] = reg[i];
        }
    };
    int64_t wb[C], ab[C][MT];
    auto load_ops = [&](int rb) {
#pragma unroll
        for (int i = 0; i < C; i++) {
            const int blk = rb + wv * C + i;
            const bool ok = blk < G;
            wb[i] = ok ? __builtin_nontemporal_load(reinterpret_cast<const int64_t*>(wrow + (int64_t)blk * 32)) : 0;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int m = mt * 16 + (lane & 15);
                ab[i][mt] = (ok && m < M) ? *reinterpret_cast<const int64_t*>(a + (int64_t)m * K + blk * 32 + kq) : 0;
            }
        }
    };

    float y[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) y[mt] = 0.f;
    float swr[SWV];
    load_sw(0, swr);
    load_ops(0);
    for (int rb = 0; rb < G; rb += R) {
        store_sw(swr);
        __syncthreads();
        // ---- produce: the terms RN(RN(float(P) sa) sw) of this wave's C blocks
#pragma unroll
        for (int i = 0; i < C; i++) {
            const int lb = wv * C + i, blk = rb + lb;
            if (blk < G) {
                const v4f sw4 = *reinterpret_cast<const v4f*>(&sws[lb][(lane >> 4) * 4]);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    v4i acc = {0, 0, 0, 0};
                    acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(wb[i], ab[i][mt], acc, 0, 0, 0);
                    float s = sa[mt];
                    if (AS_GROUP) {
                        const int m = mt * 16 + (lane & 15);
                        s = m < M ? a_s[(int64_t)m * as_sm + (int64_t)blk * as_sg] : 0.f;
                    }
                    v4f t;
#pragma unroll
                    for (int r = 0; r < 4; r++) t[r] = mul_rn(mul_rn((float)acc[r], s), sw4[r]);
                    terms[lb][mt * 16 + (lane & 15)][lane >> 4] = t;
                }
            }
        }
        const int nb = min(R, G - rb);
        if (rb + R < G) {
            load_sw(rb + R, swr);
            load_ops(rb + R);
        }
        __syncthreads();
        // ---- reduce: thread tid owns (m = tid / 16 + 16 mt, n = n0 + tid % 16); add the round's terms in order
        const float* tf = reinterpret_cast<const float*>(&terms[0][0][0]);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            float acc = y[mt];
            for (int j = 0; j < nb; j++) acc = add_rn(acc, tf[(j * MT * 16 + mt * 16) * 16 + tid]);
            y[mt] = acc;
        }
    }
    // ---- epilogue
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = mt * 16 + tid / 16, n = n0 + (tid & 15);
        if (m < live) {
            if (EPI == 0) {
                reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = (uint16_t)f32_to_bf16(y[mt]);
            } else {
                float* o = reinterpret_cast<float*>(out) + (int64_t)m * ldo + n;
                *o = add_rn(*o, y[mt]);
            }
        }
    }
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
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& pm, int& pn) {
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
    tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
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
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *reinterpret_cast<v4i*>(&As[(lr + 32 * i) * TLD + lc]) = ra[i];
            *reinterpret_cast<v4i*>(&Bs[(lr + 32 * i) * TLD + lc]) = rb[i];
        }
        sws[tid & 3][tid >> 2] = rs0;
        sws[tid & 3][64 + (tid >> 2)] = rs1;
        __syncthreads();
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
template <bool AS_GROUP, bool WS16, int EPI>
static int launch_w8a8(int kernel, const int8_t* a, const float* a_s, int64_t as_sm, int64_t as_sg, const int8_t* w,
                       const void* w_s, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int gk,
                       hipStream_t st) {
    if (kernel == 1) {
        dim3 grid(N / 16), block(256);
        const int mt = (M + 15) / 16;
#define DEC(MT, C) hipLaunchKernelGGL((w8a8_decode_kernel<MT, C, AS_GROUP, WS16, EPI>), grid, block, 0, st, a, a_s, \
                                      as_sm, as_sg, w, w_s, out, ldo, n_rows, M, N, K)
        if (mt == 1) DEC(1, 8);
        else if (mt == 2) DEC(2, 4);
        else if (mt == 3) DEC(3, 2);
        else DEC(4, 2);
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
    if (kernel == -1) kernel = (gk == 32 && M <= 64) ? 1 : 0;
    if (kernel == 1 && (gk != 32 || M > 64)) return PRISM_ERR_ARG;
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
