// Q8_0 W8A8 decode (M <= 16) on the packed layout, streamed from HBM by a balanced grid (gfx950).
//
// The work of a projection is its (16-row weight tile, block pair) chunks, tiles * K / 64 of them, 1 KB each.  W
// workgroups (one per CU at most: W <= 256 and W <= tiles) take equal contiguous ranges of that sequence, so every CU
// streams the same number of bytes whatever N / 16 is (320 tiles at N = 5120 would otherwise leave 64 CUs with two
// tiles and the rest with one).  A range therefore starts and ends inside tiles: its first tile's chunks continue a
// tile whose first chunks belong to the previous workgroup (a "tail"), its last tile's chunks start a tile the next
// workgroup finishes (a "head").  Every output's fp32 sum over blocks runs in block order (kernels/w8a8.py:74-76), so a
// tail's fold has to start from the head's running sums.  The workgroup walks its tiles last to first: the head comes
// first and its running sums are handed to the next workgroup through the workspace (one 64-bit word per output:
// the launch's tag and the fp32 bits), and the tail comes last, by when the previous workgroup has long published its
// head.  Whole tiles in between fold from zero and store their outputs.
//
// Inside a workgroup: NW compute waves take the round's block pairs (CP each); per block one MFMA with the activation
// rows as its A operand and the weight chunk's slot as its B gives the int32 sums, and every term
// RN(RN(float(P) sa) sw) goes to an LDS term buffer.  FW fold waves add the previous rounds' terms of one output per
// thread in block order while the compute waves run ahead (up to RD rounds, counted through LDS counters: no
// workgroup barriers in the loop).  Weights and their block scales are requested D - 1 rounds ahead in a register
// ring.  The activation rows travel in the ring with the weights (16 bytes per lane and pair, buffer loads); the
// build option Q8S_XL=1 copies them whole into LDS at the start where they fit (XL), which measured slower at
// every row count once the ring's activation loads took 16 bytes (5120^2 at 1 row 8.5 against 8.1 us, 5120 x 17408
// 18.4 against 17.8 us, 16 rows 11.2 against 10.6 us): the copy costs each workgroup the image's bytes up front.
// Measured on MI355X: twelve compute waves per workgroup (not eight, nor more) for one to four rows; a ring deeper
// than one round ahead and rounds of other sizes were slower.  From five rows the form depends on the shape (see the
// launch below).
//
// The walk over a range and the handoff protocol between neighbouring workgroups are handoff.h's.
#include "common.h"
#include "handoff.h"
#include "q8_stream.h"

namespace prism {

template <int NW, int R, int MX, int D, int RD, int EPI, bool XL>
__global__ __launch_bounds__((NW + (MX * 16 + 63) / 64) * 64) void w8a8_q8_stream_kernel(
    const int8_t* __restrict__ a, const float* __restrict__ a_s, int64_t as_sm, const int8_t* __restrict__ qt,
    const uint16_t* __restrict__ dt, void* __restrict__ out, int64_t ldo, const int32_t* __restrict__ n_rows, int M,
    int N, int K, unsigned long long* __restrict__ hand, unsigned tag) {
    constexpr int FW = (MX * 16 + 63) / 64;
    constexpr int NT = NW * 64;                    // compute threads; NT .. NT + 64 FW - 1 fold
    constexpr int RP = R / 2;                      // block pairs per round
    constexpr int CP = RP / NW;                    // block pairs per compute wave per round
    static_assert(CP >= 1 && CP * NW == RP, "R must be a multiple of 2 NW");
    static_assert(MX <= 16, "one 16-row activation tile");
    extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
    // terms [RD][M x 16 outputs][TL]: an output's R terms of a round are contiguous, so the fold reads them four at
    // a time; rows padded by 4 floats so the 16 lanes storing one pair's terms hit distinct banks
    constexpr int TL = R + 4;
    static_assert(TL % 2 == 0, "8-byte term stores");
    float* terms = reinterpret_cast<float*>(dsm);
    unsigned* wdone = reinterpret_cast<unsigned*>(terms + RD * M * 16 * TL);  // [RD]: compute waves done
    unsigned* fdone = wdone + RD;                                              // [RD]: fold waves done
    const int tstride = M * 16 * TL;
    // XL: the M activation rows, copied whole into LDS at the start ([M][K + 32] bytes: rows 32 bytes apart in the
    // banks, so the pieces of four rows a wave reads at once hit distinct banks), so the register ring carries only
    // the weight stream
    int8_t* xs = dsm + ((RD * M * 16 * TL * 4 + 2 * RD * 4 + 15) & ~15);

    // every argument fetched at once: the compiler would otherwise load each where first used, one scalar memory
    // round trip after another before the first weight request
    const int W = gridDim.x, v = blockIdx.x;
    asm volatile("" ::"s"(a), "s"(a_s), "s"(as_sm), "s"(qt), "s"(dt), "s"(out), "s"(ldo), "s"(n_rows), "s"(M), "s"(N),
                 "s"(K), "s"(hand), "s"(tag), "s"(W));
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int KP = K / 64;
    const int lm = lane & 15, q = lane >> 4;
    // the counters are cleared here and first used after the workgroup barrier that follows the first loads (no
    // barrier, and no global load the first weight requests would wait behind, before those requests go out)
    if (tid < 2 * RD) wdone[tid] = 0;

    // this workgroup's range of chunks (units: block pairs), walked from the last tile to the first
    const Walk walk(N / 16, KP, RP, W, v);
    const int NR = walk.NR;
    auto round_of = [&](int rho) -> Round { return walk.round(rho); };

    if (wv < NW) {
        // Compute wave: per round its CP block pairs; per lane and pair the weight chunk's 16-byte slot, the four
        // output rows' scales of both blocks (16 bytes of dt) and the two 8-byte pieces of the lane's activation row,
        // requested D - 1 rounds ahead.  Each block's int32 sums come from one MFMA (zero accumulator); the terms
        // RN(RN(float(P) sa) sw) go to ring slot r % RD once the fold waves have released it, then the wave counts
        // itself done for the round.  Waves run ahead of one another up to the ring's depth: no barriers.
        // Operands: the activation rows are the MFMA's A (lane l: row m = l % 16, 8-byte piece l / 16) and the weight
        // chunk's 16-byte slot its B as it lies (column n = l % 16), so lane l holds the sums of outputs
        // (m = 4 (l / 16) + e, n = l % 16): with MX <= 4 rows only e < MX of the lanes below 16 carry outputs, and the
        // epilogue works on those values alone; every lane's outputs share one weight row, whose two block scales
        // are one 4-byte word of dt.
        constexpr int EV = MX < 4 ? MX : 4;                            // accumulator values per lane in use
        const int mc = min(lm, M - 1);
        // buffer loads: per round the tile's base in SGPRs, per pair the offset in soffset, per lane one fixed
        // VGPR offset (weights: its 16-byte slot; scales: its row's 4-byte word; activations: its 8-byte piece)
        // activations: 16 bytes of the lane's row per pair, bytes 16 s .. 16 s + 15 with s = (0, 2, 1, 3)[q], which
        // one v_permlane16_swap per dword pair turns into the MFMA operand (lane q: bytes 8 q .. 8 q + 7 of each
        // block); one 16-byte request per lane instead of two 8-byte ones
        const int sq = ((q & 1) << 1) | (q >> 1);
        const uint32_t vw = 16 * lane, vs = 4 * lm, vx = (uint32_t)(mc * K + 16 * sq);
        const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a);
        const int wvu = __builtin_amdgcn_readfirstlane(wv);
        float sa[EV];
        struct Pair {
            v4i w;
            uint32_t s;
            v4i x;
        };
        auto load = [&](int rho, Pair* pr) {
            const Round d = round_of(rho);
            const int64_t tb = (int64_t)d.nt * KP;
            if (XL) {
#pragma unroll
                for (int i = 0; i < CP; i++) {
                    const int p = min(d.p0 + wv * CP + i, KP - 1);
                    pr[i].w = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(qt) + (tb + p) * 64 + lane);
                    pr[i].s = reinterpret_cast<const uint32_t*>(dt)[(tb + p) * 16 + lm];
                }
                return;
            }
            const __amdgpu_buffer_rsrc_t rw = buf_rsrc(qt + tb * 1024);
            const __amdgpu_buffer_rsrc_t rs = buf_rsrc(reinterpret_cast<const uint8_t*>(dt) + tb * 64);
#pragma unroll
            for (int i = 0; i < CP; i++) {
                const uint32_t p = (uint32_t)min(d.p0 + wvu * CP + i, KP - 1);
                pr[i].w = buf_load16<kBufNT>(rw, vw, p * 1024);
                pr[i].s = buf_load4(rs, vs, p * 64);
                pr[i].x = buf_load16(ra, vx, p * 64);
            }
        };
        auto compute = [&](int rho, const Pair* pr) {
            const Round d = round_of(rho);
            v4i acc[CP][2];
#pragma unroll
            for (int i = 0; i < CP; i++) {
                // lane q holds 8-byte units (u(2s), u(2s+1)) of the pair; after the swaps it holds (u(q), u(4 + q))
                uint32_t lo[2] = {0, 0}, hi[2] = {0, 0};
                if (!XL) {
                    const auto l2 = __builtin_amdgcn_permlane16_swap((uint32_t)pr[i].x[0], (uint32_t)pr[i].x[2], false,
                                                                     false);
                    const auto h2 = __builtin_amdgcn_permlane16_swap((uint32_t)pr[i].x[1], (uint32_t)pr[i].x[3], false,
                                                                     false);
                    lo[0] = l2[0], lo[1] = l2[1], hi[0] = h2[0], hi[1] = h2[1];
                }
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int64_t wf = h ? ((int64_t)(uint32_t)pr[i].w[2] | ((int64_t)pr[i].w[3] << 32))
                                         : ((int64_t)(uint32_t)pr[i].w[0] | ((int64_t)pr[i].w[1] << 32));
                    int64_t xf;
                    if (XL) {
                        const int p = min(d.p0 + wv * CP + i, KP - 1);
                        xf = *reinterpret_cast<const int64_t*>(xs + mc * (K + 32) + 64 * p + 32 * h + 8 * q);
                    } else {
                        xf = (int64_t)lo[h] | ((int64_t)hi[h] << 32);
                    }
                    const v4i zero = {0, 0, 0, 0};
                    acc[i][h] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xf, wf, zero, 0, 0, 0);
                }
            }
            float t[CP][2][EV];
#pragma unroll
            for (int i = 0; i < CP; i++)
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int e = 0; e < EV; e++) {
                        const float x = mul_rn((float)acc[i][h][e], sa[e]);
                        t[i][h][e] = h ? mul_f16_rn<1>(x, pr[i].s) : mul_f16_rn<0>(x, pr[i].s);
                    }
            const int slot = rho % RD;
            lds_wait_ge(&fdone[slot], (unsigned)(FW * (rho / RD)));      // slot released by the fold
            float* tb = terms + slot * tstride;
            // a pair's two block terms are adjacent: one 8-byte store each (3-6% faster than 4-byte stores at 1-16
            // rows; one 16-byte store of both pairs was slower from 8 rows)
#pragma unroll
            for (int i = 0; i < CP; i++)
#pragma unroll
                for (int e = 0; e < EV; e++) {
                    const int m = 4 * q + e;
                    if (m < M)
                        *reinterpret_cast<v2u*>(tb + (m * 16 + lm) * TL + 2 * (wv * CP + i)) =
                            v2u{__float_as_uint(t[i][0][e]), __float_as_uint(t[i][1][e])};
                }
            if (lane == 0) __hip_atomic_fetch_add(&wdone[slot], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        };
        // the first weight requests go out first; then the activation scales and (XL) the activation image, one
        // wave-wide 1 KB DMA per step, the image's last partial KB by the lanes it covers
        Pair ring[D][CP];
#pragma unroll
        for (int d = 0; d < D - 1; d++) load(d, ring[d]);
#pragma unroll
        for (int e = 0; e < EV; e++) sa[e] = a_s[(int64_t)min(4 * q + e, M - 1) * as_sm];
        if (XL) {
            const int cpr = (K + 1023) / 1024, nx = M * cpr;          // 1 KB copies per row, per image
            for (int c = wv; c < nx; c += NW) {
                const int m = c / cpr, k0 = (c - m * cpr) * 1024;
                if (k0 + lane * 16 < K) dma16(a + (int64_t)m * K + k0 + lane * 16, xs + m * (K + 32) + k0);
            }
        }
        __syncthreads();                          // counters cleared; with XL the activation image is in LDS
        // NR >= 1 (every workgroup has at least one chunk: W <= tiles), so the loop is entered unconditionally and
        // the prologue's requests are not sunk into a guarded block behind the barrier
        int r0 = 0;
        do {
#pragma unroll
            for (int d = 0; d < D; d++) {
                const int r = r0 + d;
                if (r < NR) {
                    load(r + D - 1, ring[(d + D - 1) % D]);   // past the end: clamped addresses, never used
                    compute(r, ring[d]);
                }
            }
            r0 += D;
        } while (r0 < NR);
    } else {
        // Fold wave: one output per thread (m = fo / 16, row fo % 16 of the tile), round by round in block order.
        const int fo = tid - NT;
        float y = 0.f;
        __syncthreads();
        const int live = min(M, __ldg(n_rows));
        // the word a tail continues from, read one round ahead (a predecessor publishes its head early, so the value
        // is normally there and the take costs no round trip); an untagged read falls back to polling
        unsigned long long pre = 0;
        // the running sums handed on: the compare-and-swap's result is checked once, at the end
        unsigned long long* pub = nullptr;
        unsigned long long pub_old = 0, pub_word = 0;
        for (int r = 0; r < NR; r++) {
            const Round d = round_of(r);
            const int slot = r % RD;
            if (r + 1 < NR && fo < M * 16) {
                const Round dn = round_of(r + 1);
                if (dn.first && dn.ps > 0) pre = hand_load(hand + (int64_t)(v - 1) * (MX * 16) + fo);
            }
            lds_wait_ge(&wdone[slot], (unsigned)(NW * (r / RD + 1)));
            if (fo < M * 16) {
                if (d.first) {
                    if (d.ps == 0) {
                        y = 0.f;
                    } else if ((pre >> 32) == tag) {
                        hand_store(hand + (int64_t)(v - 1) * (MX * 16) + fo, 0);
                        y = __uint_as_float((uint32_t)pre);
                    } else {
                        y = hand_take(hand + (int64_t)(v - 1) * (MX * 16) + fo, tag);
                    }
                }
                const float* tp = terms + slot * tstride + fo * TL;
                const int nb = 2 * d.np;
                float acc = y;
                if (nb == R) {
                    v4f u[R / 4];
#pragma unroll
                    for (int j = 0; j < R / 4; j++) u[j] = *reinterpret_cast<const v4f*>(tp + 4 * j);
#pragma unroll
                    for (int j = 0; j < R / 4; j++)
#pragma unroll
                        for (int e = 0; e < 4; e++) acc = add_rn(acc, u[j][e]);
                } else {
                    for (int j = 0; j < nb; j++) acc = add_rn(acc, tp[j]);
                }
                y = acc;
                if (d.last) {
                    if (d.pe < KP) {
                        pub = hand + (int64_t)v * (MX * 16) + fo;
                        pub_word = hand_word(y, tag);
                        pub_old = hand_publish(pub, pub_word);
                    } else {
                        const int m = fo >> 4, n = 16 * d.nt + (fo & 15);
                        if (m < live) {
                            if (EPI == 0) {
                                reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = (uint16_t)f32_to_bf16(y);
                            } else {
                                float* op = reinterpret_cast<float*>(out) + (int64_t)m * ldo + n;
                                *op = add_rn(*op, y);
                            }
                        }
                    }
                }
            }
            // the wave's reads of the slot are complete before it is counted released
            if (lane == 0) __hip_atomic_fetch_add(&fdone[slot], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        // a consumer that gave up on the word (never expected) or a stale word of another launch: settle it
        if (pub) hand_settle(pub, pub_old, pub_word);
    }
}

static size_t stream_lds(int R, int RD, int M, int K, bool xl) {
    const size_t base = (size_t)RD * M * 16 * (R + 4) * 4 + 2 * RD * 4;
    return xl ? ((base + 15) & ~(size_t)15) + (size_t)M * (K + 32) : base;
}
constexpr size_t kLdsMax = 160 * 1024;

int q8_stream_workgroups(int64_t N, int64_t K) {
    const int64_t tiles = N / 16;
    (void)K;
    return (int)(tiles < kQ8StreamMaxWG ? tiles : kQ8StreamMaxWG);
}

template <int EPI>
static void launch(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt, const uint16_t* dt, void* out,
                   int64_t ldo, const int32_t* n_rows, int M, int N, int K, unsigned long long* hand, int W,
                   hipStream_t st) {
    const unsigned tag = hand_next_tag();
#define QS(NW, R, MX, D, RD)                                                                                        \
    do {                                                                                                            \
        constexpr int NTH = (NW + (MX * 16 + 63) / 64) * 64;                                                        \
        if (Q8S_XL && stream_lds(R, RD, M, K, true) <= kLdsMax) {                                                   \
            auto fn = w8a8_q8_stream_kernel<NW, R, MX, D, RD, EPI, true>;                                           \
            allow_lds(fn, stream_lds(R, RD, M, K, true));                                                           \
            hipLaunchKernelGGL(fn, dim3(W), dim3(NTH), stream_lds(R, RD, M, K, true), st, a, a_s, as_sm, qt, dt,    \
                               out, ldo, n_rows, M, N, K, hand, tag);                                               \
        } else {                                                                                                    \
            auto fn = w8a8_q8_stream_kernel<NW, R, MX, D, RD, EPI, false>;                                          \
            allow_lds(fn, stream_lds(R, RD, M, K, false));                                                          \
            hipLaunchKernelGGL(fn, dim3(W), dim3(NTH), stream_lds(R, RD, M, K, false), st, a, a_s, as_sm, qt, dt,   \
                               out, ldo, n_rows, M, N, K, hand, tag);                                               \
        }                                                                                                           \
    } while (0)
#ifndef Q8S_XL
#define Q8S_XL 0
#endif
#ifndef Q8S_SMALL
#define Q8S_SMALL 12, 48, 4, 2, 4
#endif
#ifndef Q8S_ONE
#define Q8S_ONE 12, 48, 1, 2, 4
#endif
#ifndef Q8S_BIG
#define Q8S_BIG 8, 32, 16, 2, 2
#endif
#ifndef Q8S_ONE10
#define Q8S_ONE10 10, 40, 1, 2, 4
#endif
#ifndef Q8S_SMALL10
#define Q8S_SMALL10 10, 40, 4, 2, 4
#endif
#ifndef Q8S_WIDE10
#define Q8S_WIDE10 10, 40, 16, 2, 2
#endif
#ifndef Q8S_WIDE
#define Q8S_WIDE 12, 48, 16, 2, 2
#endif
#define QS_(...) QS(__VA_ARGS__)
    // 5..16 rows (activations in the ring): twelve compute waves and 24-pair rounds up to 12 rows, eight waves and
    // 16-pair rounds beyond (measured at 5120 x 17408: 8 rows 23.7 -> 20.9 us and 12 rows 24.8 -> 22.8 us with twelve,
    // 16 rows 0.5-0.9 us slower with twelve).  With the XL build option the image forms come first where they fit:
    // twelve waves where a workgroup's share spans four 24-pair rounds, else eight.
    const bool wide = (int64_t)(N / 16) * (K / 64) >= 4LL * 24 * W;
    // every row count: ten compute waves (20-pair rounds) instead of twelve (24) when that takes no more rounds of a
    // workgroup's share (5120^2, 100 pairs: five full rounds, 8.1 -> 7.7 us at one row; at 4096^2 and 5120 x 17408,
    // where twelve waves need fewer rounds, twelve are 0.3-3 us faster)
    const int64_t share = ((int64_t)(N / 16) * (K / 64) + W - 1) / W;
    const bool ten = (share + 19) / 20 <= (share + 23) / 24;
    if (M == 1 && ten) QS_(Q8S_ONE10);
    else if (M == 1) QS_(Q8S_ONE);
    else if (M <= 4 && ten) QS_(Q8S_SMALL10);
    else if (M <= 4) QS_(Q8S_SMALL);
    else if (Q8S_XL && wide && stream_lds(48, 2, M, K, true) <= kLdsMax) QS_(Q8S_WIDE);
    else if (ten && M > 12) QS_(Q8S_WIDE10);        // 5120^2 at 16 rows 11.1 -> 10.1 us
    else if (M > 12 && wide) QS_(Q8S_WIDE);         // 5120 x 17408 at 13 rows 25.5-26.8 -> 23.8-24.4 us, 16 a tie
    else if ((Q8S_XL && stream_lds(32, 2, M, K, true) <= kLdsMax) || M > 12) QS_(Q8S_BIG);
    else if (ten) QS_(Q8S_WIDE10);                  // as at 1-4 rows (5120^2 at 12 rows 10.3 -> 9.2 us)
    else QS_(Q8S_WIDE);
#undef QS_
#undef QS
}

int q8_stream_launch(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt, const uint16_t* dt,
                     void* out, int64_t ldo, const int32_t* n_rows, int64_t M, int64_t N, int64_t K, int epi,
                     void* hand, int64_t hand_bytes, hipStream_t st) {
    if (M < 1 || M > 16 || (N / 16) * (K / 64) >= ((int64_t)1 << 31) || M * K >= ((int64_t)1 << 31))
        return PRISM_ERR_SHAPE;                  // 32-bit chunk and activation offsets
    const int W = q8_stream_workgroups(N, K);
    if (!hand || !PRISM_ALIGNED(hand, 8) || hand_bytes < q8_stream_workspace_bytes(N, K)) return PRISM_ERR_ARG;
    auto* h = reinterpret_cast<unsigned long long*>(hand);
    if (epi == 0)
        launch<0>(a, a_s, as_sm, qt, dt, out, ldo, n_rows, (int)M, (int)N, (int)K, h, W, st);
    else
        launch<1>(a, a_s, as_sm, qt, dt, out, ldo, n_rows, (int)M, (int)N, (int)K, h, W, st);
    return PRISM_OK;
}

int64_t q8_stream_workspace_bytes(int64_t N, int64_t K) {
    return (int64_t)q8_stream_workgroups(N, K) * 16 * 16 * 8;
}

}  // namespace prism
