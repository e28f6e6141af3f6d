// W4A8 decode on Q4_K weights (M <= 16) streamed by a balanced grid (gfx950): the Q8_0 "stream" kernel's structure
// (w8a8_q8_stream.hip) on Q4_K super-blocks.
//
// Units are (16-row weight tile, super-block): 2 KB of packed nibbles and 256 bytes of meta.  W workgroups (one per CU
// at most) take equal ranges of the projection's units and hand running sums across tile boundaries (handoff.h), so
// every CU streams the same bytes whatever N / 16 is.  Inside a workgroup NW compute waves take a round's units (one
// each) and FW fold waves add finished terms in super-block order, meeting at LDS counters (no barriers in the loop).
// The activation rows (padded 32 bytes per row, so a wave's 16-byte reads of different rows fall in different banks),
// their split sums and their scales are copied into LDS once at the start; the register ring carries only the weight
// stream, one round ahead.
//
// Arithmetic per output (m, n) and super-block b, as every W4A8 kernel (kernels/w4a8.py:14-22, 177-199): acc over the
// eight sub-blocks (two-plane MFMA weight operands, exact), mins on the MFMA (exact), t = q4k_term(d, dmin, acc,
// mins), then y = fma(a[b, m], t, y) in increasing b.  The terms and the chain are the stream kernel's bit for bit.
#include "common.h"
#include "handoff.h"
#include "w4a8_bal.h"
#include "w4a8_common.h"

namespace prism {

template <int NW, int MX, int RD, int EPI>
__global__ __launch_bounds__((NW + (MX * 16 + 63) / 64) * 64) void w4a8_q4k_bal_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ a, int64_t a_sb, const int8_t* __restrict__ xs,
    const uint8_t* __restrict__ qv, const uint8_t* __restrict__ meta, void* __restrict__ out, int64_t ldo,
    const int32_t* __restrict__ n_rows, int M, int N, int K, unsigned long long* __restrict__ hand, unsigned tag) {
    constexpr int FW = (MX * 16 + 63) / 64;
    constexpr int NT = NW * 64;                    // compute threads; NT .. NT + 64 FW - 1 fold
    constexpr int RP = NW;                         // super-blocks per round, one per compute wave
    static_assert(MX <= 16, "one 16-row activation tile");
    const int W = gridDim.x, v = blockIdx.x;
    kernel_args_now(xq, a, a_sb, xs, qv, meta, out, ldo, n_rows, M, N, K, hand, tag, W);
    const int NB = K / 256;
    const int LDX = K + 32;                        // activation image row (bytes)
    extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
    // LDS: terms [RD][RP][M x 16] (a unit's terms of all outputs contiguous: one 16-byte store per lane), the
    // counters, the activation image [M][LDX], the split sums [NB][M][16] and the scales [NB][M] (or [M])
    float* terms = reinterpret_cast<float*>(dsm);
    unsigned* wdone = reinterpret_cast<unsigned*>(terms + RD * RP * M * 16);
    unsigned* fdone = wdone + RD;
    int8_t* xl = dsm + ((RD * RP * M * 16 * 4 + 2 * RD * 4 + 15) & ~15);
    int8_t* sl = xl + M * LDX;
    float* al = reinterpret_cast<float*>(sl + NB * M * 16);
    const int tstride = RP * M * 16;
    const int NA = a_sb ? NB : 1;                  // scale rows: one per super-block, or one per token

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int lm = lane & 15, q = lane >> 4;
    if (tid < 2 * RD) wdone[tid] = 0;
    const Walk walk(N / 16, NB, RP, W, v);
    const int NR = walk.NR;

    if (wv < NW) {
        // Compute wave: super-block p0 + wv of each round.  Lane (lm, q): weight row lm of the tile and activation
        // row lm (clamped); the MFMA leaves lane l the sums of outputs (n = 4 q + e, m = lm).
        const int m = min(lm, M - 1);
        const v4u* cw = reinterpret_cast<const v4u*>(qv) + lane;
        const v4u* cm = reinterpret_cast<const v4u*>(meta) + lm;
        struct Unit {
            v4u w[2];
            v4u mt;
        };
        auto load = [&](int rho, Unit& u) {
            const Round d = walk.round(rho);
            const int64_t c = (int64_t)d.nt * NB + min(d.p0 + wv, NB - 1);
            u.w[0] = __builtin_nontemporal_load(cw + c * 128);
            u.w[1] = __builtin_nontemporal_load(cw + c * 128 + 64);
            u.mt = cm[c * 16];
        };
        // the first weights go out before anything else; then the activation image, sums and scales
        Unit ring[2];
        load(0, ring[0]);
        {
            const int cpr = (K + 1023) / 1024;
            for (int c = wv; c < M * cpr; c += NW) {
                const int mm = c / cpr, k0 = (c - mm * cpr) * 1024;
                if (k0 + lane * 16 < K) dma16(xq + (int64_t)mm * K + k0 + lane * 16, xl + mm * LDX + k0);
            }
            const int sb = NB * M * 16;                // the split sums as they lie
            for (int c = wv; c < (sb + 1023) / 1024; c += NW)
                if (c * 1024 + lane * 16 < sb) dma16(xs + c * 1024 + lane * 16, sl + c * 1024);
            for (int i = tid; i < NA * M; i += NT) al[i] = a[(int64_t)(i / M) * a_sb + i % M];
        }
        __syncthreads();                           // counters cleared; activation image, sums and scales in LDS
        const int8_t* xrow = xl + m * LDX + 16 * q;
        int r = 0;
        do {                                       // NR >= 1: every workgroup has a unit (W <= tiles)
#pragma unroll
            for (int d = 0; d < 2; d++) {
                const int rho = r + d;
                if (rho < NR) {
                    load(rho + 1, ring[(d + 1) & 1]);  // past the end: clamped addresses, never used
                    const Round rd = walk.round(rho);
                    const Unit& u = ring[d];
                    const int b = min(rd.p0 + wv, NB - 1);
                    const float dd = f16_to_f32(u.mt[0] & 0xffffu), dm = f16_to_f32(u.mt[0] >> 16);
                    uint32_t sp[4];
                    q4k_lane_splits(u.mt, q >> 1, sp);
                    v4i alo = {0, 0, 0, 0}, ahi = {0, 0, 0, 0};
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        v4i wl, wh;
                        two_plane(u.w[p >> 1][2 * (p & 1)], u.w[p >> 1][2 * (p & 1) + 1], sp[p], wl, wh);
                        const v4i x = *reinterpret_cast<const v4i*>(xrow + b * 256 + 64 * p);
                        alo = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl, x, alo, 0, 0, 0);
                        ahi = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh, x, ahi, 0, 0, 0);
                    }
                    const v4i s = *reinterpret_cast<const v4i*>(sl + (b * M + m) * 16);
                    const int64_t mn8 = q == 0 ? q4k_mins8(u.mt) : 0;
                    const int64_t slo = q == 0 ? ((int64_t)(uint32_t)s[0] | ((int64_t)(uint32_t)s[1] << 32)) : 0;
                    const int64_t shi = q == 0 ? ((int64_t)(uint32_t)s[2] | ((int64_t)(uint32_t)s[3] << 32)) : 0;
                    const v4i mins = mins_mfma(mn8, slo, shi);
                    v4f t;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float de = __shfl(dd, 4 * q + e, kWave), dme = __shfl(dm, 4 * q + e, kWave);
                        t[e] = q4k_term(de, dme, alo[e] + 8 * ahi[e], mins[e]);
                    }
                    const int slot = rho % RD;
                    lds_wait_ge(&fdone[slot], (unsigned)(FW * (rho / RD)));    // slot released by the fold
                    if (lm < M && wv < rd.np)
                        *reinterpret_cast<v4f*>(&terms[slot * tstride + wv * M * 16 + lm * 16 + 4 * q]) = t;
                    if (lane == 0)
                        __hip_atomic_fetch_add(&wdone[slot], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
            r += 2;
        } while (r < NR);
    } else {
        // Fold wave: one output per thread (m = fo / 16, row fo % 16 of the tile), round by round in super-block
        // order, y = fma(a[b, m], t, y).
        const int fo = tid - NT;
        const int mo = fo >> 4;
        float y = 0.f;
        __syncthreads();
        const int live = min(M, __ldg(n_rows));
        unsigned long long pre = 0, pub_old = 0, pub_word = 0;
        unsigned long long* pub = nullptr;
        for (int r = 0; r < NR; r++) {
            const Round d = walk.round(r);
            const int slot = r % RD;
            if (r + 1 < NR && fo < M * 16) {
                const Round dn = walk.round(r + 1);
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
                const float* tp = terms + slot * tstride + fo;
                float acc = y;
                for (int j = 0; j < d.np; j++)
                    acc = fmaf(al[(a_sb ? d.p0 + j : 0) * M + mo], tp[j * M * 16], acc);
                y = acc;
                if (d.last) {
                    if (d.pe < NB) {
                        pub = hand + (int64_t)v * (MX * 16) + fo;
                        pub_word = hand_word(y, tag);
                        pub_old = hand_publish(pub, pub_word);
                    } else if (mo < live) {
                        const int n = 16 * d.nt + (fo & 15);
                        if (EPI == 0) {
                            reinterpret_cast<uint16_t*>(out)[(int64_t)mo * ldo + n] = (uint16_t)f32_to_bf16(y);
                        } else {
                            float* op = reinterpret_cast<float*>(out) + (int64_t)mo * ldo + n;
                            *op = add_rn(*op, y);
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

constexpr int kQ4BalNW = 12;
constexpr int kQ4BalRD = 3;

static size_t q4k_bal_lds(int64_t M, int64_t K) {
    const size_t terms = (size_t)kQ4BalRD * kQ4BalNW * M * 16 * 4 + 2 * kQ4BalRD * 4;
    const size_t NB = (size_t)K / 256;
    return ((terms + 15) & ~(size_t)15) + (size_t)M * (K + 32) + NB * M * 16 + NB * M * 4;
}

int q4k_bal_workgroups(int64_t N) { return (int)(N / 16 < 256 ? N / 16 : 256); }

bool q4k_bal_fits(int64_t M, int64_t N, int64_t K) {
    return M >= 1 && M <= 16 && (N / 16) * (K / 256) < ((int64_t)1 << 31) && q4k_bal_lds(M, K) <= 160 * 1024;
}

int64_t q4k_bal_workspace_bytes(int64_t N) { return (int64_t)q4k_bal_workgroups(N) * 16 * 16 * 8; }

template <int MX, int EPI>
static void q4k_bal_run(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs, const uint8_t* qv,
                        const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K,
                        unsigned long long* hand, hipStream_t st) {
    auto fn = w4a8_q4k_bal_kernel<kQ4BalNW, MX, kQ4BalRD, EPI>;
    const unsigned tag = hand_next_tag();
    const size_t lds = q4k_bal_lds(M, K);
    allow_lds(fn, lds);
    hipLaunchKernelGGL(fn, dim3(q4k_bal_workgroups(N)), dim3((kQ4BalNW + (MX * 16 + 63) / 64) * 64), lds, st, xq, a,
                       a_sb, xs, qv, meta, out, ldo, n_rows, M, N, K, hand, tag);
}

int q4k_bal_launch(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs, const uint8_t* qv,
                   const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int64_t M, int64_t N,
                   int64_t K, int epi, void* hand, int64_t hand_bytes, hipStream_t st) {
    if (!q4k_bal_fits(M, N, K)) return PRISM_ERR_SHAPE;
    if (!hand || !PRISM_ALIGNED(hand, 8) || hand_bytes < q4k_bal_workspace_bytes(N)) return PRISM_ERR_ARG;
    auto* h = reinterpret_cast<unsigned long long*>(hand);
    const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
    if (M <= 4) {
        if (epi == 0) q4k_bal_run<4, 0>(xq, a, a_sb, xs, qv, meta, out, ldo, n_rows, Mi, Ni, Ki, h, st);
        else q4k_bal_run<4, 1>(xq, a, a_sb, xs, qv, meta, out, ldo, n_rows, Mi, Ni, Ki, h, st);
    } else {
        if (epi == 0) q4k_bal_run<16, 0>(xq, a, a_sb, xs, qv, meta, out, ldo, n_rows, Mi, Ni, Ki, h, st);
        else q4k_bal_run<16, 1>(xq, a, a_sb, xs, qv, meta, out, ldo, n_rows, Mi, Ni, Ki, h, st);
    }
    return PRISM_OK;
}

}  // namespace prism
