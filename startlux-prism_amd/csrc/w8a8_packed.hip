// Q8_0 W8A8 GEMM on an MFMA-native weight layout (gfx950).
//
// Packed layout, made once at load (prism_q8_0_pack), like the reference's own load-time repacks
// (kernels/w8a8.py:274-286 weight_from_q8, kernels/w4a8.py:70-94 repack):
//   qt  int8 [N/16][K/64][64][16]: one 1 KB chunk per (16-row tile nt, block pair j).  Lane slot l holds row
//       16 nt + l % 16, q = l / 16: bytes 0..7 = k 64 j + 8 q .. +8 (block 2 j), bytes 8..15 = k 64 j + 32 + 8 q .. +8
//       (block 2 j + 1).  One dwordx4 per lane reads a whole chunk (1 KB contiguous per wave instruction) and its
//       halves are the A operands of v_mfma_i32_16x16x32_i8 for the two blocks, with no re-layout.
//   dt  fp16 [N/16][K/64][16][2]: the Q8_0 block scales of the chunk, row-major over (row, block of the pair), so a
//       lane's four output rows 4 (l / 16) .. +3 are one 16-byte load.
// Per-channel int8 weights (prism_i8_pack, no blocks to keep apart) use the same chunks with lane slot l holding
// inputs 64 j + 16 q .. + 15 of its row: the 16-byte operand of v_mfma_i32_16x16x64_i8 / 32x32x32_i8 as it lies.
// Arithmetic: identical to the row-major kernels (kernels/w8a8.py:64-85), every output's fp32 sum over blocks in
// block order, so both layouts give the same bits.
#include <mutex>

#include "common.h"
#include "q8_stream.h"


namespace prism {

// ---------------------------------------------------------------------------------------------- pack
__global__ __launch_bounds__(256) void q8_0_pack_kernel(const int8_t* __restrict__ qs, const uint16_t* __restrict__ d,
                                                        int8_t* __restrict__ qt, uint16_t* __restrict__ dt, int N,
                                                        int K) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;     // (nt, j, l)
    const int KP = K / 64;
    const int64_t total = (int64_t)(N / 16) * KP * 64;
    if (e >= total) return;
    const int l = (int)(e & 63), r = l & 15, q = l >> 4;
    const int64_t c = e >> 6;
    const int j = (int)(c % KP), nt = (int)(c / KP);
    if (!d) {                                          // per-channel: inputs 16 q .. 16 q + 15 of the chunk
        reinterpret_cast<v4u*>(qt)[e] =
            *reinterpret_cast<const v4u*>(qs + (int64_t)(16 * nt + r) * K + 64 * j + 16 * q);
        return;
    }
    const int8_t* src = qs + (int64_t)(16 * nt + r) * K + 64 * j + 8 * q;
    v2u lo = *reinterpret_cast<const v2u*>(src), hi = *reinterpret_cast<const v2u*>(src + 32);
    v4u o;
    o[0] = lo[0];
    o[1] = lo[1];
    o[2] = hi[0];
    o[3] = hi[1];
    reinterpret_cast<v4u*>(qt)[e] = o;
    if (q == 0 && dt) {                                // 16 rows x 2 blocks of scales per chunk
        const int G = K / 32;
        dt[(c * 16 + r) * 2 + 0] = d[(int64_t)(16 * nt + r) * G + 2 * j];
        dt[(c * 16 + r) * 2 + 1] = d[(int64_t)(16 * nt + r) * G + 2 * j + 1];
    }
}

// ---------------------------------------------------------------------------------------------- decode
// A workgroup of NW waves owns one 16-row tile and every activation row (M <= MX <= 64).  Round r covers R blocks;
// wave w takes block pairs r R / 2 + w CP .. + CP - 1.  Per round, the only per-wave global loads are the weight
// chunks (one dwordx4 per lane per 1 KB chunk, requested D - 1 rounds ahead); the round's block scales (1 KB) and
// activation rows (M R 32 bytes) are fetched by all threads with row-contiguous 16-byte loads and staged in one of
// two LDS buffers a round ahead.  Each block's int32 sums come from one MFMA on a chunk half, become the term
// RN(RN(float(P) sa) sw) and go to one of two LDS term buffers [block][m][n].  FW more waves own the outputs: each
// of their threads adds round r - 1's terms of one output in block order (the reference's sequential fp32 sum over
// groups) while the NW compute waves compute round r, so the fold's serial chain overlaps the weight stream; one
// barrier per round separates producers from consumers of every buffer.
template <int NW, int FW, int R, int MX, int D, int EPI>
__global__ __launch_bounds__((NW + FW) * 64) void w8a8_packed_decode_kernel(const int8_t* __restrict__ a,
                                                                     const float* __restrict__ a_s, int64_t as_sm,
                                                                     const int8_t* __restrict__ qt,
                                                                     const uint16_t* __restrict__ dt,
                                                                     void* __restrict__ out, int64_t ldo,
                                                                     const int32_t* __restrict__ n_rows, int M, int N,
                                                                     int K) {
    constexpr int MT = (MX + 15) / 16;             // activation tiles of 16 rows
    constexpr int NT = NW * 64;                    // compute threads; threads NT .. NT + 64 FW - 1 fold
    static_assert(FW * 64 >= MX * 16, "one fold thread per output");
    constexpr int CP = R / (2 * NW);               // block pairs per wave per round
    static_assert(CP >= 1 && CP * 2 * NW == R, "R must be a multiple of 2 NW");
    constexpr int RB = R * 32;                     // activation bytes per row per round
    constexpr int LDA = RB + 16;                   // padded LDS activation row
    constexpr int CPR = RB / 16;                   // 16-byte chunks per activation row per round
    constexpr int XPT = (MX * CPR + NT - 1) / NT;
    constexpr int SCH = R * 16 * 2 / 16;           // 16-byte chunks of scales per round (16 rows x R fp16)
    constexpr int SPT = (SCH + NT - 1) / NT;
    extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
    float* terms = reinterpret_cast<float*>(dsm);                              // [2][R][M][16]
    float* sws = terms + 2 * R * M * 16;                                       // [2][R][16]
    int8_t* xs = reinterpret_cast<int8_t*>(sws + 2 * R * 16);                  // [2][M][LDA]
    const int tstride = R * M * 16, xstride = M * LDA;

    kernel_args_now(a, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nt = blockIdx.x;
    const int live = min(M, __ldg(n_rows));
    const int KP = K / 64, G = K / 32;
    const int nr = (G + R - 1) / R;
    const int lm = lane & 15, q = lane >> 4;
    const int xch = M * CPR;

    const v4i* cw = reinterpret_cast<const v4i*>(qt) + (int64_t)nt * KP * 64 + lane;
    const v4u* cs = reinterpret_cast<const v4u*>(dt) + (int64_t)nt * KP * 4;
    float sa[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) sa[mt] = a_s[(int64_t)min(mt * 16 + lm, M - 1) * as_sm];

    // a round's scales and activation chunks: loaded unconditionally (indices clamped in range), stored to LDS
    // conditionally
    struct Staged {
        v4u s[SPT];
        v4i x[XPT];
    };
    auto stage_load = [&](int r, Staged& sg) {
        const int p0 = r * (R / 2);
#pragma unroll
        for (int i = 0; i < SPT; i++) {
            const int sc = min(tid + i * NT, SCH - 1);                 // 4 chunks of 16 bytes per pair
            sg.s[i] = cs[(int64_t)min(p0 + sc / 4, KP - 1) * 4 + (sc & 3)];
        }
        const int64_t k0 = (int64_t)r * RB;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int c = min(tid + i * NT, xch - 1);
            const int64_t kk = min(k0 + (c % CPR) * 16, (int64_t)K - 16);
            sg.x[i] = *reinterpret_cast<const v4i*>(a + (int64_t)(c / CPR) * K + kk);
        }
    };
    auto stage_store = [&](const Staged& sg, int buf) {
        float* sp = sws + buf * R * 16;
#pragma unroll
        for (int i = 0; i < SPT; i++) {
            const int sc = tid + i * NT;
            if (sc < SCH) {                                            // pair sc / 4, rows 4 (sc % 4) .. +3
                const int pl = sc >> 2, r0 = 4 * (sc & 3);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sp[(2 * pl) * 16 + r0 + e] = f16_to_f32(sg.s[i][e] & 0xffffu);
                    sp[(2 * pl + 1) * 16 + r0 + e] = f16_to_f32(sg.s[i][e] >> 16);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int c = tid + i * NT;
            if (c < xch) *reinterpret_cast<v4i*>(&xs[buf * xstride + (c / CPR) * LDA + (c % CPR) * 16]) = sg.x[i];
        }
    };
    auto load_w = [&](int r, v4i* w) {
#pragma unroll
        for (int i = 0; i < CP; i++)
            w[i] = __builtin_nontemporal_load(cw + (int64_t)min(r * (R / 2) + wv * CP + i, KP - 1) * 64);
    };
    auto compute = [&](int r, const v4i* w, int buf) {
        const float* sp = sws + buf * R * 16;
        const int8_t* xp = xs + buf * xstride;
        float* tb = terms + (r & 1) * tstride;
#pragma unroll
        for (int i = 0; i < CP; i++) {
            const int lp = wv * CP + i;                                // pair within the round
            if (r * (R / 2) + lp < KP) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int lb = 2 * lp + h;
                    const int64_t wf = h ? ((int64_t)(uint32_t)w[i][2] | ((int64_t)w[i][3] << 32))
                                         : ((int64_t)(uint32_t)w[i][0] | ((int64_t)w[i][1] << 32));
                    const v4f sw = *reinterpret_cast<const v4f*>(&sp[lb * 16 + 4 * q]);
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        const int m = mt * 16 + lm;
                        const int64_t xf = *reinterpret_cast<const int64_t*>(&xp[min(m, M - 1) * LDA + lb * 32 + 8 * q]);
                        const v4i zero = {0, 0, 0, 0};
                        const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf, xf, zero, 0, 0, 0);
                        v4f t;
#pragma unroll
                        for (int e = 0; e < 4; e++) t[e] = mul_rn(mul_rn((float)acc[e], sa[mt]), sw[e]);
                        if (m < M) *reinterpret_cast<v4f*>(&tb[(lb * M + m) * 16 + 4 * q]) = t;
                    }
                }
            }
        }
    };
    const bool folder = wv >= NW;
    const int fo = tid - NT;                                           // the fold thread's output (m = fo / 16)
    float y = 0.f;
    auto fold = [&](int r) {
        if (fo < M * 16) {
            const float* tp = terms + (r & 1) * tstride + fo;
            const int nb = min(R, G - r * R);
            const int st = M * 16;
            float acc = y;
            int j = 0;
            for (; j + 16 <= nb; j += 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = tp[(j + u) * st];
#pragma unroll
                for (int u = 0; u < 16; u++) acc = add_rn(acc, v[u]);
            }
            for (; j < nb; j++) acc = add_rn(acc, tp[j * st]);
            y = acc;
        }
    };

    // prologue: round 0 staged in LDS buffer 0; rounds 1 .. D's scales and activations in the register ring sg
    // (round q in slot q % D, loaded D rounds before it is stored); weights of rounds 0 .. D-2
    v4i wr[D][CP];
    Staged sg[D];
    if (!folder) {
#pragma unroll
        for (int d = 0; d < D - 1; d++) load_w(d, wr[d]);
        stage_load(0, sg[0]);
        stage_store(sg[0], 0);
#pragma unroll
        for (int d = 1; d <= D; d++) stage_load(d, sg[d % D]);
    }
    lds_barrier();
    for (int r0 = 0; r0 < nr; r0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int r = r0 + d;
            if (!folder) {
                load_w(r + D - 1, wr[(d + D - 1) % D]);    // past the end: the last chunk again (a cache hit)
                stage_store(sg[(d + 1) % D], (r + 1) & 1);  // round r + 1's scales and activations
                stage_load(r + 1 + D, sg[(d + 1) % D]);     // the slot's next round
                if (r < nr) compute(r, wr[d], r & 1);
            } else if (r >= 1 && r <= nr) {
                fold(r - 1);
            }
            lds_barrier();
        }
    }
    if (nr % D == 0 && folder) fold(nr - 1);
    const int m = fo >> 4, n = 16 * nt + (fo & 15);
    if (folder && fo < M * 16 && m < live) {
        if (EPI == 0) {
            reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = (uint16_t)f32_to_bf16(y);
        } else {
            float* op = reinterpret_cast<float*>(out) + (int64_t)m * ldo + n;
            *op = add_rn(*op, y);
        }
    }
}

// ---------------------------------------------------------------------------------------------- prefill tile
// 128 x 128 output tile per 256-thread workgroup (2 x 2 waves of 64 x 64), v_mfma_i32_32x32x32_i8 per (32 x 32,
// block), 4 blocks (2 chunk pairs) per stage.  The weight tile of a stage is 8 tiles x 2 chunks = 8 runs of 2 KB,
// copied to LDS as they are; a B fragment (column n, 16 bytes of a block) is two 8-byte pieces of a chunk.
constexpr int PBM = 128, PBN = 128;
constexpr int PLDA = 128 + 16;          // activation tile row (bytes), padded
constexpr int PLDB = 2048 + 64;         // one 16-row tile's two chunks, padded

// RA: the reassociated order (one activation scale per token, factored out of the block sum): per block
// y = fma(float(P), sw, y), then y = RN(y sa) once; 2 VALU operations per output and block instead of 4.
// PAN: `a` is the panel copy of q8_act_panel_kernel, so a wave's activation load for a stage is one 1 KB piece
// (8 rows x 128 bytes of the tile's 16 KB stage chunk) instead of 8 rows' 128 bytes K apart.
template <int EPI, bool RA, bool PAN = false>
__global__ __launch_bounds__(256, 2) void w8a8_packed_tile_kernel(const int8_t* __restrict__ a,
                                                                  const float* __restrict__ a_s, int64_t as_sm,
                                                                  const int8_t* __restrict__ qt,
                                                                  const uint16_t* __restrict__ dt,
                                                                  void* __restrict__ out, int64_t ldo,
                                                                  const int32_t* __restrict__ n_rows, int M, int N,
                                                                  int K, int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(16))) int8_t As[PBM * PLDA];
    __shared__ __attribute__((aligned(16))) int8_t Bs[8 * PLDB];
    __shared__ float sws[4][PBN];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv >> 1, wn = wv & 1;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * PBM, n0 = pn * PBN;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int G = K / 32, KP = K / 64;
    const int nt0 = n0 / 16, ntiles = N / 16;

    // activation loader: chunk i = row lr + 32 i, bytes lc .. lc + 15 of the stage's 128 bytes
    const int lr = tid >> 3, lc = (tid & 7) * 16;
    const int8_t* ap[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (PAN) {                                   // the tile's panel: row lr + 32 i of each 16 KB stage chunk
            ap[i] = a + (int64_t)m0 * K + (lr + 32 * i) * 128 + lc;
        } else {
            ap[i] = a + (int64_t)min(m0 + lr + 32 * i, M - 1) * K + lc;
        }
    }
    // weight loader: chunk c = tid + 256 i -> tile c / 128 (clamped in range), 16 bytes (c % 128) of its 2 KB run
    const v4i* bp[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = tid + 256 * i;
        const int t = min(nt0 + (c >> 7), ntiles - 1);
        bp[i] = reinterpret_cast<const v4i*>(qt) + (int64_t)t * KP * 64 + (c & 127);
    }
    // scale loader: thread t < 64 -> tile t / 8, 16 bytes (t % 8) of the tile's 2 x 64 bytes (2 pairs)
    const int st_t = min(nt0 + (tid >> 3), ntiles - 1);
    const v4u* sp = reinterpret_cast<const v4u*>(dt) + (int64_t)st_t * KP * 4 + (tid & 7);

    v4i ra[4], rb[4];
    v4u rs;
    auto gload = [&](int kb) {                       // kb: first block of the stage (a multiple of 4)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            ra[i] = *reinterpret_cast<const v4i*>(ap[i] + (PAN ? (int64_t)(kb / 4) * 16384 : (int64_t)kb * 32));
            rb[i] = __builtin_nontemporal_load(bp[i] + (int64_t)(kb / 2) * 64);
        }
        rs = sp[(int64_t)(kb / 2) * 4];
    };

    const int lrow = 4 * (lane >> 5);
    float sa[2][16];
    auto load_sa = [&]() {
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = min(m0 + wm * 64 + mt * 32 + 8 * (r >> 2) + lrow + (r & 3), M - 1);
                sa[mt][r] = a_s[(int64_t)m * as_sm];
            }
    };
    if (!RA) load_sa();                              // RA applies the scales once, after the K loop
    float y[2][2][16];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int r = 0; r < 16; r++) y[mt][nt][r] = 0.f;

    const int arow0 = (wm * 64 + (lane & 31)) * PLDA + (lane >> 5) * 16;
    // B fragment of column j = wn * 64 + nt * 32 + lane % 32 (tile-local), lane group g = lane / 32: pieces
    // q = 2 g and 2 g + 1 of row j % 16 in 16-row tile j / 16
    int bofs[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int j = wn * 64 + t * 32 + (lane & 31);
        bofs[t] = (j >> 4) * PLDB + ((j & 15) + 32 * (lane >> 5)) * 16;
    }
    const int swc = wn * 64 + (lane & 31);
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    gload(0);
    for (int kb = 0; kb < G; kb += 4) {
        lds_barrier();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<v4i*>(&As[(lr + 32 * i) * PLDA + lc]) = ra[i];
            *reinterpret_cast<v4i*>(&Bs[(c >> 7) * PLDB + (c & 127) * 16]) = rb[i];
        }
        if (tid < 64) {
            // rs: tile tid / 8, pair (tid % 8) / 4, rows 4 ((tid % 8) % 4) .. +3, both blocks of the pair
            const int tl = tid >> 3, pr = (tid & 7) >> 2, r0 = 4 * (tid & 3);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                sws[2 * pr][16 * tl + r0 + e] = f16_to_f32(rs[e] & 0xffffu);
                sws[2 * pr + 1][16 * tl + r0 + e] = f16_to_f32(rs[e] >> 16);
            }
        }
        lds_barrier();
        if (kb + 4 < G) gload(kb + 4);
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
            v4i fa[2], fb[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                fa[t] = *reinterpret_cast<const v4i*>(&As[arow0 + t * 32 * PLDA + bi * 32]);
                const int o = bofs[t] + (bi >> 1) * 1024 + 8 * (bi & 1);
                const int64_t p0 = *reinterpret_cast<const int64_t*>(&Bs[o]);
                const int64_t p1 = *reinterpret_cast<const int64_t*>(&Bs[o + 16 * 16]);
                fb[t] = v4i{(int)p0, (int)(p0 >> 32), (int)p1, (int)(p1 >> 32)};
            }
            const float sw[2] = {sws[bi][swc], sws[bi][swc + 32]};
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const v16i acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[mt], fb[nt], zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        if (RA)
                            y[mt][nt][r] = __builtin_fmaf((float)acc[r], sw[nt], y[mt][nt][r]);
                        else
                            y[mt][nt][r] = add_rn(y[mt][nt][r], mul_rn(mul_rn((float)acc[r], sa[mt][r]), sw[nt]));
                    }
                }
        }
    }
    if (RA) load_sa();
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
                    if (RA) y[mt][nt][r] = mul_rn(y[mt][nt][r], sa[mt][r]);
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

// ---------------------------------------------------------------------------------------------- mid
// From 17 rows (and for narrow projections at any row count, where the tile kernel's 128 x 128 tiles leave most CUs
// idle): one wave (one workgroup) per (MT x 16 activation rows, TG adjacent 16-row weight tiles), walking every block
// pair in order; the m-tiles of one weight tile are grid rows blockIdx.y of the same XCD, so their weight chunks come
// from HBM once.  The activations are the MFMA's A operand, so lane (i, q) = (lane % 16, lane / 16) ends with the sums of
// activation rows 4q..4q+3 of each m-tile against weight row i: its weight scales are one 4-byte word per pair (both
// blocks of row i) and its activation scales four constants per m-tile.  Per pair a lane loads its weight chunk slot
// as it lies (16 bytes), one 16-byte piece of its activation row per m-tile and that word, PD pairs ahead.  The piece
// is bytes 16 s(q)..+15 of the pair with s = (0, 2, 1, 3), and one v_permlane16_swap_b32 per dword pair turns the four
// lanes' pieces into the operand layout of the weight chunk (lane q: bytes 8q..8q+7 of each block).  Loading the
// activation rows in 64-byte runs instead of eight-byte pieces halved this kernel's time.  Each block's int32 sums
// come from one v_mfma_i32_16x16x32_i8 with a zero accumulator and the lane folds RN(RN(float(P) sa) sw) into its
// outputs in block order, in registers.
template <int PD, int MT, int TG, int EPI>
__global__ __launch_bounds__(64) void w8a8_packed_mid_kernel(const int8_t* __restrict__ a,
                                                              const float* __restrict__ a_s, int64_t as_sm,
                                                              const int8_t* __restrict__ qt,
                                                              const uint16_t* __restrict__ dt,
                                                              void* __restrict__ out, int64_t ldo,
                                                              const int32_t* __restrict__ n_rows, int M, int N,
                                                              int K) {
    // every argument fetched at once (else one scalar round trip per first use before the first weight request)
    asm volatile("" ::"s"(a), "s"(a_s), "s"(as_sm), "s"(qt), "s"(dt), "s"(out), "s"(ldo), "s"(n_rows), "s"(M), "s"(N),
                 "s"(K));
    const int lane = threadIdx.x & 63, m0 = blockIdx.y * MT * 16;
    const int nt0 = blockIdx.x * TG;
    // no row-count read before the first requests (it would hold them back by a round trip): workgroups past the
    // live rows still run, and the stores skip rows >= n_rows
    if (m0 >= M) return;
    const int KP = K / 64;
    const int li = lane & 15, q = lane >> 4;
    float sa[MT][4];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int e = 0; e < 4; e++) sa[t][e] = a_s[(int64_t)min(m0 + 16 * t + 4 * q + e, M - 1) * as_sm];
    const v4i* cw = reinterpret_cast<const v4i*>(qt) + (int64_t)nt0 * KP * 64 + lane;
    const uint32_t* cs = reinterpret_cast<const uint32_t*>(dt) + (int64_t)nt0 * KP * 16 + li;
    const int sq = ((q & 1) << 1) | (q >> 1);
    const int8_t* xa[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) xa[t] = a + (int64_t)min(m0 + 16 * t + li, M - 1) * K + 16 * sq;

    struct Pair {
        v4i w[TG];
        v4u x[MT];
        uint32_t s[TG];
    };
    auto load = [&](int j, Pair& p) {
        const int jj = min(j, KP - 1);
#pragma unroll
        for (int g = 0; g < TG; g++) p.w[g] = cw[((int64_t)g * KP + jj) * 64];
#pragma unroll
        for (int t = 0; t < MT; t++) p.x[t] = *reinterpret_cast<const v4u*>(xa[t] + 64 * jj);
#pragma unroll
        for (int g = 0; g < TG; g++) p.s[g] = cs[((int64_t)g * KP + jj) * 16];
    };
    float y[TG][MT][4] = {};
    const v4i zero = {0, 0, 0, 0};
    // the int32 sums of a pair's two blocks (one MFMA each per weight tile and m-tile, zero accumulator)
    auto sums = [&](const Pair& p, v4i (*acc)[MT][2]) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
            // lane q holds 8-byte units (u(2s), u(2s+1)) of the pair; after the swap it holds (u(q), u(4 + q)):
            // block 0's bytes 8q..8q+7 and block 1's
            const auto lo = __builtin_amdgcn_permlane16_swap(p.x[t][0], p.x[t][2], false, false);
            const auto hi = __builtin_amdgcn_permlane16_swap(p.x[t][1], p.x[t][3], false, false);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int64_t xf = (int64_t)(uint32_t)lo[h] | ((int64_t)hi[h] << 32);
#pragma unroll
                for (int g = 0; g < TG; g++) {
                    const int64_t wf = h ? ((int64_t)(uint32_t)p.w[g][2] | ((int64_t)p.w[g][3] << 32))
                                         : ((int64_t)(uint32_t)p.w[g][0] | ((int64_t)p.w[g][1] << 32));
                    acc[g][t][h] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xf, wf, zero, 0, 0, 0);
                }
            }
        }
    };
    // fold the pair's terms into the outputs, block 2j before 2j + 1
    auto fold = [&](v4i (*acc)[MT][2], const Pair& p) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int g = 0; g < TG; g++)
#pragma unroll
                for (int t = 0; t < MT; t++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float x = mul_rn((float)acc[g][t][h][e], sa[t][e]);
                        y[g][t][e] = add_rn(y[g][t][e], h ? mul_f16_rn<1>(x, p.s[g]) : mul_f16_rn<0>(x, p.s[g]));
                    }
    };
    Pair ring[PD];
#pragma unroll
    for (int d = 0; d < PD; d++) load(d, ring[d]);
    // branch-free body, so the compiler's wait counts let the later pairs stay in flight; pairs go two at a time (their
    // MFMAs, then the two folds in order), so the VALU fold of one waits on MFMAs issued before the other's
    static_assert(PD % 2 == 0, "pairs are taken two at a time");
    const int full = KP / PD * PD;
    v4i acc0[TG][MT][2], acc1[TG][MT][2];
    for (int j0 = 0; j0 < full; j0 += PD) {
#pragma unroll
        for (int d = 0; d < PD; d += 2) {
            sums(ring[d], acc0);
            sums(ring[d + 1], acc1);
            fold(acc0, ring[d]);
            fold(acc1, ring[d + 1]);
            load(j0 + d + PD, ring[d]);          // past the end: the last pair again (a cache hit)
            load(j0 + d + 1 + PD, ring[d + 1]);
            // keep each step's work in place: hoisted across steps, the MFMAs would wait for the whole ring
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int d = 0; d < PD; d++)
        if (full + d < KP) {
            sums(ring[d], acc0);
            fold(acc0, ring[d]);
        }
    const int live = min(M, __ldg(n_rows));
#pragma unroll
    for (int g = 0; g < TG; g++) {
        const int n = 16 * (nt0 + g) + li;
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int row = m0 + 16 * t + 4 * q + e;
                if (row < live) {
                    if (EPI == 0) {
                        reinterpret_cast<uint16_t*>(out)[(int64_t)row * ldo + n] = (uint16_t)f32_to_bf16(y[g][t][e]);
                    } else {
                        float* o = reinterpret_cast<float*>(out) + (int64_t)row * ldo + n;
                        *o = add_rn(*o, y[g][t][e]);
                    }
                }
            }
    }
}

static size_t packed_decode_lds(int R, int M) {
    return 2 * (size_t)R * M * 16 * 4 + 2 * (size_t)R * 16 * 4 + 2 * (size_t)M * (R * 32 + 16);
}

// Panel copy of the activations for w8a8_packed_tile_kernel<.., true>: 128-row tiles of K / 128 chunks of 16 KB, tile
// t starting at byte 128 t K, chunk st holding rows 128 t .. + 127 (clamped to M - 1), inputs 128 st .. + 127,
// row-major inside the chunk, so a tile's stage is one 16 KB piece.  One workgroup per (16 rows, 1024 inputs); each
// row's 1 KB is read in one piece.
__global__ __launch_bounds__(256) void q8_act_panel_kernel(const int8_t* __restrict__ a, int8_t* __restrict__ pan,
                                                           int M, int K) {
    const int rb = blockIdx.y;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int piece = threadIdx.x + 256 * j, r = piece >> 6;
        const int k = 1024 * blockIdx.x + 16 * (piece & 63);
        if (k >= K) continue;
        const v4i v = *reinterpret_cast<const v4i*>(a + (int64_t)min(16 * rb + r, M - 1) * K + k);
        const int row = 16 * rb + r;
        *reinterpret_cast<v4i*>(pan + (int64_t)(row >> 7) * 128 * K + (int64_t)(k >> 7) * 16384 + (row & 127) * 128 +
                                (k & 127)) = v;
    }
}

// pan: the panel buffer for the tile kernels (kernels 0 and 3), or null for row-major activations
template <int EPI>
static void launch_packed(int kernel, const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                          const uint16_t* dt, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K,
                          hipStream_t st, int8_t* pan) {
    if (kernel == 1) {
        dim3 grid(N / 16);
#define PDEC(NW, R, MX, D)                                                                                         \
    hipLaunchKernelGGL((w8a8_packed_decode_kernel<NW, (MX * 16 + 63) / 64, R, MX, D, EPI>), grid,                   \
                       dim3((NW + (MX * 16 + 63) / 64) * 64), packed_decode_lds(R, M),                              \
                       st, a, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K)
#ifndef Q8V_SMALL
#define Q8V_SMALL 8, 32, 4, 2
#endif
#ifndef Q8V_BIG
#define Q8V_BIG 8, 16, 16, 3
#endif
#define PDEC_(...) PDEC(__VA_ARGS__)
        if (M <= 4) PDEC_(Q8V_SMALL);
        else if (M <= 16) PDEC_(Q8V_BIG);
        else kernel = 2;
#undef PDEC_
#undef PDEC
    }
    if (kernel == 2) {
        // from 33 rows: each wave one m-tile and two weight tiles (one activation request serves both; the same wave
        // count and fold work as two m-tiles of one tile, with fewer activation line requests: M = 64 at 5120^2
        // 21.0 -> 19.0 us, at 5120 x 17408 59.7 -> 59.1 us), else two m-tiles (shared weight and scale loads; one
        // m-tile per wave with twice the waves ran 60-65 us against 58 us at 64 rows x 5120 x 17408)
#ifndef Q8M_TG
#define Q8M_TG 2
#endif
        if (M > 32 && Q8M_TG == 2 && N % 32 == 0)
            hipLaunchKernelGGL((w8a8_packed_mid_kernel<6, 1, 2, EPI>), dim3(N / 32, (M + 15) / 16), dim3(64), 0, st,
                               a, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K);
        else if (M > 32)
            hipLaunchKernelGGL((w8a8_packed_mid_kernel<6, 2, 1, EPI>), dim3(N / 16, (M + 31) / 32), dim3(64), 0, st,
                               a, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K);
        else
            hipLaunchKernelGGL((w8a8_packed_mid_kernel<8, 1, 1, EPI>), dim3(N / 16, (M + 15) / 16), dim3(64), 0, st,
                               a, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K);
    } else if (kernel == 0 || kernel == 3) {
        const int tiles_m = (M + PBM - 1) / PBM, tiles_n = (N + PBN - 1) / PBN;
        if (pan) {                                   // the panel copy first, then the tile kernel reads it
            hipLaunchKernelGGL(q8_act_panel_kernel, dim3((unsigned)((K + 1023) / 1024), (unsigned)((M + 127) / 128 * 8)),
                               dim3(256), 0, st, a, pan, M, K);
            if (kernel == 0)
                hipLaunchKernelGGL((w8a8_packed_tile_kernel<EPI, false, true>), dim3(tiles_m * tiles_n), dim3(256), 0,
                                   st, pan, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K, tiles_m, tiles_n);
            else
                hipLaunchKernelGGL((w8a8_packed_tile_kernel<EPI, true, true>), dim3(tiles_m * tiles_n), dim3(256), 0,
                                   st, pan, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K, tiles_m, tiles_n);
        } else if (kernel == 0)
            hipLaunchKernelGGL((w8a8_packed_tile_kernel<EPI, false>), dim3(tiles_m * tiles_n), dim3(256), 0, st, a,
                               a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL((w8a8_packed_tile_kernel<EPI, true>), dim3(tiles_m * tiles_n), dim3(256), 0, st, a,
                               a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K, tiles_m, tiles_n);
    }
}

}  // namespace prism

using namespace prism;

extern "C" int prism_q8_0_pack(const int8_t* qs, const uint16_t* d, int8_t* qt, uint16_t* dt, int64_t N, int64_t K,
                               void* stream) {
    if (!qs || !d || !qt || !dt) return PRISM_ERR_ARG;
    // K % 128: the packed GEMM's rule (its prefill tile stages 128 inputs), so a packed operand is always usable
    if (N <= 0 || K <= 0 || N % 16 || K % 128 || N > (1 << 30) || K > (1 << 30)) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(qs, 16) || !PRISM_ALIGNED(qt, 16) || !PRISM_ALIGNED(dt, 16)) return PRISM_ERR_ALIGN;
    const int64_t total = N / 16 * (K / 64) * 64;
    hipLaunchKernelGGL(q8_0_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, qs,
                       d, qt, dt, (int)N, (int)K);
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_i8_pack(const int8_t* w, int8_t* qt, int64_t N, int64_t K, void* stream) {
    if (!w || !qt) return PRISM_ERR_ARG;
    if (N <= 0 || K <= 0 || N % 16 || K % 64 || N > (1 << 30) || K > (1 << 30)) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(w, 16) || !PRISM_ALIGNED(qt, 16)) return PRISM_ERR_ALIGN;
    const int64_t total = N / 16 * (K / 64) * 64;
    hipLaunchKernelGGL(q8_0_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, w,
                       nullptr, qt, nullptr, (int)N, (int)K);
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

// The workspace's first kQ8PanelOffset bytes hold the balanced decode kernel's handoff words (zero between launches,
// at most kQ8StreamMaxWG x 2 KB for any shape); the prefill's panel copy goes after them.
constexpr int64_t kQ8PanelOffset = 512 * 1024;
static_assert(kQ8StreamMaxWG * 16 * 16 * 8 <= kQ8PanelOffset, "the handoff words end before the panel copy");

static int packed_gemm(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt, const uint16_t* dt,
                       void* out, int64_t ldo, const int32_t* n_rows, int64_t M, int64_t N, int64_t K, int epi,
                       int kernel, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!a || !a_s || !qt || !dt || !out || !n_rows) return PRISM_ERR_ARG;
    if (epi != 0 && epi != 1) return PRISM_ERR_ARG;
    if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 128 || ldo < N || M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
        return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(a, 16) || !PRISM_ALIGNED(qt, 16) || !PRISM_ALIGNED(dt, 16)) return PRISM_ERR_ALIGN;
    if (kernel < -1 || kernel > 4) return PRISM_ERR_ARG;
    const bool can_stream = M >= 1 && M <= 16 && (N / 16) * (K / 64) < ((int64_t)1 << 31) &&
                            M * K < ((int64_t)1 << 31) && workspace &&
                            workspace_bytes >= q8_stream_workspace_bytes(N, K);
    // by default: the balanced kernel up to 16 rows (given its workspace), the row-round decode kernel up to 64 rows
    // (and up to 16 without a workspace), the tile kernel beyond
    if (kernel == -1) kernel = M >= 1 && M <= 16 && can_stream ? 4 : M <= 64 ? 1 : 0;
    if (kernel == 1 && M > 64) return PRISM_ERR_ARG;
    if (kernel == 4 && !can_stream) return M > 16 ? PRISM_ERR_SHAPE : PRISM_ERR_ARG;
    if (kernel == 2 && M > 65535 * 16) return PRISM_ERR_SHAPE;         // grid rows: one per 16 activation rows
    if (M == 0) return PRISM_OK;
    hipStream_t st = (hipStream_t)stream;
    if (kernel == 4) {
        const int rc = q8_stream_launch(a, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K, epi, workspace,
                                        workspace_bytes, st);
        if (rc != PRISM_OK) return rc;
        PRISM_LAUNCH_CHECK();
        return PRISM_OK;
    }
    // the tile kernels on a panel copy of the activations where the workspace holds it past the handoff words and the
    // shape repays the copy (2 M K bytes of traffic): from 1024 rows on projections at least 16384 wide
    int8_t* pan = nullptr;
    if ((kernel == 0 || kernel == 3) && M >= 1024 && N >= 16384 && M <= 8191 * 128 && workspace &&
        PRISM_ALIGNED(workspace, 256) && workspace_bytes >= kQ8PanelOffset + (M + 127) / 128 * 128 * K)
        pan = static_cast<int8_t*>(workspace) + kQ8PanelOffset;
    if (epi == 0)
        launch_packed<0>(kernel, a, a_s, as_sm, qt, dt, out, ldo, n_rows, (int)M, (int)N, (int)K, st, pan);
    else
        launch_packed<1>(kernel, a, a_s, as_sm, qt, dt, out, ldo, n_rows, (int)M, (int)N, (int)K, st, pan);
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

extern "C" int prism_w8a8_q8_0_packed_gemm(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                           const uint16_t* dt, void* out, int64_t ldo, const int32_t* n_rows,
                                           int64_t M, int64_t N, int64_t K, int epi, int kernel, void* workspace,
                                           int64_t workspace_bytes, void* stream) {
    return packed_gemm(a, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K, epi, kernel, workspace, workspace_bytes,
                       stream);
}

extern "C" int64_t prism_w8a8_q8_0_packed_workspace_bytes(int64_t N, int64_t K) {
    if (N <= 0 || K <= 0 || N % 16) return 0;
    return q8_stream_workspace_bytes(N, K);
}

// ---------------------------------------------------------------------------------------------- no-allocation form
// For callers that cannot allocate (code under graph capture, serving loops, harnesses that forbid hipMalloc): the
// balanced decode kernel's workspace is this file-scope device array instead of a caller's buffer.  Each GPU holds
// its own copy, zero-initialised when the code object loads; the first call on a device that is not being captured
// clears it once more with a fill kernel and waits for that clear before the address is kept.  A first call under
// graph capture records no clear into the caller's graph: it relies on the load-time zero, and the address is kept
// only once a clear has run.  Every launch leaves the array zeroed (each handoff word is reset by the workgroup that
// consumes it, and words of a launch that did not complete carry another launch's tag, never taken).
// In host code the array's name is not a device address; its per-device address comes from hipGetSymbolAddress.
constexpr int64_t kScratchBytes = 512 * 1024;
static __device__ __align__(256) unsigned long long scratch[kScratchBytes / 8];
static_assert(kQ8StreamMaxWG * 16 * 16 * 8 <= kScratchBytes, "the scratch array holds the largest workspace");

__global__ void scratch_clear_kernel(unsigned long long* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

constexpr int kMaxDevices = 64;
static void* g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

// The device's scratch address, or nullptr.  At the first call on the device outside capture: looked up, cleared on
// `st` and waited for, then kept.  Under capture: looked up and returned, not kept, nothing recorded.
static void* device_scratch(hipStream_t st) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev]) return g_scratch[dev];
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return nullptr;
    if (cs != hipStreamCaptureStatusNone) return ptr;
    hipLaunchKernelGGL(scratch_clear_kernel, dim3(64), dim3(256), 0, st, (unsigned long long*)ptr, kScratchBytes / 8);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) return nullptr;
    g_scratch[dev] = ptr;
    return ptr;
}

extern "C" int prism_w8a8_q8_0_packed_gemm_noalloc(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                                   const uint16_t* dt, void* out, int64_t ldo, const int32_t* n_rows,
                                                   int64_t M, int64_t N, int64_t K, int epi, int kernel,
                                                   void* stream) {
    if (N > 0 && K > 0 && N % 16 == 0 && q8_stream_workspace_bytes(N, K) > kScratchBytes) return PRISM_ERR_SHAPE;
    void* ws = device_scratch((hipStream_t)stream);
    if (!ws) return PRISM_ERR_LAUNCH;
    return packed_gemm(a, a_s, as_sm, qt, dt, out, ldo, n_rows, M, N, K, epi, kernel, ws, kScratchBytes, stream);
}
