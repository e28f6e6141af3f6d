// W4A8 prefill on Q4_K weights (gfx950): the tile kernel for M beyond the decode sizes.
//
// Arithmetic, per output (m, n) and super-block b in increasing b, as every W4A8 kernel (kernels/w4a8.py:14-22,
// 177-199; w4a8.hip's header): acc = sum_g sc P_g (two-plane MFMA weight operands, exact), mins = sum_g mn S_g (exact),
// t = RN(d float(acc)), t = fma(-dmin, float(mins), t), y = fma(a[b, m], t, y); bf16(y) (epi 0) or out = RN(out + y)
// (epi 1).  Bits equal the decode kernels' and the oracle's.
//
// Tile: 128 (n) x 128 (m) per 512-thread workgroup, one workgroup per CU (two waves per SIMD), one super-block per
// stage, two stages in LDS: the weight chunks and the activation rows arrive by LDS-DMA, the stage's meta through
// registers, unpacked into LDS ready for the MFMAs (split scale words, the mins and the activation rows' split sums as
// fp16, d and dmin and the activation scales as fp32).  Wave wv owns one 16-row weight tile (n rows 16 wv ..) against
// all 128 activation rows (eight 16-row blocks j), so the VALU that expands its nibbles into the two scale planes
// serves eight output blocks.  Per block: eight int8 MFMAs (lo and hi planes over the four sub-block pairs), one fp16
// MFMA for the mins, then five VALU instructions per output:
//   * the mins come out of the fp16 MFMA as float(mins) directly: A = [mn_0..7, 64 mn_0..7], B = [S_lo 0..7,
//     S_hi 0..7] (S = S_lo + 64 S_hi), every product and partial sum an integer below 2^24, so the fp32 accumulation
//     is exact in any order (the int8 form needs two MFMAs, a combine and a convert per output);
//   * blocks 0..3 run pair by pair (the planes of a pair, then its MFMAs for four blocks), blocks 4..7 one by one with
//     the epilogue of block j - 4 between the MFMAs of block j, so the VALU issues between MFMAs.
// Measured on MI355X at C3 (2048 x 5120 x 13824): 445 us for the previous 128 x 64 four-wave kernel, 355-362 us here.
// What bounds it: with two scale planes the int8 MFMA work is twice the GEMM's (1088 MFMA cycles per wave and
// super-block), and the VALU (about 290 instructions per wave and super-block, 160 of them the epilogue) overlaps the
// MFMAs only in part: a wave issues about two VALU instructions under each 16-cycle MFMA for free, each further one
// delays the next MFMA.
#include "common.h"
#include "w4a8_common.h"
#include "w4a8_prefill.h"

namespace prism {

typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Four signed bytes (-128..127) as four exact halves.
__device__ __forceinline__ v4h s8x4_f16(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const v2h k = {(_Float16)1152.0f, (_Float16)1152.0f};
    const v2h lo = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - k;
    const v2h hi = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - k;
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
}

constexpr int T8N = 128, T8M = 128;

template <int EPI>
__global__ __launch_bounds__(512, 1) void w4a8_q4k_tile_kernel(const int8_t* __restrict__ xq,
                                                                const float* __restrict__ a, int64_t a_sb,
                                                                const int8_t* __restrict__ xs,
                                                                const uint8_t* __restrict__ qv,
                                                                const uint8_t* __restrict__ meta,
                                                                void* __restrict__ out, int64_t ldo,
                                                                const int32_t* __restrict__ n_rows, int M, int N,
                                                                int K, int tiles_m, int tiles_n) {
    // stage buffers as separate objects (see the loop below): 8 weight tiles x 2 KB as packed; the activation rows,
    // chunk c of row r at 16-byte slot c ^ (r & 15), so the 16 rows a 16-lane read spans fall in distinct banks
    __shared__ __attribute__((aligned(16))) uint8_t Bs0[8 * 2048];
    __shared__ __attribute__((aligned(16))) uint8_t Bs1[8 * 2048];
    __shared__ __attribute__((aligned(16))) int8_t As0[T8M * 256];
    __shared__ __attribute__((aligned(16))) int8_t As1[T8M * 256];
    // split scales [sub-block][weight row] (rows padded by 4 words: the two sub-blocks a wave reads at once sit 4 banks
    // apart)
    __shared__ uint32_t scl[2][8][T8N + 4];
    __shared__ __attribute__((aligned(16))) _Float16 mnh[2][T8N][8];  // mins as fp16
    __shared__ __attribute__((aligned(16))) float dl[2][T8N], dml[2][T8N];
    // split sums as fp16, per row S & 63 x 8 then S >> 6 x 8 in four 8-byte quads; rows 8..15 of every 16 keep their
    // halves swapped (quad qq at qq ^ 2), so a wave's read of 16 rows meets no bank twice
    __shared__ __attribute__((aligned(16))) _Float16 shh[2][T8M][16];
    __shared__ float al[2][T8M];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lm = lane & 15, q = lane >> 4;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * T8M, n0 = pn * T8N;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int NB = K / 256, ntiles = N / 16;

    // DMA: per stage 1024 weight chunks (2 per thread) and 2048 activation chunks (4 per thread) of 16 bytes
    uint32_t woff[2], xoff[4];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int c = tid + 512 * i;
        woff[i] = (uint32_t)((min(n0 / 16 + (c >> 7), ntiles - 1) * NB * 128 + (c & 127)) * 16);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = tid + 512 * i, r = c >> 4;
        xoff[i] = (uint32_t)(min(m0 + r, M - 1) * K + (((c & 15) ^ (r & 15)) * 16));
    }
    auto dma = [&](int b, uint8_t* Bd, int8_t* Ad) {
#pragma unroll
        for (int i = 0; i < 2; i++) dma16(qv + (woff[i] + (uint32_t)b * 2048u), &Bd[(512 * i + 64 * wv) * 16]);
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(xq + (xoff[i] + (uint32_t)b * 256u), &Ad[(512 * i + 64 * wv) * 16]);
    };
    // meta: waves 0-3 unpack the weight rows (waves 0-1 sub-blocks 0..3 and d, waves 2-3 sub-blocks 4..7 and dmin),
    // waves 4-7 convert the activation rows' split sums (waves 4-5 the S & 63 half and the scale, 6-7 the S >> 6
    // half): one row per lane, the half wave-uniform, so no lane-dependent branches
    const int hrow = tid & 127, hh = (wv >> 1) & 1;
    const bool wside = wv < 4;
    // one 16-byte load per thread and stage from either source (no branch, so the loaded values need no merge):
    // the weight row's meta (16 rows x 16 B per tile and super-block) or the activation row's split sums
    const uint8_t* gsrc = wside ? meta + ((int64_t)min(n0 / 16 + (hrow >> 4), ntiles - 1) * NB * 16 + (hrow & 15)) * 16
                                : reinterpret_cast<const uint8_t*>(xs) + (int64_t)min(m0 + hrow, M - 1) * 16;
    const int64_t gstride = wside ? 256 : (int64_t)M * 16;
    const int srow = min(m0 + hrow, M - 1);
    v4u rm;
    float ra;
    auto gmeta = [&](int b) {
        rm = *reinterpret_cast<const v4u*>(gsrc + (int64_t)b * gstride);
        ra = a[(int64_t)b * a_sb + srow];
    };
    auto smeta = [&](int buf) {
        if (wside) {
            // ggml get_scale_min_k4 for sub-blocks 4 hh + t: bytes 4..7 s0, 8..11 s4, 12..15 s8
            const float dv = f16_to_f32(hh ? (rm[0] >> 16) : (rm[0] & 0xffffu));
            uint32_t mpk[2];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t s0 = (rm[1] >> (8 * t)) & 0xff, s4 = (rm[2] >> (8 * t)) & 0xff,
                               s8 = (rm[3] >> (8 * t)) & 0xff;
                const int sc = hh ? (int)((s8 & 0xf) | ((s0 >> 6) << 4)) : (int)(s0 & 63);
                const int mn = hh ? (int)((s8 >> 4) | ((s4 >> 6) << 4)) : (int)(s4 & 63);
                scl[buf][4 * hh + t][hrow] = split_scale(sc);
                // mn < 64: the fp16 bits of 1024 + mn, minus 1024, exactly
                const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(0x6400 | mn)) - (_Float16)1024.0f;
                const uint32_t hb = __builtin_bit_cast(uint16_t, h);
                mpk[t >> 1] = (t & 1) ? (mpk[t >> 1] | (hb << 16)) : hb;
            }
            *reinterpret_cast<v2u*>(&mnh[buf][hrow][4 * hh]) = v2u{mpk[0], mpk[1]};
            if (hh) dml[buf][hrow] = dv;
            else dl[buf][hrow] = dv;
        } else {
            const v4h lo = s8x4_f16(rm[2 * hh]), hi = s8x4_f16(rm[2 * hh + 1]);
            const int hs = hh ^ ((hrow >> 3) & 1);
            *reinterpret_cast<v4h*>(&shh[buf][hrow][8 * hs]) = lo;
            *reinterpret_cast<v4h*>(&shh[buf][hrow][8 * hs + 4]) = hi;
            if (!hh) al[buf][hrow] = ra;
        }
    };

    float y[8][4];
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) y[j][e] = 0.f;
    // lanes q >= 2 carry the k = 8..15 half of the mins operand: 64 mn against S >> 6
    const _Float16 mm = q >= 2 ? (_Float16)64.0f : (_Float16)1.0f;
    const v4h mmul4 = {mm, mm, mm, mm};
    const int wrow = 16 * wv + lm;

    gmeta(0);
    dma(0, Bs0, As0);
    vm_wait<0>();
    smeta(0);
    lds_barrier();
    // the loop runs two super-blocks per trip so that each stage's buffers are distinct LDS objects: the
    // compiler then sees that the next stage's DMA does not write what this stage reads, and issues the reads
    // without first waiting for the DMA (with one array indexed by b & 1 it waited for every DMA at once)
    auto step = [&](const int b, const int cb, const uint8_t* __restrict__ Bc, const int8_t* __restrict__ Ac,
                    uint8_t* __restrict__ Bn, int8_t* __restrict__ An) __attribute__((always_inline)) {
        {
            // the next stage, unconditionally (past the last super-block: the last one again, never used), so the
            // meta loads need no merge with the previous values and no wait for their data here
            const int bn = min(b + 1, NB - 1);
            gmeta(bn);
            dma(bn, Bn, An);
        }
        v4u wq[2];
        uint32_t sp[4];
#pragma unroll
        for (int h = 0; h < 2; h++) wq[h] = *reinterpret_cast<const v4u*>(&Bc[wv * 2048 + h * 1024 + lane * 16]);
#pragma unroll
        for (int p = 0; p < 4; p++) sp[p] = scl[cb][2 * p + (q >> 1)][wrow];
        const v4h ma = *reinterpret_cast<const v4h*>(&mnh[cb][wrow][4 * (q & 1)]) * mmul4;
        const v4f dd = *reinterpret_cast<const v4f*>(&dl[cb][16 * wv + 4 * q]);
        const v4f ndm = -*reinterpret_cast<const v4f*>(&dml[cb][16 * wv + 4 * q]);
        v4i wl[4], wh[4];
        auto epilogue = [&](int j, v4i lo, v4i hi, v4f mf, float am) {
#pragma unroll
            for (int e = 0; e < 4; e++)
                y[j][e] = fmaf(am, fmaf(ndm[e], mf[e], mul_rn(dd[e], (float)(lo[e] + 8 * hi[e]))), y[j][e]);
            asm volatile("" : "+v"(y[j][0]), "+v"(y[j][1]), "+v"(y[j][2]), "+v"(y[j][3]));
        };
        // blocks j = 0..7, 16 activation rows each
        v4i af[8][4], los[8], his[8];
        v4h sbv[8];
        v4f mfs[8];
        float amv[8];
        auto acts = [&](int j) {
#pragma unroll
            for (int p = 0; p < 4; p++)
                af[j][p] = *reinterpret_cast<const v4i*>(&Ac[(16 * j + lm) * 256 + (((4 * p + q) ^ lm) * 16)]);
            sbv[j] = *reinterpret_cast<const v4h*>(&shh[cb][16 * j + lm][4 * (q ^ ((lm >> 2) & 2))]);
            amv[j] = al[cb][16 * j + lm];
        };
        // first half: blocks 0..3 pair by pair (the scale planes of pair p, then its MFMAs for the four blocks: the
        // planes' VALU issues between MFMAs instead of holding up block 0); second half: blocks 4..7 one by one, the
        // epilogue of block j - 4 between the MFMAs of block j
#pragma unroll
        for (int j = 0; j < 4; j++) acts(j);
        {
            v4i lo4[4], hi4[4];
#pragma unroll
            for (int j = 0; j < 4; j++) lo4[j] = hi4[j] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                two_plane(wq[p >> 1][2 * (p & 1)], wq[p >> 1][2 * (p & 1) + 1], sp[p], wl[p], wh[p]);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    lo4[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl[p], af[j][p], lo4[j], 0, 0, 0);
                    hi4[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh[p], af[j][p], hi4[j], 0, 0, 0);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                los[j] = lo4[j], his[j] = hi4[j];
                mfs[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(ma, sbv[j], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
            acts(4);
            acts(5);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 4; j < 8; j++) {
            v4i lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl[p], af[j][p], lo, 0, 0, 0);
                hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh[p], af[j][p], hi, 0, 0, 0);
            }
            los[j] = lo, his[j] = hi;
            mfs[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(ma, sbv[j], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            epilogue(j - 4, los[j - 4], his[j - 4], mfs[j - 4], amv[j - 4]);
            if (j + 2 < 8) acts(j + 2);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 4; j < 8; j++) epilogue(j, los[j], his[j], mfs[j], amv[j]);
        vm_wait<0>();
        smeta(cb ^ 1);
        lds_barrier();
        };
    for (int b = 0; b < NB; b += 2) {
        step(b, 0, Bs0, As0, Bs1, As1);
        if (b + 1 < NB) step(b + 1, 1, Bs1, As1, Bs0, As0);
    }
    // D element (j, e): n = n0 + 16 wv + 4 q + e, m = m0 + 16 j + lm
    const int nb = n0 + 16 * wv + 4 * q;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int m = m0 + 16 * j + lm;
        if (m < live && nb < N) {
            if (EPI == 0) {
                const uint32_t lo = f32_to_bf16(y[j][0]) | (f32_to_bf16(y[j][1]) << 16);
                const uint32_t hi = f32_to_bf16(y[j][2]) | (f32_to_bf16(y[j][3]) << 16);
                uint16_t* o = reinterpret_cast<uint16_t*>(out) + (int64_t)m * ldo + nb;
                if ((((uintptr_t)o) & 7) == 0) {
                    *reinterpret_cast<v2u*>(o) = v2u{lo, hi};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) o[e] = (uint16_t)f32_to_bf16(y[j][e]);
                }
            } else {
                float* o = reinterpret_cast<float*>(out) + (int64_t)m * ldo + nb;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = add_rn(o[e], y[j][e]);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------- Q6_K prefill
// Q6_K (prism_q6k_pack: values q - 32 as int8, 16 int8 scales per row and super-block, one per 16 inputs) on the same
// 128 x 128 tile, eight waves, two LDS stages and block schedule as the Q4_K kernel above.  Per super-block
// (kernels/w4a8.py:19-20, 193-197): acc = sum_h sc_h P_h over the sixteen 16-input sub-blocks, exact in int32;
// y = fma(a[b, m], RN(d float(acc)), y) in super-block order.  The scales go into the MFMA weight operand as two
// int8 planes: a lane's 16 inputs of an operand are one sub-block, w = sc v (|w| <= 4096) is split as
// w = (w & 63) + 64 (w >> 6), both parts int8, and two MFMA chains give acc = lo + 64 hi over the whole super-block
// (the form of the reference's own CUDA kernel, csrc/w4a8_wgmma.cu:9-10): nothing per output until the super-block
// ends (the 32 x 32 x 16 kernel it replaces does one v_mad per output and 16-input sub-block).
// A lane's operand for inputs 64 p + 16 q .. + 15 is two 8-byte pieces of the packed chunk p: lane slots
// 32 (q & 1) + lm and 32 (q & 1) + 16 + lm, bytes 8 (q >> 1) .. + 7 of each.

// Four signed weights (bytes of v) times the scale pair sc16 (sc in both 16-bit halves) as the two plane dwords
// (w & 63, w >> 6) in byte order.
__device__ __forceinline__ void q6_planes(uint32_t v, uint32_t sc16, uint32_t& lo, uint32_t& hi) {
    typedef short s2 __attribute__((ext_vector_type(2)));
    const s2 ev = __builtin_bit_cast(s2, v << 8) >> (s2){8, 8};       // bytes 0, 2 sign-extended
    const s2 od = __builtin_bit_cast(s2, v) >> (s2){8, 8};            // bytes 1, 3
    const s2 sc = __builtin_bit_cast(s2, sc16);
    const s2 we = ev * sc, wo = od * sc;                              // |w| <= 4096: exact in 16 bits
    const uint32_t le = __builtin_bit_cast(uint32_t, we) & 0x003f003fu, lo_ = __builtin_bit_cast(uint32_t, wo) & 0x003f003fu;
    const uint32_t he = __builtin_bit_cast(uint32_t, (s2)(we >> (s2){6, 6}));
    const uint32_t ho = __builtin_bit_cast(uint32_t, (s2)(wo >> (s2){6, 6}));
    lo = __builtin_amdgcn_perm(lo_, le, 0x06020400u);                  // bytes e0 o0 e1 o1
    hi = __builtin_amdgcn_perm(ho, he, 0x06020400u);
}

template <int EPI>
__global__ __launch_bounds__(512, 1) void w4a8_q6k_tile_kernel(const int8_t* __restrict__ xq,
                                                                const float* __restrict__ a, int64_t a_sb,
                                                                const uint8_t* __restrict__ qv,
                                                                const uint8_t* __restrict__ meta,
                                                                void* __restrict__ out, int64_t ldo,
                                                                const int32_t* __restrict__ n_rows, int M, int N,
                                                                int K, int tiles_m, int tiles_n) {
    // stage buffers as separate objects: 8 weight tiles x 4 KB as packed; the activation rows, chunk c of row r at
    // 16-byte slot c ^ (r & 15)
    __shared__ __attribute__((aligned(16))) uint8_t Bs0[8 * 4096];
    __shared__ __attribute__((aligned(16))) uint8_t Bs1[8 * 4096];
    __shared__ __attribute__((aligned(16))) int8_t As0[T8M * 256];
    __shared__ __attribute__((aligned(16))) int8_t As1[T8M * 256];
    __shared__ __attribute__((aligned(16))) v4u scl[2][T8N];           // per weight row: its 16 int8 scales
    __shared__ __attribute__((aligned(16))) float dl[2][T8N];
    __shared__ float al[2][T8M];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lm = lane & 15, q = lane >> 4;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * T8M, n0 = pn * T8N;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int NB = K / 256, ntiles = N / 16;

    // DMA: per stage 2048 weight chunks and 2048 activation chunks of 16 bytes, four of each per thread
    uint32_t woff[4], xoff[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = tid + 512 * i;
        woff[i] = (uint32_t)((min(n0 / 16 + (c >> 8), ntiles - 1) * NB * 256 + (c & 255)) * 16);
        const int r = c >> 4;
        xoff[i] = (uint32_t)(min(m0 + r, M - 1) * K + (((c & 15) ^ (r & 15)) * 16));
    }
    auto dma = [&](int b, uint8_t* Bd, int8_t* Ad) {
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(qv + (woff[i] + (uint32_t)b * 4096u), &Bd[(512 * i + 64 * wv) * 16]);
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(xq + (xoff[i] + (uint32_t)b * 256u), &Ad[(512 * i + 64 * wv) * 16]);
    };
    // meta: thread t loads weight row t % 128's 16 scale bytes and d, and activation row t % 128's scale, every
    // thread unconditionally (no branch, so the loaded values need no merge); waves 0-1 store the scales, 2-3 d,
    // 4-5 the activation scales
    const int hrow = tid & 127;
    const uint8_t* msrc = meta + (int64_t)min(n0 / 16 + (hrow >> 4), ntiles - 1) * NB * Q6_META;
    const int srow = min(m0 + hrow, M - 1);
    v4u rm;
    uint32_t rd;
    float ra;
    auto gmeta = [&](int b) {
        const uint8_t* mp = msrc + (int64_t)b * Q6_META;
        rm = reinterpret_cast<const v4u*>(mp)[hrow & 15];
        rd = reinterpret_cast<const uint16_t*>(mp + 256)[hrow & 15];
        ra = a[(int64_t)b * a_sb + srow];
    };
    auto smeta = [&](int buf) {
        if (wv < 2) scl[buf][hrow] = rm;
        else if (wv < 4) dl[buf][hrow] = f16_to_f32(rd);
        else if (wv < 6) al[buf][hrow] = ra;
    };

    float y[8][4];
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) y[j][e] = 0.f;
    const int wrow = 16 * wv + lm;
    // this lane's two lane slots of a chunk and the byte half (see the comment above)
    const int bs0 = (wv * 4 * 64 + 32 * (q & 1) + lm) * 16 + 8 * (q >> 1);

    gmeta(0);
    dma(0, Bs0, As0);
    vm_wait<0>();
    smeta(0);
    lds_barrier();
    // two super-blocks per trip, each stage's buffers distinct LDS objects (see the Q4_K kernel)
    auto step = [&](const int b, const int cb, const uint8_t* __restrict__ Bc, const int8_t* __restrict__ Ac,
                    uint8_t* __restrict__ Bn, int8_t* __restrict__ An) __attribute__((always_inline)) {
        {
            const int bn = min(b + 1, NB - 1);
            gmeta(bn);
            dma(bn, Bn, An);
        }
        // this lane's sub-block scales (sub-block 4 p + q: byte q of scale dword p) as 16-bit pairs
        const v4u sv = scl[cb][wrow];
        uint32_t sc16[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t sc = (uint32_t)__builtin_amdgcn_sbfe((int)sv[p], 8 * q, 8) & 0xffffu;
            sc16[p] = sc | (sc << 16);
        }
        const v4f dd = *reinterpret_cast<const v4f*>(&dl[cb][16 * wv + 4 * q]);
        v4i wl[4], wh[4];
        auto planes = [&](int p) {
            const v2u x0 = *reinterpret_cast<const v2u*>(&Bc[bs0 + p * 1024]);
            const v2u x1 = *reinterpret_cast<const v2u*>(&Bc[bs0 + p * 1024 + 256]);
            uint32_t l[4], h[4];
            q6_planes(x0[0], sc16[p], l[0], h[0]);
            q6_planes(x0[1], sc16[p], l[1], h[1]);
            q6_planes(x1[0], sc16[p], l[2], h[2]);
            q6_planes(x1[1], sc16[p], l[3], h[3]);
            wl[p] = v4i{(int)l[0], (int)l[1], (int)l[2], (int)l[3]};
            wh[p] = v4i{(int)h[0], (int)h[1], (int)h[2], (int)h[3]};
        };
        auto epilogue = [&](int j, v4i lo, v4i hi, float am) {
#pragma unroll
            for (int e = 0; e < 4; e++) y[j][e] = fmaf(am, mul_rn(dd[e], (float)(lo[e] + 64 * hi[e])), y[j][e]);
            asm volatile("" : "+v"(y[j][0]), "+v"(y[j][1]), "+v"(y[j][2]), "+v"(y[j][3]));
        };
        v4i af[8][4], los[8], his[8];
        float amv[8];
        auto acts = [&](int j) {
#pragma unroll
            for (int p = 0; p < 4; p++)
                af[j][p] = *reinterpret_cast<const v4i*>(&Ac[(16 * j + lm) * 256 + (((4 * p + q) ^ lm) * 16)]);
            amv[j] = al[cb][16 * j + lm];
        };
        // blocks 0..3 pair by pair, then blocks 4..7 one by one with the epilogue of block j - 4 between the MFMAs
        // of block j (the Q4_K kernel's schedule)
#pragma unroll
        for (int j = 0; j < 4; j++) acts(j);
        {
            v4i lo4[4], hi4[4];
#pragma unroll
            for (int j = 0; j < 4; j++) lo4[j] = hi4[j] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                planes(p);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    lo4[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl[p], af[j][p], lo4[j], 0, 0, 0);
                    hi4[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh[p], af[j][p], hi4[j], 0, 0, 0);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) los[j] = lo4[j], his[j] = hi4[j];
            acts(4);
            acts(5);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 4; j < 8; j++) {
            v4i lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl[p], af[j][p], lo, 0, 0, 0);
                hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh[p], af[j][p], hi, 0, 0, 0);
            }
            los[j] = lo, his[j] = hi;
            epilogue(j - 4, los[j - 4], his[j - 4], amv[j - 4]);
            if (j + 2 < 8) acts(j + 2);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 4; j < 8; j++) epilogue(j, los[j], his[j], amv[j]);
        vm_wait<0>();
        smeta(cb ^ 1);
        lds_barrier();
    };
    for (int b = 0; b < NB; b += 2) {
        step(b, 0, Bs0, As0, Bs1, As1);
        if (b + 1 < NB) step(b + 1, 1, Bs1, As1, Bs0, As0);
    }
    // D element (j, e): n = n0 + 16 wv + 4 q + e, m = m0 + 16 j + lm
    const int nb = n0 + 16 * wv + 4 * q;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int m = m0 + 16 * j + lm;
        if (m < live && nb < N) {
            if (EPI == 0) {
                const uint32_t lo = f32_to_bf16(y[j][0]) | (f32_to_bf16(y[j][1]) << 16);
                const uint32_t hi = f32_to_bf16(y[j][2]) | (f32_to_bf16(y[j][3]) << 16);
                uint16_t* o = reinterpret_cast<uint16_t*>(out) + (int64_t)m * ldo + nb;
                if ((((uintptr_t)o) & 7) == 0) {
                    *reinterpret_cast<v2u*>(o) = v2u{lo, hi};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) o[e] = (uint16_t)f32_to_bf16(y[j][e]);
                }
            } else {
                float* o = reinterpret_cast<float*>(out) + (int64_t)m * ldo + nb;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = add_rn(o[e], y[j][e]);
            }
        }
    }
}

void q6k_tile_launch(const int8_t* xq, const float* a, int64_t a_sb, const uint8_t* qv, const uint8_t* meta,
                     void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int epi, hipStream_t st) {
    const int tm = (M + T8M - 1) / T8M, tn = (N + T8N - 1) / T8N;
    if (epi == 0)
        hipLaunchKernelGGL((w4a8_q6k_tile_kernel<0>), dim3(tm * tn), dim3(512), 0, st, xq, a, a_sb, qv, meta, out, ldo,
                           n_rows, M, N, K, tm, tn);
    else
        hipLaunchKernelGGL((w4a8_q6k_tile_kernel<1>), dim3(tm * tn), dim3(512), 0, st, xq, a, a_sb, qv, meta, out, ldo,
                           n_rows, M, N, K, tm, tn);
}

void q4k_tile_launch(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs, const uint8_t* qv,
                     const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int epi,
                     hipStream_t st) {
    const int tm = (M + T8M - 1) / T8M, tn = (N + T8N - 1) / T8N;
    if (epi == 0)
        hipLaunchKernelGGL((w4a8_q4k_tile_kernel<0>), dim3(tm * tn), dim3(512), 0, st, xq, a, a_sb, xs, qv, meta, out,
                           ldo, n_rows, M, N, K, tm, tn);
    else
        hipLaunchKernelGGL((w4a8_q4k_tile_kernel<1>), dim3(tm * tn), dim3(512), 0, st, xq, a, a_sb, xs, qv, meta, out,
                           ldo, n_rows, M, N, K, tm, tn);
}

}  // namespace prism
