// Per-channel W8A8 GEMM (gk = K: one activation scale per token, one weight scale per output channel) for gfx950.
// The engine's production projections (kernels/w8a8.py:183-231 with gk == K; the CUDA w8a8_kernel epilogue,
// csrc/w8a8_gemm.cu:298-402): P = sum_k a w in int32 (exact), y = RN(RN(float(P) sa) sw); epilogue 0 stores bf16(y),
// epilogue 1 out = RN(out + y).  With a single group there is no per-block fp32 work, so this is a plain int8 MFMA
// GEMM with an epilogue, and the int32 sum is exact in any order.
//
// Packed weights (the engine's operand): w8a8_pc_wd_kernel, 128 x 256 tiles of 4 waves of 128 x 64, the activation
// rows staged through LDS and each wave's weight fragments loaded straight into registers (below).  Plain int8
// weights: w8a8_pc_tile_kernel, TM x 256 outputs (TM = 128 by default, or 256), waves of 128 x 64 (4 x 2
// v_mfma_i32_32x32x32_i8 per 32 inputs, 128 int32 accumulators per lane), 128 x 256 tiles of 4 waves in two LDS
// stages, three workgroups per CU, whose phases drift apart so that one's LDS fragment reads overlap another's MFMAs;
// one 256 x 256 workgroup of 8 waves per CU ran 4-6% slower, 4 waves of 128 x 128 6-13% slower, 16 waves of 128 x 32
// no faster.  Its operands go global -> LDS by LDS-DMA (global_load_lds_dwordx4), NS stages of 64 inputs: per stage
// and operand TM or 256 rows x 64 bytes, each DMA instruction 16 rows x 64 bytes (lane L: row L / 4, 16-byte chunk
// L % 4 swizzled by row, pc_swz).  MFMA operand mapping: lane l holds row l % 32 and the 16 inputs of chunk
// 2 s + l / 32 for the stage's 32-input step s, the same for both operands.
#include "common.h"

namespace prism {

constexpr int PCT = 256;                        // tile columns (and the default tile rows)
constexpr int PCK = 64;                         // inputs per stage
constexpr int PC_OPER = PCT * PCK;              // bytes per operand per stage (16 KB)
constexpr int PC_STAGE = 2 * PC_OPER;

// 16-byte chunk swizzle of a 64-byte operand row in LDS: chunk c of row r lies at slot c ^ ((r / 4) % 4), so the 16
// lanes a ds_read_b128 serves together (16 consecutive rows, one chunk each) fall on 16 distinct 16-byte bank groups
// ((r / 2) % 4, conflict-free over 8 rows only, cost 4 conflict cycles per read, measured).
__device__ __forceinline__ int pc_swz(int row) { return (row >> 2) & 3; }

// Staged activations of the decode kernel (STG): bytes per LDS row for `bytes` of a row (whole 1 KB pieces, plus 16 so
// the 16 rows' fragment reads spread over the banks).  Taken from kPcStageRows rows while the image fits kPcStageLds
// and the grid fits the CUs at once (one workgroup per CU then): 5120^2 / 5120 x 6144 / 3072 x 5120 at 16 rows 9.5 /
// 12.4 / 9.6 -> 8.5 / 10.2 / 8.4 us.  With more workgroups than CUs (17408 or 27648 x 5120) every round waits for its
// copy and it measured 20-25% slower; below 8 rows it does not pay.
__host__ __device__ constexpr int pc_stage_row_bytes(int bytes) { return (bytes + 1023) / 1024 * 1024 + 16; }
constexpr int kPcStageRows = 8;
constexpr size_t kPcStageLds = 150 * 1024;
constexpr int64_t kPcStageGrid = 256;


// Epilogue of a wave's 128 x 32 TN outputs at tile rows ml0 .. + 127, columns nl0 .. + 32 TN - 1: y = RN(RN(float(P) sa)
// sw), stored as bf16 (EPI 0) or added to the fp32 output (EPI 1).  acc[t][u] lane l: row 32 t + l % 32, columns
// 32 u + 8 g + 4 (l / 32) + e for element 4 g + e.
template <int EPI, int TN>
__device__ __forceinline__ void pc_store(const v16i (&acc)[4][TN], const float* sal, const float* swl, int ml0,
                                         int nl0, int lane, int m0, int n0, int live, int N, void* out, int64_t ldo) {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int ml = ml0 + 32 * t + r;
        const int m = m0 + ml;
        if (m >= live) continue;
        const float sa = sal[ml];
#pragma unroll
        for (int u = 0; u < TN; u++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int nl = nl0 + 32 * u + 8 * g + 4 * h;
                const int n = n0 + nl;
                if (n >= N) continue;
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = mul_rn(mul_rn((float)acc[t][u][4 * g + e], sa), swl[nl + e]);
                if (EPI == 0) {
                    uint16_t* o = static_cast<uint16_t*>(out) + (int64_t)m * ldo + n;
                    *reinterpret_cast<v2u*>(o) = v2u{f32_to_bf16(y[0]) | (f32_to_bf16(y[1]) << 16),
                                                     f32_to_bf16(y[2]) | (f32_to_bf16(y[3]) << 16)};
                } else {
                    float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * ldo + n);
                    const float4 p = *o;
                    *o = make_float4(add_rn(p.x, y[0]), add_rn(p.y, y[1]), add_rn(p.z, y[2]), add_rn(p.w, y[3]));
                }
            }
    }
}

template <bool WPACK, bool WS16, int EPI, int NS, int NWV, int TM>
__global__ __launch_bounds__(64 * NWV, TM == 128 ? 2 : 1) void w8a8_pc_tile_kernel(const int8_t* __restrict__ a,
                                                              const float* __restrict__ a_s, int64_t as_sm,
                                                              const int8_t* __restrict__ w,
                                                              const void* __restrict__ w_s, void* __restrict__ out,
                                                              int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                              int N, int K, int tiles_m, int tiles_n) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];   // NS x [A TM x 64 | W 256 x 64]
    __shared__ float sal[TM], swl[PCT];
    constexpr int AOPER = TM * PCK, STAGE = AOPER + PC_OPER;        // A operand bytes, stage bytes
    static_assert(TM == 128 || TM == 256, "tile rows");
    static_assert(NS * STAGE + (TM + PCT) * sizeof(float) <= (TM == 128 ? 80 : 160) * 1024,
                  "the stages and scales exceed the LDS share of a workgroup");
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * TM, n0 = pn * PCT;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int KS = K / PCK;
    constexpr int DIA = TM / 16 / NWV, DIW = 16 / NWV;   // DMA instructions per wave and stage: A, W
    static_assert(DIA >= 1 && DIW >= 1, "every wave copies a share of each operand");
    constexpr int WNC = NWV / (TM / 128);           // wave columns: TM / 128 waves of 128 rows by WNC of 256 / WNC
    constexpr int CW = PCT / WNC, TN = CW / 32;

    // epilogue scales of the tile
    if (tid < TM) sal[tid] = a_s[(int64_t)min(m0 + tid, M - 1) * as_sm];
    for (int t = tid; t < PCT; t += 64 * NWV) {
        const int n = min(n0 + t, N - 1);
        swl[t] = WS16 ? f16_to_f32(static_cast<const uint16_t*>(w_s)[n]) : static_cast<const float*>(w_s)[n];
    }

    // DMA sources: instruction i of wave wv covers operand rows 16 (D wv + i) .. + 15 (D = DIA, DIW); packed
    // weights: the 1 KB chunk of 16-row tile DIW wv + i as it lies (lane slot l: row l % 16, inputs 16 q .. + 15, q = l / 16)
    const int8_t* asrc[DIA];
    const int8_t* wsrc[DIW];
#pragma unroll
    for (int i = 0; i < DIA; i++) {
        const int row = 16 * (DIA * wv + i) + (lane >> 2);
        asrc[i] = a + (int64_t)min(m0 + row, M - 1) * K + 16 * ((lane & 3) ^ pc_swz(row));
    }
#pragma unroll
    for (int i = 0; i < DIW; i++) {
        const int row = 16 * (DIW * wv + i) + (lane >> 2);
        if (WPACK)
            wsrc[i] = w + ((int64_t)min(n0 / 16 + DIW * wv + i, N / 16 - 1) * (K / 64)) * 1024 + 16 * lane;
        else
            wsrc[i] = w + (int64_t)min(n0 + row, N - 1) * K + 16 * ((lane & 3) ^ pc_swz(row));
    }
    auto issue = [&](int st, int buf) {
        uint8_t* b = lds + buf * STAGE;
#pragma unroll
        for (int i = 0; i < DIA; i++) dma16(asrc[i] + (int64_t)st * PCK, b + (DIA * wv + i) * 1024);
#pragma unroll
        for (int i = 0; i < DIW; i++)
            dma16(wsrc[i] + (int64_t)st * (WPACK ? 1024 : PCK), b + AOPER + (DIW * wv + i) * 1024);
    };

    const int wm = wv / WNC, wn = wv % WNC;
    const int r = lane & 31, h = lane >> 5;
    // fragment byte offsets within an operand stage, for the two 32-input steps s: both operands' lanes hold inputs
    // 16 (2 s + h) .. + 15 (packed weights: the chunk's lane slot q = 2 s + h of the row).
    int aoff[2][4], woff[2][TN];
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int ra = 128 * wm + 32 * t + r;
            aoff[s][t] = ra * PCK + 16 * ((2 * s + h) ^ pc_swz(ra));
        }
#pragma unroll
        for (int u = 0; u < TN; u++) {
            const int rw = CW * wn + 32 * u + r;
            woff[s][u] = WPACK ? (rw >> 4) * 1024 + (16 * (2 * s + h) + (rw & 15)) * 16
                               : rw * PCK + 16 * ((2 * s + h) ^ pc_swz(rw));
        }
    }

    v16i acc[4][TN];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int u = 0; u < TN; u++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[t][u][e] = 0;

#pragma unroll
    for (int i = 0; i < NS - 1; i++)
        if (i < KS) issue(i, i);

    for (int st = 0; st < KS; st++) {
        const int pend = min(KS - 1, st + NS - 2) - st;     // stages issued after this one
        if (NS >= 4 && pend >= 2) vm_wait<2 * (DIA + DIW)>();
        else if (pend >= 1) vm_wait<DIA + DIW>();
        else vm_wait<0>();
        lds_barrier();
        if (st + NS - 1 < KS) issue(st + NS - 1, (st + NS - 1) % NS);
        const uint8_t* b = lds + (st % NS) * STAGE;
#pragma unroll
        for (int s = 0; s < 2; s++) {
            v4i fa[4], fw[TN];
#pragma unroll
            for (int t = 0; t < 4; t++) fa[t] = *reinterpret_cast<const v4i*>(b + aoff[s][t]);
#pragma unroll
            for (int u = 0; u < TN; u++) fw[u] = *reinterpret_cast<const v4i*>(b + AOPER + woff[s][u]);
            // D = W x A: lane l holds activation row l % 32 of the m-subtile and weight rows
            // 8 (e / 4) + 4 (l / 32) + e % 4 of the n-subtile
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int u = 0; u < TN; u++)
                    acc[t][u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[u], fa[t], acc[t][u], 0, 0, 0);
        }
    }

    pc_store<EPI, TN>(acc, sal, swl, 128 * wm, CW * wn, lane, m0, n0, live, N, out, ldo);
}

// Packed weights straight to registers: 128 x 256 tiles of 4 waves, wave wv computing all 128 rows by columns
// 64 wv .. + 63.  Only the activation rows, which all four waves read, go through LDS (two buffers); each weight
// fragment is read by one wave only, so it comes from the packed chunks by buffer loads (lane l: the 16 bytes of lane
// slot 2 s + l / 32, row l % 16 of a 16-row tile: the MFMA operand as it lies) two stages ahead in a register ring.
// That takes the weights' LDS writes and fragment reads (44% of the tile kernel's LDS traffic) off the LDS.  The
// activation rows are staged through registers (buffer loads two stages ahead, then one ds_write per 16 bytes)
// rather than by LDS-DMA: every request is then a plain load, and those complete in order, so one counted wait
// covers both operands (an LDS-DMA and later buffer loads were measured to complete out of order).  The rings are
// indexed by stage mod 6 in a loop unrolled by six, so every slot is a fixed register.  PAN: `a` is the panel image
// of pc_act_panel_kernel, so a wave's activation load for a stage is one 1 KB piece (C1 shape 1.20 -> 1.11 ms with
// the copy; the row-major form reads 16 rows' 64 bytes K apart per load).
template <bool WS16, int EPI, int TN, bool PAN = false>
__global__ __launch_bounds__(256, TN == 2 ? 2 : 1) void w8a8_pc_wd_kernel(const int8_t* __restrict__ a, const float* __restrict__ a_s,
                                                            int64_t as_sm, const int8_t* __restrict__ w,
                                                            const void* __restrict__ w_s, void* __restrict__ out,
                                                            int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                            int N, int K, int tiles_m, int tiles_n) {
    constexpr int TM = 128, TW = 128 * TN, DIA = 2, WL = 2 * TN, U = 6;   // tile columns TW; DIA activation and WL
                                                                          // weight loads per wave and stage
    constexpr int AOPER = TM * PCK;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * AOPER];
    __shared__ float sal[TM], swl[TW];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int pm, pn;
    xcd_tile_coords(blockIdx.x, tiles_m, tiles_n, pm, pn);
    const int m0 = pm * TM, n0 = pn * TW;
    const int live = min(M, __ldg(n_rows));
    if (m0 >= live) return;
    const int KS = K / PCK;

    if (tid < TM) sal[tid] = a_s[(int64_t)min(m0 + tid, M - 1) * as_sm];
    for (int t = tid; t < TW; t += 256) {
        const int n = min(n0 + t, N - 1);
        swl[t] = WS16 ? f16_to_f32(static_cast<const uint16_t*>(w_s)[n]) : static_cast<const float*>(w_s)[n];
    }

    // activations: lane L of copy i holds row 16 (DIA wv + i) + L / 4, 16-byte chunk (L % 4) ^ swz of the stage's 64
    // inputs, stored at LDS byte (DIA wv + i) 1024 + 16 L
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a + (int64_t)m0 * K);
    uint32_t ao[DIA];
#pragma unroll
    for (int i = 0; i < DIA; i++) {
        const int row = 16 * (DIA * wv + i) + (lane >> 2);
        ao[i] = PAN ? (uint32_t)((min(m0 / 16 + DIA * wv + i, (M - 1) / 16) - m0 / 16) * KS * 1024 + 16 * lane)
                    : (uint32_t)(min(row, M - 1 - m0) * K + 16 * ((lane & 3) ^ pc_swz(row)));
    }
    const int r = lane & 31, h = lane >> 5;
    const int nt0 = n0 >> 4;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(w + (int64_t)nt0 * KS * 1024);
    uint32_t wo[2][TN];
#pragma unroll
    for (int u = 0; u < TN; u++) {
        const int t = min(nt0 + 2 * TN * wv + 2 * u + (r >> 4), N / 16 - 1) - nt0;
#pragma unroll
        for (int s = 0; s < 2; s++) wo[s][u] = (uint32_t)(t * KS * 1024 + (16 * (2 * s + h) + (r & 15)) * 16);
    }
    v4i xr[2][DIA], wr[3][2][TN];
    auto load = [&](int st, v4i (&x)[DIA], v4i (&f)[2][TN]) {       // activations first, then weights
#pragma unroll
        for (int i = 0; i < DIA; i++) x[i] = buf_load16(ra, ao[i], (uint32_t)st * (PAN ? 1024 : PCK));
        __builtin_amdgcn_sched_barrier(0);         // kept in this order: the waits count the weight loads last
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int u = 0; u < TN; u++) f[s][u] = buf_load16(rw, wo[s][u], (uint32_t)st * 1024);
    };
    auto stage_store = [&](int st, const v4i (&x)[DIA]) {
#pragma unroll
        for (int i = 0; i < DIA; i++)
            *reinterpret_cast<v4i*>(lds + (st & 1) * AOPER + (DIA * wv + i) * 1024 + 16 * lane) = x[i];
    };
    int aoff[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int ra_ = 32 * t + r;
            aoff[s][t] = ra_ * PCK + 16 * ((2 * s + h) ^ pc_swz(ra_));
        }

    v16i acc[4][TN];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int u = 0; u < TN; u++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[t][u][e] = 0;

    // Stage indices past the last are clamped to it (redundant loads into slots never read), so every step issues
    // the same DIA + WL loads and the waits are fixed counts.  Step st: wait for stage st + 1's activations and
    // stage st's weights (only stage st + 1's WL weight loads were issued after the former); store those
    // activations into the free LDS buffer; read stage st's fragments; request stage st + 2; barrier; MFMAs.
    load(0, xr[0], wr[0]);
    load(min(1, KS - 1), xr[1], wr[1]);
    vm_wait_tracked<DIA + 2 * WL>();
    stage_store(0, xr[0]);
    lds_barrier();
    auto step = [&](int st, int j) {                 // j = st mod 6: register slots st mod 2 and st mod 3
        vm_wait_tracked<WL>();
        stage_store(st + 1, xr[(j + 1) % 2]);       // past the end: into the free buffer, never read
        const uint8_t* b = lds + (st & 1) * AOPER;
        v4i fa[2][4];
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int t = 0; t < 4; t++) fa[s][t] = *reinterpret_cast<const v4i*>(b + aoff[s][t]);
        load(min(st + 2, KS - 1), xr[j % 2], wr[(j + 2) % 3]);
        lds_barrier();
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int u = 0; u < TN; u++)
                    acc[t][u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wr[j % 3][s][u], fa[s][t], acc[t][u], 0, 0, 0);
    };
    int st = 0;
    for (; st + U <= KS; st += U) {
#pragma unroll
        for (int j = 0; j < U; j++) step(st + j, j);
    }
#pragma unroll
    for (int j = 0; j < U - 1; j++)
        if (st + j < KS) step(st + j, j);
    pc_store<EPI, TN>(acc, sal, swl, 0, 32 * TN * wv, lane, m0, n0, live, N, out, ldo);
}

// Panel image of the activations for w8a8_pc_wd_kernel<.., true>: 16-row blocks of K / 64 chunks of 1 KB, block b
// starting at byte 16 b K; chunk st holds what the kernel's lane L stores at LDS byte 16 L for the block's stage st:
// row 16 b + L / 4 (clamped to M - 1), inputs 64 st + 16 ((L % 4) ^ pc_swz(L / 4)) .. + 15.  One workgroup per
// (block, 1024 inputs); each row's 1 KB is read in one piece.
__global__ __launch_bounds__(256) void pc_act_panel_kernel(const int8_t* __restrict__ a, int8_t* __restrict__ pan,
                                                           int M, int K) {
    const int rb = blockIdx.y, KS = K / PCK;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int piece = threadIdx.x + 256 * j, r = piece >> 6;
        const int k = 1024 * blockIdx.x + 16 * (piece & 63);
        if (k >= K) continue;
        const v4i v = *reinterpret_cast<const v4i*>(a + (int64_t)min(16 * rb + r, M - 1) * K + k);
        const int L = 4 * r + (((k >> 4) & 3) ^ pc_swz(r));
        *reinterpret_cast<v4i*>(pan + ((int64_t)rb * KS + (k >> 6)) * 1024 + 16 * L) = v;
    }
}

// The panel copy (2 M K bytes of traffic first) pays where many column tiles read each activation panel: measured
// at 27648 x 5120, 2048 / 4096 rows 281 / 597 -> 271 / 555 us; at N = 1024 - 5120 it cost 0-15%, at 17408 x 5120
// and 1024 rows 1% (M N below 2^25).
constexpr int kPcPanelRows = 1024, kPcPanelCols = 16384;
// The split decode reads a panel copy too from 48 rows on K >= 8192 (the copy is a launch and 2 M K bytes).
constexpr int kPcDecodePanelRows = 48, kPcDecodePanelK = 8192;

int64_t pc_panel_bytes(int64_t M, int64_t K) { return (M + 15) / 16 * 16 * K; }

// The tile kernel on the panel image of `a` built in ws first.  The caller has checked the shapes, the alignment,
// packed weights with N K < 2^31 and ws of pc_panel_bytes.
int launch_w8a8_pc_panels(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* w, const void* w_s,
                          bool ws16, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int epi,
                          void* ws, hipStream_t st) {
    int8_t* pan = static_cast<int8_t*>(ws);
    hipLaunchKernelGGL(pc_act_panel_kernel, dim3((unsigned)((K + 1023) / 1024), (unsigned)((M + 15) / 16)), dim3(256),
                       0, st, a, pan, M, K);
    PRISM_LAUNCH_CHECK();
    constexpr int TN = 2;
    const int tiles_m = (M + 127) / 128, tiles_n = (N + 128 * TN - 1) / (128 * TN);
#define PPL(W16, E)                                                                                                \
    hipLaunchKernelGGL((w8a8_pc_wd_kernel<W16, E, TN, true>), dim3(tiles_m * tiles_n), dim3(256), 0, st, pan, a_s, \
                       as_sm, w, w_s, out, ldo, n_rows, M, N, K, tiles_m, tiles_n)
    if (ws16) { if (epi == 0) PPL(true, 0); else PPL(true, 1); }
    else { if (epi == 0) PPL(false, 0); else PPL(false, 1); }
#undef PPL
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

// ---------------------------------------------------------------------------------------------- decode
// Rows r0 .. r0 + 16 MT - 1 with r0 = 16 MT blockIdx.y (grid rows cover M beyond 64: for narrow projections, whose
// few 128 x 256 tiles leave the tile kernel's CUs idle, the weight tiles then come from L2 / MALL once per 64 rows).
// One workgroup per G 16-row weight tiles; wave w takes the 64-input chunks w, w + NW, ... of every tile (the int32
// sums are exact in any order), PD = 4 chunks in flight in registers (at most 8 waves, so up to 256 VGPRs).  Per
// chunk a lane loads 16 bytes of each tile's weights (row l % 16, inputs 16 q .. + 15: packed, the chunk's lane slot, 1 KB per wave
// instruction) and the same 16 inputs of its activation row per m-tile, reused across the G tiles; one
// v_mfma_i32_16x16x64_i8 per (tile, m-tile) accumulates into int32.  The waves' sums meet in LDS, and the epilogue
// applies the two roundings.
// PAN: `a` is the panel copy of pc_act_panel_kernel (lane (lm, q)'s 16 bytes of a chunk at 16 (4 lm + (q ^
// pc_swz(lm))) of the block's 1 KB), so each activation load is one 1 KB piece.
// STG (MT == 1): the workgroup first copies its 16 activation rows over its K range into LDS by LDS-DMA, one 1 KB
// row piece per instruction (rows pc_stage_row_bytes apart), and the MFMA operands come from there instead of 16
// rows' 64 bytes per load.
template <int G, int MT, bool WPACK, bool WS16, int EPI, bool PAN = false, bool STG = false>
__global__ __launch_bounds__(512) void w8a8_pc_decode_kernel(const int8_t* __restrict__ a,
                                                              const float* __restrict__ a_s, int64_t as_sm,
                                                              const int8_t* __restrict__ w,
                                                              const void* __restrict__ w_s, void* __restrict__ out,
                                                              int64_t ldo, const int32_t* __restrict__ n_rows, int M,
                                                              int N, int K, int64_t zstride) {
    constexpr int PD = 4;
    extern __shared__ __attribute__((aligned(16))) v4i red[];          // [NW][G][MT][64]
    // every argument fetched at once (else one scalar round trip per first use before the first weight request)
    const int gz = gridDim.z;
    asm volatile("" ::"s"(a), "s"(a_s), "s"(as_sm), "s"(w), "s"(w_s), "s"(out), "s"(ldo), "s"(n_rows), "s"(M), "s"(N),
                 "s"(K), "s"(zstride), "s"(gz));
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, NW = blockDim.x >> 6;
    const int nt0 = blockIdx.x * G, r0 = 16 * MT * blockIdx.y;
    const int KP = K / 64, NT = N / 16;
    // split z of gridDim.z takes the 64-input chunks kc0 .. kc1 - 1 (EPI 2: its int32 sums go to slot z)
    const int z = blockIdx.z;
    const int kc0 = KP * z / gz, KC = KP * (z + 1) / gz - kc0;        // KP * split < 2^31 (host)
    const int lm = lane & 15, q = lane >> 4;

    const int8_t* wb[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int t = min(nt0 + g, NT - 1);
        wb[g] = WPACK ? w + (int64_t)t * KP * 1024 + 16 * lane : w + (int64_t)(16 * t + lm) * K + 16 * q;
    }
    const int8_t* ab[MT];
#pragma unroll
    for (int u = 0; u < MT; u++)
        ab[u] = PAN ? a + (int64_t)min((r0 + 16 * u) / 16, (M - 1) / 16) * 16 * K + 16 * (4 * lm + (q ^ pc_swz(lm)))
                    : a + (int64_t)min(r0 + 16 * u + lm, M - 1) * K + 16 * q;

    // both layouts give lane (lm, q) the 16 inputs 64 j + 16 q .. + 15 of its weight row and of its activation row:
    // one v_mfma_i32_16x16x64_i8 per (tile, m-tile) and chunk
    struct Chunk {
        v4i w[G];
        v4i x[MT];
    };
    auto load = [&](int j, Chunk& c) {
        const int jj = kc0 + min(j, KC - 1);
#pragma unroll
        for (int g = 0; g < G; g++) c.w[g] = *reinterpret_cast<const v4i*>(wb[g] + (int64_t)jj * (WPACK ? 1024 : 64));
        if (!STG) {
#pragma unroll
            for (int u = 0; u < MT; u++) c.x[u] = *reinterpret_cast<const v4i*>(ab[u] + (int64_t)jj * (PAN ? 1024 : 64));
        }
    };
    const int rowb = STG ? (KC * 64 + 1023) / 1024 * 1024 + 16 : 0;
    // one 16-row block: the image after the reduction buffer; more: the image where the reduction buffer goes (a
    // barrier separates the last image read from the first reduction write)
    const int8_t* img = reinterpret_cast<const int8_t*>(MT == 1 ? red + NW * G * MT * 64 : red);
    if (STG) {
        const int pieces = (KC * 64 + 1023) / 1024;
        for (int row = wv; row < 16 * MT; row += NW) {
            const int8_t* src = a + (int64_t)min(r0 + row, M - 1) * K + (int64_t)kc0 * 64;
            for (int pc = 0; pc < pieces; pc++)
                // lanes past the range re-read its last 16 bytes into the row's padding (never read)
                __builtin_amdgcn_global_load_lds(
                    src + min(1024 * pc + 16 * lane, KC * 64 - 16),
                    (__attribute__((address_space(3))) void*)(img + row * rowb + 1024 * pc), 16, 0, 0);
        }
    }
    v4i acc[G][MT];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int u = 0; u < MT; u++) acc[g][u] = v4i{0, 0, 0, 0};
    auto mma = [&](Chunk& c, int j) {
        if (STG) {
#pragma unroll
            for (int u = 0; u < MT; u++)
                c.x[u] = *reinterpret_cast<const v4i*>(img + (16 * u + lm) * rowb + min(j, KC - 1) * 64 + 16 * q);
        }
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int u = 0; u < MT; u++) acc[g][u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c.w[g], c.x[u], acc[g][u], 0, 0, 0);
    };
    // this wave's chunks: j = wv + NW i, i < cnt; branch-free body over whole rings of PD
    const int cnt = wv < KC ? (KC - wv + NW - 1) / NW : 0;
    Chunk ring[PD];
#pragma unroll
    for (int d = 0; d < PD; d++) load(wv + NW * d, ring[d]);
    if (STG) {                                       // the image complete before the first fragment read
        vm_wait_tracked<0>();
        __syncthreads();
    }
    const int full = cnt / PD * PD;
    for (int i0 = 0; i0 < full; i0 += PD) {
#pragma unroll
        for (int d = 0; d < PD; d++) {
            mma(ring[d], wv + NW * (i0 + d));
            load(wv + NW * (i0 + d + PD), ring[d]);
            // keep each chunk's MFMAs in place: hoisted across chunks, they would wait for the whole ring
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int d = 0; d < PD; d++)
        if (full + d < cnt) mma(ring[d], wv + NW * (full + d));

    if (STG && MT > 1) __syncthreads();              // every wave's image reads done: the sums overwrite it
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int u = 0; u < MT; u++) red[((wv * G + g) * MT + u) * 64 + lane] = acc[g][u];
    __syncthreads();
    // the live-row count only here: read before the first requests it would hold them back by a round trip, so
    // every workgroup computes and the stores skip rows >= n_rows (no early exit either: with one after the first
    // requests this kernel computed wrong sums on MI355X at 8 x 368 x 3008, epilogue 1, a case the random-shape
    // test holds)
    const int live = min(M, __ldg(n_rows));
    for (int idx = tid; idx < G * MT * 64; idx += blockDim.x) {
        const int g = idx / (MT * 64), u = (idx >> 6) % MT, l = idx & 63;
        const int m = r0 + 16 * u + (l & 15), t = nt0 + g;
        if (m >= live || t >= NT) continue;
        v4i P = red[idx];
        for (int v = 1; v < NW; v++) {
            const v4i u = red[v * G * MT * 64 + idx];
            P = v4i{P.x + u.x, P.y + u.y, P.z + u.z, P.w + u.w};
        }
        const int n = 16 * t + 4 * (l >> 4);
        if (EPI == 2) {                                                 // a deferred split: the raw int32 sums
            *reinterpret_cast<v4i*>(static_cast<int32_t*>(out) + z * zstride + (int64_t)m * ldo + n) = P;
            continue;
        }
        const float sa = a_s[(int64_t)m * as_sm];
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float sw = WS16 ? f16_to_f32(static_cast<const uint16_t*>(w_s)[n + e])
                                  : static_cast<const float*>(w_s)[n + e];
            y[e] = mul_rn(mul_rn((float)P[e], sa), sw);
        }
        if (EPI == 0) {
            uint16_t* o = static_cast<uint16_t*>(out) + (int64_t)m * ldo + n;
            *reinterpret_cast<v2u*>(o) = v2u{f32_to_bf16(y[0]) | (f32_to_bf16(y[1]) << 16),
                                             f32_to_bf16(y[2]) | (f32_to_bf16(y[3]) << 16)};
        } else {
            float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * ldo + n);
            const float4 p = *o;
            *o = make_float4(add_rn(p.x, y[0]), add_rn(p.y, y[1]), add_rn(p.z, y[2]), add_rn(p.w, y[3]));
        }
    }
}


// Per-channel launch: kernel 1 the decode kernel (up to 64 rows per workgroup, grid rows beyond), else the tile
// kernel.  epi 2 (decode kernel only): K in `split` parts, part z's int32 sums to out + z zstride.  The caller has
// checked K % 64 == 0, 16-byte aligned a / w, ldo % 4 == 0 and an 8 / 16-byte aligned out.
int launch_w8a8_pc(int kernel, bool wpack, const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* w,
                   const void* w_s, bool ws16, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K,
                   int epi, hipStream_t st, int split, int64_t zstride) {
    if (kernel == 1) {
        const int MT = min(4, (M + 15) / 16);
        const int G = (N % 32 == 0) ? 2 : 1;
        const int KP = K / 64 / split;
        int nw = min(8, max(1, KP / 4));  // 8 waves (the launch bound), 4 chunks each in flight (16 waves measured slower)
        const size_t lds = (size_t)nw * G * MT * 64 * sizeof(v4i);
        dim3 grid((unsigned)(N / (16 * G)), (unsigned)((M + 16 * MT - 1) / (16 * MT)), (unsigned)split);
#ifndef PC_STG
#define PC_STG 1
#endif
        const size_t stg = lds + 16 * (size_t)pc_stage_row_bytes((KP + 1) * 64);
        if (PC_STG && MT == 1 && wpack && epi != 2 && M >= kPcStageRows && stg <= kPcStageLds &&
            (int64_t)grid.x * grid.y * grid.z <= kPcStageGrid) {
#define PDS(GV, W16, E)                                                                                            \
    do {                                                                                                           \
        allow_lds(w8a8_pc_decode_kernel<GV, 1, true, W16, E, false, true>, stg);                                   \
        hipLaunchKernelGGL((w8a8_pc_decode_kernel<GV, 1, true, W16, E, false, true>), grid, dim3(64 * nw), stg, st, a, \
                           a_s, as_sm, w, w_s, out, ldo, n_rows, M, N, K, zstride);                                \
    } while (0)
#define PDS_G(W16, E) do { if (G == 2) PDS(2, W16, E); else PDS(1, W16, E); } while (0)
            if (ws16) { if (epi == 0) PDS_G(true, 0); else PDS_G(true, 1); }
            else { if (epi == 0) PDS_G(false, 0); else PDS_G(false, 1); }
#undef PDS_G
#undef PDS
            PRISM_LAUNCH_CHECK();
            return PRISM_OK;
        }
#define PDL(GV, MTV, WP, W16, E)                                                                                   \
    hipLaunchKernelGGL((w8a8_pc_decode_kernel<GV, MTV, WP, W16, E>), grid, dim3(64 * nw), lds, st, a, a_s, as_sm, w, \
                       w_s, out, ldo, n_rows, M, N, K, zstride)
#define PDL_MT(GV, WP, W16, E)                                                                                     \
    do {                                                                                                           \
        if (MT == 1) PDL(GV, 1, WP, W16, E); else if (MT == 2) PDL(GV, 2, WP, W16, E);                             \
        else if (MT == 3) PDL(GV, 3, WP, W16, E); else PDL(GV, 4, WP, W16, E);                                     \
    } while (0)
#define PDL_G(WP, W16, E) do { if (G == 2) PDL_MT(2, WP, W16, E); else PDL_MT(1, WP, W16, E); } while (0)
#define PDL_WP(W16, E) do { if (wpack) PDL_G(true, W16, E); else PDL_G(false, W16, E); } while (0)
        if (epi == 2) PDL_WP(false, 2);
        else if (ws16) { if (epi == 0) PDL_WP(true, 0); else PDL_WP(true, 1); }
        else { if (epi == 0) PDL_WP(false, 0); else PDL_WP(false, 1); }
#undef PDL_WP
#undef PDL_G
#undef PDL_MT
#undef PDL
        PRISM_LAUNCH_CHECK();
        return PRISM_OK;
    }
#ifndef PC_WD
#define PC_WD 1                                   // packed weights: the direct-weight tile kernel, 128 x 256 TN
                                                  // (1: TN 2, 2: TN 4; 0: the LDS tile kernel)
#endif
    if (PC_WD && wpack && (int64_t)N * K < (1LL << 31)) {
#define PWL(W16, E, TN)                                                                                            \
    hipLaunchKernelGGL((w8a8_pc_wd_kernel<W16, E, TN>), dim3(tiles_m * tiles_n), dim3(256), 0, st, a, a_s, as_sm, w,\
                       w_s, out, ldo, n_rows, M, N, K, tiles_m, tiles_n)
#define PWL_T(TN)                                                                                                  \
    do {                                                                                                           \
        const int tiles_m = (M + 127) / 128, tiles_n = (N + 128 * TN - 1) / (128 * TN);                           \
        if (ws16) { if (epi == 0) PWL(true, 0, TN); else PWL(true, 1, TN); }                                       \
        else { if (epi == 0) PWL(false, 0, TN); else PWL(false, 1, TN); }                                          \
    } while (0)
        if (PC_WD == 2) PWL_T(4);
        else PWL_T(2);
#undef PWL_T
#undef PWL
        PRISM_LAUNCH_CHECK();
        return PRISM_OK;
    }
#ifndef PC_TILE
#define PC_TILE 2, 4, 128                         // LDS stages, waves per workgroup, tile rows (tile columns: 256)
#endif
#define PCT_(A, B, C) constexpr int NS = A, PC_NWV = B, PC_TM = C;
#define PCT__(...) PCT_(__VA_ARGS__)
    PCT__(PC_TILE)
#undef PCT__
#undef PCT_
    const int tiles_m = (M + PC_TM - 1) / PC_TM, tiles_n = (N + PCT - 1) / PCT;
    const size_t lds = (size_t)NS * (PC_TM * PCK + PC_OPER);
#define PCL(WP, W16, E)                                                                                            \
    do {                                                                                                           \
        allow_lds(w8a8_pc_tile_kernel<WP, W16, E, NS, PC_NWV, PC_TM>, lds);                                         \
        hipLaunchKernelGGL((w8a8_pc_tile_kernel<WP, W16, E, NS, PC_NWV, PC_TM>), dim3(tiles_m * tiles_n),          \
                           dim3(64 * PC_NWV),                                                                      \
                           lds, st, a,                                                                             \
                           a_s, as_sm, w, w_s, out, ldo, n_rows, M, N, K, tiles_m, tiles_n);                        \
    } while (0)
#define PCL_WP(W16, E) do { if (wpack) PCL(true, W16, E); else PCL(false, W16, E); } while (0)
    if (ws16) { if (epi == 0) PCL_WP(true, 0); else PCL_WP(true, 1); }
    else { if (epi == 0) PCL_WP(false, 0); else PCL_WP(false, 1); }
#undef PCL_WP
#undef PCL
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

// The split decode on packed weights (kernel 2): four 16-row weight tiles per workgroup (two where N is not a
// multiple of 64) and K in three parts, each part's int32 sums into its slot of the workspace (the decode kernel's
// epilogue 2), then pc_fold_kernel adds the three slots (exact in any order) and applies the epilogue.  Every
// workgroup reads all activation rows over its K range, so with four tiles per workgroup the activation rows are read
// half as often per weight byte as with the unsplit kernel's two, while 3 N / 64 workgroups still cover the CUs:
// at 64 rows, 5120 x 17408 -> 5120, 46.8 -> 25.9 us for the sums.  Two or four parts lost most of that gain.  The
// parts meet at the launch boundary rather than through counters and a last-arriving part: the partial sums would
// then have to be written and read device-coherently (agent scope), past the XCDs' separate L2s, which measured
// 38 us for the same product.
constexpr int kPcSplit = 3;
constexpr int kPcSplitRows = 512;     // rows the split takes (grid rows of 64 beyond 64)

int64_t pc_split_workspace_bytes(int64_t M, int64_t N) { return (int64_t)kPcSplit * M * N * 4; }

// out rows m < n_rows: y = RN(RN(float(sum_z slots[z][m][n]) sa) sw), stored as bf16 (EPI 0) or added (EPI 1).
template <bool WS16, int EPI>
__global__ __launch_bounds__(256) void pc_fold_kernel(const int32_t* __restrict__ slots, int64_t zstride, int S,
                                                      const float* __restrict__ a_s, int64_t as_sm,
                                                      const void* __restrict__ w_s, void* __restrict__ out,
                                                      int64_t ldo, const int32_t* __restrict__ n_rows, int M, int N) {
    const int m = blockIdx.y, n = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (n >= N || m >= min(M, __ldg(n_rows))) return;
    v4i P = v4i{0, 0, 0, 0};
    for (int z = 0; z < S; z++) {
        const v4i u = *reinterpret_cast<const v4i*>(slots + z * zstride + (int64_t)m * N + n);
        P = v4i{P.x + u.x, P.y + u.y, P.z + u.z, P.w + u.w};
    }
    const float sa = a_s[(int64_t)m * as_sm];
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float sw = WS16 ? f16_to_f32(static_cast<const uint16_t*>(w_s)[n + e]) : static_cast<const float*>(w_s)[n + e];
        y[e] = mul_rn(mul_rn((float)P[e], sa), sw);
    }
    if (EPI == 0) {
        uint16_t* o = static_cast<uint16_t*>(out) + (int64_t)m * ldo + n;
        *reinterpret_cast<v2u*>(o) = v2u{f32_to_bf16(y[0]) | (f32_to_bf16(y[1]) << 16),
                                         f32_to_bf16(y[2]) | (f32_to_bf16(y[3]) << 16)};
    } else {
        float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * ldo + n);
        const float4 p = *o;
        *o = make_float4(add_rn(p.x, y[0]), add_rn(p.y, y[1]), add_rn(p.z, y[2]), add_rn(p.w, y[3]));
    }
}

// pan: null, or room for the panel copy of `a` (pc_panel_bytes) that the decode kernel then reads
int launch_w8a8_pc_split(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* w, const void* w_s,
                         bool ws16, void* out, int64_t ldo, const int32_t* n_rows, int M, int N, int K, int epi,
                         void* ws, hipStream_t st, int8_t* pan) {
    const int MT = min(4, (M + 15) / 16);
    const int G = N % 64 == 0 ? 4 : (N % 32 == 0 ? 2 : 1);
    const int KP = K / 64 / kPcSplit;
    const int nw = min(8, max(1, KP / 4));
    const size_t lds = (size_t)nw * G * MT * 64 * sizeof(v4i);
    int32_t* slots = static_cast<int32_t*>(ws);
    const int64_t zstride = (int64_t)M * N;
    dim3 grid((unsigned)(N / (16 * G)), (unsigned)((M + 16 * MT - 1) / (16 * MT)), (unsigned)kPcSplit);
    if (pan) {
        hipLaunchKernelGGL(pc_act_panel_kernel, dim3((unsigned)((K + 1023) / 1024), (unsigned)((M + 15) / 16)),
                           dim3(256), 0, st, a, pan, M, K);
        PRISM_LAUNCH_CHECK();
    }
    // staged activations: one 16-row block (image after the sums), or up to four (image in the sums' place)
    const size_t img = 16 * (size_t)MT * pc_stage_row_bytes((KP + 1) * 64);
    const size_t stg = MT == 1 ? lds + img : std::max(lds, img);
#ifndef PC_STG_MT
#define PC_STG_MT 4
#endif
    if (PC_STG && MT <= PC_STG_MT && !pan && M >= kPcStageRows && stg <= kPcStageLds &&
        (int64_t)grid.x * grid.y * grid.z <= kPcStageGrid) {
#define PSS(GV, MTV)                                                                                               \
    do {                                                                                                           \
        allow_lds(w8a8_pc_decode_kernel<GV, MTV, true, false, 2, false, true>, stg);                               \
        hipLaunchKernelGGL((w8a8_pc_decode_kernel<GV, MTV, true, false, 2, false, true>), grid, dim3(64 * nw), stg, \
                           st, a, a_s, as_sm, w, w_s, slots, (int64_t)N, n_rows, M, N, K, zstride);                \
    } while (0)
#define PSS_MT(GV)                                                                                                 \
    do {                                                                                                           \
        if (MT == 1) PSS(GV, 1); else if (MT == 2) PSS(GV, 2); else if (MT == 3) PSS(GV, 3); else PSS(GV, 4);      \
    } while (0)
        if (G == 4) PSS_MT(4); else if (G == 2) PSS_MT(2); else PSS_MT(1);
#undef PSS_MT
#undef PSS
    } else {
#define PSL(GV, MTV)                                                                                               \
    do {                                                                                                           \
        if (pan)                                                                                                   \
            hipLaunchKernelGGL((w8a8_pc_decode_kernel<GV, MTV, true, false, 2, true>), grid, dim3(64 * nw), lds, st, \
                               pan, a_s, as_sm, w, w_s, slots, (int64_t)N, n_rows, M, N, K, zstride);              \
        else                                                                                                       \
            hipLaunchKernelGGL((w8a8_pc_decode_kernel<GV, MTV, true, false, 2>), grid, dim3(64 * nw), lds, st, a,  \
                               a_s, as_sm, w, w_s, slots, (int64_t)N, n_rows, M, N, K, zstride);                   \
    } while (0)
#define PSL_MT(GV)                                                                                                 \
    do {                                                                                                           \
        if (MT == 1) PSL(GV, 1); else if (MT == 2) PSL(GV, 2); else if (MT == 3) PSL(GV, 3); else PSL(GV, 4);      \
    } while (0)
    if (G == 4) PSL_MT(4); else if (G == 2) PSL_MT(2); else PSL_MT(1);
#undef PSL_MT
#undef PSL
    }
    PRISM_LAUNCH_CHECK();
    dim3 fgrid((unsigned)((N / 4 + 255) / 256), (unsigned)M);
#define PFL(W16, E) hipLaunchKernelGGL((pc_fold_kernel<W16, E>), fgrid, dim3(256), 0, st, slots, zstride, kPcSplit, a_s, \
                                       as_sm, w_s, out, ldo, n_rows, M, N)
    if (ws16) { if (epi == 0) PFL(true, 0); else PFL(true, 1); }
    else { if (epi == 0) PFL(false, 0); else PFL(false, 1); }
#undef PFL
    PRISM_LAUNCH_CHECK();
    return PRISM_OK;
}

}  // namespace prism

using namespace prism;

extern "C" int prism_w8a8_pc_packed_gemm(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                         const void* w_s, int ws_fp16, void* out, int64_t ldo, const int32_t* n_rows,
                                         int64_t M, int64_t N, int64_t K, int epi, int kernel, void* stream);

extern "C" int64_t prism_w8a8_pc_split_workspace_bytes(int64_t M, int64_t N) {
    if (M <= 0 || N <= 0 || M > kPcSplitRows || N % 16) return 0;
    return pc_split_workspace_bytes(M, N);
}

// prism_w8a8_pc_packed_gemm with the workspace of the split decode (kernel 2).  kernel -1 with a workspace that holds
// the split takes it where it measured faster (below), else picks as prism_w8a8_pc_packed_gemm; 0 / 1 as there.
extern "C" int prism_w8a8_pc_packed_gemm_ws(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                            const void* w_s, int ws_fp16, void* out, int64_t ldo,
                                            const int32_t* n_rows, int64_t M, int64_t N, int64_t K, int epi,
                                            int kernel, void* ws, int64_t ws_bytes, void* stream) {
    if (kernel < -1 || kernel > 2) return PRISM_ERR_ARG;
    const bool fits = ws && M >= 1 && M <= kPcSplitRows && N % 16 == 0 && K / 64 >= 4 * kPcSplit &&
                      ws_bytes >= pc_split_workspace_bytes(M, N) && PRISM_ALIGNED(ws, 256);
    if (kernel == 2 && !fits) return ws ? PRISM_ERR_SHAPE : PRISM_ERR_ARG;
    // without a table entry: the split where it measured faster (long K from 16 rows: 5120 x 17408 -> 5120 at 16 /
    // 32 / 64 rows 24.5 / 34.0 / 46.5 -> 21.8 / 24.0 / 29.7 us, at 128 / 256 / 384 rows 80.4 / 117.4 / 151.5 ->
    // 43.5 / 70.4 / 87.1 us with the panel copy, against 107.7 us for the tile kernel at 384; up to N = 5120 at 48 - 64
    // rows: 5120^2 at 64 rows 17.9 -> 16.5 us); below 16 rows, on wide projections and from 512 rows on (the tile
    // kernel) the unsplit kernels stay ahead
    if (kernel == -1 && fits && M >= 16 &&
        ((M <= 64 && (K >= 12288 || (M >= 48 && N <= 5120))) || (M <= 384 && K >= 12288 && N <= 8192)))
        kernel = 2;
    // the tile kernel on panel activations where ws holds them and the shape is wide enough to repay the copy; the
    // table's "tile" choice and kernel 0 take it too
    if ((kernel == 0 || (kernel == -1 && M > 64)) && M >= kPcPanelRows && N >= kPcPanelCols &&
        M * N >= (1LL << 25) && ws &&
        ws_bytes >= pc_panel_bytes(M, K) &&
        PRISM_ALIGNED(ws, 256) && N * K < (1LL << 31) && M <= 65535 * 16 && N % 16 == 0 && K % 64 == 0 &&
        K <= (1 << 17)) {
        if (!a || !a_s || !qt || !w_s || !out || !n_rows) return PRISM_ERR_ARG;
        if (epi != 0 && epi != 1) return PRISM_ERR_ARG;
        if (ldo < N) return PRISM_ERR_SHAPE;
        if (!PRISM_ALIGNED(a, 16) || !PRISM_ALIGNED(qt, 16) || ldo % 4 || !PRISM_ALIGNED(out, epi ? 16 : 8))
            return PRISM_ERR_ALIGN;
        return launch_w8a8_pc_panels(a, a_s, as_sm, qt, w_s, ws_fp16 != 0, out, ldo, n_rows, (int)M, (int)N, (int)K,
                                     epi, ws, (hipStream_t)stream);
    }
    if (kernel != 2)
        return prism_w8a8_pc_packed_gemm(a, a_s, as_sm, qt, w_s, ws_fp16, out, ldo, n_rows, M, N, K, epi, kernel,
                                         stream);
    if (!a || !a_s || !qt || !w_s || !out || !n_rows) return PRISM_ERR_ARG;
    if (epi != 0 && epi != 1) return PRISM_ERR_ARG;
    if (N <= 0 || K <= 0 || K % 64 || ldo < N || K > (1 << 17)) return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(a, 16) || !PRISM_ALIGNED(qt, 16) || ldo % 4 || !PRISM_ALIGNED(out, epi ? 16 : 8))
        return PRISM_ERR_ALIGN;
    // the decode kernel on a panel copy of the activations, after the slots, from 48 rows on long K (5120 x 17408 at
    // 64 rows: 31.7 -> 28.x us with the copy)
    int8_t* pan = nullptr;
    const int64_t slot_bytes = (pc_split_workspace_bytes(M, N) + 255) / 256 * 256;
    if (M >= kPcDecodePanelRows && K >= kPcDecodePanelK && ws_bytes >= slot_bytes + pc_panel_bytes(M, K))
        pan = static_cast<int8_t*>(ws) + slot_bytes;
    return launch_w8a8_pc_split(a, a_s, as_sm, qt, w_s, ws_fp16 != 0, out, ldo, n_rows, (int)M, (int)N, (int)K,
                                epi, ws, (hipStream_t)stream, pan);
}

extern "C" int prism_w8a8_pc_packed_gemm(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                         const void* w_s, int ws_fp16, void* out, int64_t ldo, const int32_t* n_rows,
                                         int64_t M, int64_t N, int64_t K, int epi, int kernel, void* stream) {
    if (!a || !a_s || !qt || !w_s || !out || !n_rows) return PRISM_ERR_ARG;
    if (epi != 0 && epi != 1) return PRISM_ERR_ARG;
    if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 64 || ldo < N || M > (1 << 30) || N > (1 << 30) ||
        K > (1 << 17))
        return PRISM_ERR_SHAPE;
    if (!PRISM_ALIGNED(a, 16) || !PRISM_ALIGNED(qt, 16) || ldo % 4 || !PRISM_ALIGNED(out, epi ? 16 : 8))
        return PRISM_ERR_ALIGN;
    if (kernel < -1 || kernel > 1) return PRISM_ERR_ARG;
    if (kernel == -1) kernel = M <= 64 ? 1 : 0;
    if (kernel == 1 && M > 65535 * 64) return PRISM_ERR_SHAPE;           // grid rows: one per 64 activation rows
    if (M == 0) return PRISM_OK;
    return launch_w8a8_pc(kernel, true, a, a_s, as_sm, qt, w_s, ws_fp16 != 0, out, ldo, n_rows, (int)M, (int)N,
                          (int)K, epi, (hipStream_t)stream, 1, 0);
}

extern "C" int prism_w8a8_pc_packed_gemm_split(const int8_t* a, const int8_t* qt, int32_t* slots, int64_t slot_stride,
                                               int64_t lds, const int32_t* n_rows, int64_t M, int64_t N, int64_t K,
                                               int split, void* stream) {
    if (!a || !qt || !slots || !n_rows) return PRISM_ERR_ARG;
    if (split < 1 || split > 16) return PRISM_ERR_ARG;
    if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 64 || lds < N || M > 65535 * 64 || N > (1 << 30) ||
        K > (1 << 17) || K / 64 < split)
        return PRISM_ERR_SHAPE;
    if (split > 1 && slot_stride < M * lds) return PRISM_ERR_SHAPE;    // the slots must not overlap
    if (!PRISM_ALIGNED(a, 16) || !PRISM_ALIGNED(qt, 16) || !PRISM_ALIGNED(slots, 16) || lds % 4 || slot_stride % 4)
        return PRISM_ERR_ALIGN;
    if (M == 0) return PRISM_OK;
    return launch_w8a8_pc(1, true, a, nullptr, 0, qt, nullptr, false, slots, lds, n_rows, (int)M, (int)N, (int)K, 2,
                          (hipStream_t)stream, split, slot_stride);
}
