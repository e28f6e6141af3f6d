/*
 * prism_amd.h -- C ABI of the MI355X (gfx950) quantized linear-layer library (libprism_amd.so).
 *
 * Every entry point takes device pointers, plain sizes and a HIP stream (hipStream_t passed as void*; NULL is the
 * null stream), launches asynchronously on that stream, never synchronizes the host and never allocates.  It
 * returns PRISM_OK (0) or one of the error codes below; prism_error_string() names them.  Argument meaning,
 * layouts and the "live rows" convention follow StartLux-Prism's kernel ops (citations are relative to its
 * source tree):
 *   - n_rows: a DEVICE int32[1] holding the live row count, read inside the kernels so one captured graph serves
 *     every batch size; rows >= *n_rows of the outputs are left untouched (kernels/w8a8.py:44-46, 77-85).
 *   - operands are K-contiguous ("TN"): activations [M, K], weights [N, K] (csrc/w8a8_gemm.cu:3-6).
 *   - bf16 / fp16 values are passed as uint16_t bit patterns.
 */
#ifndef PRISM_AMD_H
#define PRISM_AMD_H

#include <stdint.h>

#if defined(__GNUC__)
#define PRISM_API __attribute__((visibility("default")))
#else
#define PRISM_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum {
    PRISM_OK = 0,
    PRISM_ERR_SHAPE = 1,       /* a size is not supported (e.g. K not a multiple of 32) */
    PRISM_ERR_ALIGN = 2,       /* a pointer or stride is not aligned as the kernel needs */
    PRISM_ERR_ARG = 3,         /* a bad argument value (epilogue, group size, null pointer) */
    PRISM_ERR_LAUNCH = 4,      /* the HIP runtime rejected the launch */
    PRISM_ERR_DEVICE = 5,      /* the current device is not a gfx950 (MI355X / MI350X) */
};

/* Version of this ABI (major * 100 + minor). */
PRISM_API int prism_version(void);

/* Static description of an error code. */
PRISM_API const char* prism_error_string(int code);

/*
 * Per-token int8 activation quantization.  Replaces kernels/quant.py:481-486 (rows_q8, mode 0) and its kernel
 * _rows_q8_kernel (kernels/quant.py:287-309).
 *   y = x * inv_s[k] (inv_s may be NULL: y = x); scale = max(max_k |y|, 1e-10) / 127 (IEEE division);
 *   q = rint(y / scale) (IEEE division, ties to even).
 * x bf16 [M, K] with row stride ldx (elements); q int8 [M, K] (row stride K); s fp32 [M].
 * Needs K % 8 == 0, ldx % 8 == 0, 16-byte aligned x and q, K <= 65536.
 */
PRISM_API int prism_quant_rows_i8(const uint16_t* x, int64_t ldx, const float* inv_s, int8_t* q, float* s,
                        const int32_t* n_rows, int64_t M, int64_t K, void* stream);

/*
 * Per-(row, group) int8 quantization.  Replaces kernels/w8a8.py:264-271 (quant_rows) and _quant_rows_kernel
 * (kernels/w8a8.py:101-112): per gk inputs scale = max(amax, 1e-10) / 127, q = rint(x / scale).
 * x bf16 [M, K] -> q int8 [M, K], s fp32 [M, K / gk].  gk in {32, 64, 128, 256, ...}, a multiple of 32 dividing K.
 */
PRISM_API int prism_quant_rows_groups(const uint16_t* x, int8_t* q, float* s, const int32_t* n_rows, int64_t M, int64_t K,
                            int64_t gk, void* stream);

/*
 * W4A8 activation producer.  Replaces kernels/quant.py:409-411 (rows_g) and _store_g (kernels/quant.py:314-330);
 * bit-identical to kernels/w4a8.py:144-155 (quantize_ref).
 *   per `group` inputs (256 as the reference, or K for one scale per token) a = max(amax, 1e-10) / 127,
 *   xq = rint(x / a); per 32 inputs the int32 sum S of xq stored as S & 63 and S >> 6.
 * x bf16 [M, K] (row stride ldx); xq int8 [M, K]; a fp32 [K / group, M]; xs int8 [K / 256, M, 16].
 * Needs K % 256 == 0, ldx % 8 == 0.
 */
PRISM_API int prism_quant_rows_g(const uint16_t* x, int64_t ldx, int8_t* xq, float* a, int8_t* xs, const int32_t* n_rows,
                       int64_t M, int64_t K, int64_t group, void* stream);

/*
 * W8A8 GEMM with per-group scales along K (Q8_0 when gk == 32; per-channel when gk == K).  Replaces
 * kernels/w8a8.py:183-231 (gemm, epilogues 0 and 1) with the arithmetic of _w8a8_kernel (kernels/w8a8.py:64-85);
 * the native schema it stands for is startlux_prism::w8a8_gemm (csrc/w8a8_gemm.cu:737-767, 794-797).
 *   per group g, in increasing g:  P = sum_{k in g} a[m,k] w[n,k]  (int32, exact)
 *                                  y = RN(y + RN(RN(float(P) * sa[m,g]) * sw[n,g]))
 *   epi 0: out bf16 [m, n] = RN_bf16(y);  epi 1: out fp32 [m, n] = RN(out[m, n] + y).
 * a int8 [M, K]; a_s fp32, element (m, g) at a_s[m * as_sm + g * as_sg] (as_sg = 0: one scale per token);
 * w int8 [N, K]; w_s [N, K / gk], fp16 bits (ws_fp16 = 1, Q8_0's own block scales) or fp32 (ws_fp16 = 0);
 * out row stride ldo (elements).  kernel: -1 picks by shape; 0 the tile kernel; 1 the decode kernel (gk == 32,
 * M <= 64; per channel any M).  Needs K % 32 == 0, gk % 32 == 0, K % gk == 0, N % 16 == 0, 16-byte aligned a and w.
 */
PRISM_API int prism_w8a8_gemm(const int8_t* a, const float* a_s, int64_t as_sm, int64_t as_sg, const int8_t* w,
                    const void* w_s, int ws_fp16, void* out, int64_t ldo, const int32_t* n_rows, int64_t M,
                    int64_t N, int64_t K, int64_t gk, int epi, int kernel, void* stream);

/*
 * Repack Q8_0 planes into the MFMA-native layout the packed kernels read (a load-time step, as the reference's
 * weight_from_q8 (kernels/w8a8.py:274-286) and repack (kernels/w4a8.py:70-94) are).  qs int8 [N, K], d fp16 [N, K/32]
 * -> qt int8 [N/16][K/64][64][16] (per 16-row tile and block pair a 1 KB chunk; lane slot l: row l % 16,
 * bytes 0..7 = k 8 (l/16) .. +8 of the pair's first block, bytes 8..15 the same of its second), dt fp16
 * [N/16][K/64][16][2].  Needs N % 16 == 0, K % 128 == 0 (the packed GEMM's rule).
 */
PRISM_API int prism_q8_0_pack(const int8_t* qs, const uint16_t* d, int8_t* qt, uint16_t* dt, int64_t N, int64_t K,
                              void* stream);

/*
 * The chunked layout for plain int8 weights w [N, K] (per-channel, gk = K): qt int8 [N/16][K/64][64][16], lane
 * slot l of chunk (nt, j) holding inputs 64 j + 16 (l / 16) .. + 15 of row 16 nt + l % 16 (no blocks to keep apart,
 * so a slot is one MFMA operand as it lies).  The load-time repack of the per-channel weights kernels/w8a8.py:274-286
 * produces.  Needs N % 16 == 0, K % 64 == 0.
 */
PRISM_API int prism_i8_pack(const int8_t* w, int8_t* qt, int64_t N, int64_t K, void* stream);

/*
 * Per-channel W8A8 GEMM (gk = K) on packed int8 weights (prism_i8_pack): the production projections of
 * kernels/w8a8.py:183-231 with gk == K (the CUDA w8a8_kernel, csrc/w8a8_gemm.cu:298-402, schema :794-797):
 * P = sum_k a w (int32, exact), y = RN(RN(float(P) a_s[m]) w_s[n]); epi 0 bf16(y), epi 1 out = RN(out + y).
 * a int8 [M, K]; a_s fp32, row m at a_s[m * as_sm]; w_s fp32 [N] (fp16 when ws_fp16); out row stride ldo (a
 * multiple of 4, out 8-byte aligned for bf16, 16 for fp32).  kernel: -1 picks by M; 0 the tile kernel; 1 the
 * split-K decode kernel (64 rows per workgroup, grid rows beyond: the choice for narrow projections).  Needs
 * N % 16 == 0, K % 64 == 0, K <= 131072 (int32 sums stay exact).
 * prism_w8a8_gemm with gk == K runs the same kernels on row-major weights.
 */
PRISM_API int prism_w8a8_pc_packed_gemm(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                        const void* w_s, int ws_fp16, void* out, int64_t ldo, const int32_t* n_rows,
                                        int64_t M, int64_t N, int64_t K, int epi, int kernel, void* stream);

/*
 * The deferred split-K form of the per-channel GEMM (the CUDA kernel's SPLIT_DEFER mode, csrc/w8a8_gemm.cu:266-271,
 * :433-440, behind kernels/w8a8.py:200-204): K in `split` parts of whole 64-input chunks (part z: chunks
 * floor(z KP / split) .. floor((z + 1) KP / split) - 1), part z's raw int32 sums sum_k a w written to
 * slots + z slot_stride, row m at m * lds.  No scales: the reader of the residual (prism_norm_quant_fold,
 * prism_fold_parts) adds the parts and applies epilogue 1.  Rows >= *n_rows are not written.  Needs N % 16 == 0,
 * K % 64 == 0, K / 64 >= split, 1 <= split <= 16, lds >= N and slot_stride >= M lds (multiples of 4).
 */
PRISM_API int prism_w8a8_pc_packed_gemm_split(const int8_t* a, const int8_t* qt, int32_t* slots, int64_t slot_stride,
                                              int64_t lds, const int32_t* n_rows, int64_t M, int64_t N, int64_t K,
                                              int split, void* stream);

/*
 * The per-channel GEMM on packed weights with the split decode (kernel 2), the CUDA kernel's split-K of the
 * per-channel product (csrc/w8a8_gemm.cu:624-671, :737-766, its workspace kernels/cuda_ext.py:138-143): K in three
 * parts, each part's int32 sums into a slot of `ws`, then a second kernel adds the slots (exact in any order) and
 * applies the epilogue; bits equal the unsplit kernels'.  Arguments as prism_w8a8_pc_packed_gemm, plus ws (256-byte
 * aligned, ws_bytes of it; no initial contents needed).  kernel: -1 the split where ws holds it and it measured faster
 * (16 - 64 rows at K >= 12288, 48 - 64 rows up to N = 5120, 65 - 384 rows at K >= 12288 up to N = 8192)
 * (prism_w8a8_pc_split_workspace_bytes), else as prism_w8a8_pc_packed_gemm; 0 / 1 as there; 2 the split (an error
 * when ws cannot hold it; from 48 rows on K >= 8192 it reads a panel copy of the activations placed after the slots
 * when ws holds both).  With kernel -1 (M > 64) or 0, M >= 1024, N >= 16384, M N >= 2^25 and ws of at least
 * ceil(M / 16) 16 K bytes, the tile kernel first copies the activations into ws as panels (each 16-row, 64-input
 * stage in one 1 KB piece, the order the kernel's lanes store to LDS): same bits, 8% faster at config 1's shape.
 * Calls that overlap on one GPU must not share ws.
 */
PRISM_API int prism_w8a8_pc_packed_gemm_ws(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                           const void* w_s, int ws_fp16, void* out, int64_t ldo,
                                           const int32_t* n_rows, int64_t M, int64_t N, int64_t K, int epi,
                                           int kernel, void* ws, int64_t ws_bytes, void* stream);
/* Bytes of ws the split decode needs at M rows (1..512) and N columns; 0 for shapes it does not take. */
PRISM_API int64_t prism_w8a8_pc_split_workspace_bytes(int64_t M, int64_t N);

/*
 * Q8_0 W8A8 GEMM (gk = 32, one activation scale per token) on packed weights: the arithmetic and bits of
 * prism_w8a8_gemm with gk = 32 (kernels/w8a8.py:64-85), the engine entry kernels/w8a8.py:183-231.
 * a int8 [M, K]; a_s fp32, row m at a_s[m * as_sm]; qt / dt from prism_q8_0_pack; out as prism_w8a8_gemm.
 * kernel: -1 picks by M; 0 the prefill tile kernel; 1 the decode kernels (M <= 64: M <= 16 folds through LDS,
 * larger M as kernel 2); 2 the register-fold kernel, one wave per 16 x 16 output tile (any M up to 65535 x 16: the
 * choice for narrow projections, whose few 128 x 128 tiles leave CUs idle); 3 the prefill tile kernel in a
 * reassociated order that is not the reference's: per block y = fma(float(P), sw, y), then y = RN(y a_s[m]) (the
 * per-token scale factored out of the block sum), half the epilogue's vector work.  Kernel 3's bf16 outputs equal
 * kernel 0's on all but a few in 10^4 outputs and are within 1 bf16 ulp plus 2 (K/32 + 2) 2^-24 sum |terms| of them.
 * 4 the balanced decode kernel (1 <= M <= 16): min(N/16, 256) workgroups take equal shares of the projection's
 * 1 KB weight chunks, so every CU streams the same bytes; a 16-row tile split between two workgroups hands its
 * running fp32 sums from the first to the second through `workspace` (bits identical to kernels 0-2).  kernel -1
 * takes kernel 4 when M <= 16 and a workspace is given.
 * workspace: device memory of at least prism_w8a8_q8_0_packed_workspace_bytes(N, K) bytes, zeroed once before its
 * first use (every launch leaves it zeroed), or NULL (kernel 4 is then unavailable).  Launches that share a
 * workspace must not run concurrently.  This argument is the reference schema's `workspace`
 * (csrc/w8a8_gemm.cu:794-797), which its engine allocates once per device (kernels/cuda_ext.py:138-143).
 * Bytes past the first 512 KB (the most any shape's handoff words take) are scratch for the tile kernels (0, 3):
 * from M >= 1024 on N >= 16384, where they hold ceil(M / 128) 128 K bytes, the activations are first copied there as
 * 128-row panels (each 128-input stage of a tile in one 16 KB piece); same bits, about 1% faster at config 1.
 * Needs K % 128 == 0.
 */
PRISM_API int prism_w8a8_q8_0_packed_gemm(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                          const uint16_t* dt, void* out, int64_t ldo, const int32_t* n_rows,
                                          int64_t M, int64_t N, int64_t K, int epi, int kernel, void* workspace,
                                          int64_t workspace_bytes, void* stream);

/* Workspace bytes prism_w8a8_q8_0_packed_gemm's kernel 4 needs for N x K weights (0 for an unsupported shape). */
PRISM_API int64_t prism_w8a8_q8_0_packed_workspace_bytes(int64_t N, int64_t K);

/*
 * prism_w8a8_q8_0_packed_gemm without a workspace argument and without any allocation: the same kernels and bits,
 * with kernel 4's handoff words in a 512 KB array of device memory that the library holds, one per GPU, for the life
 * of the process (zero when the library loads; found with hipGetSymbolAddress at the first call on a device, which,
 * outside graph capture, also clears it with a fill kernel on `stream` and waits for that clear; a first call under
 * capture records no clear into the graph).  This entry point has no counterpart in the reference; it is for callers that cannot allocate (code
 * under graph capture, tight serving loops, harnesses that forbid hipMalloc).  Calls on one GPU share the array:
 * calls that overlap in time on one GPU (two streams) race; calls in sequence are safe, since every launch leaves
 * the array zeroed (and a launch's handoff words carry its own tag, so a word another launch left is never taken).  Workspace needs above 512 KB are rejected with PRISM_ERR_SHAPE (none arises: the balanced
 * kernel runs at most 256 workgroups, 2 KB each).  PRISM_ERR_LAUNCH if the array's address cannot be found.
 */
PRISM_API int prism_w8a8_q8_0_packed_gemm_noalloc(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt,
                                                  const uint16_t* dt, void* out, int64_t ldo, const int32_t* n_rows,
                                                  int64_t M, int64_t N, int64_t K, int epi, int kernel, void* stream);

/*
 * Repack Q4_K weights into the MFMA-native layout the W4A8 kernels read: a byte permutation of the GGUF block_q4_K
 * bytes (the load-time step the reference's repack is: kernels/w4a8.py:70-94).  raw uint8 [N, K/256, 144] ->
 * qv uint8 [N/16][K/256][2][64][16] (per 16-row tile and super-block, lane slot l = row l % 16, q = l / 16; bytes
 * j of half h: pair p = 2 h + j / 8, t = j % 8, k0 = 64 p + 16 q + t, byte = v[k0] | v[k0 + 8] << 4), meta uint8
 * [N/16][K/256][16][16] (per row the block's first 16 bytes: d, dmin, 12 bytes of 6-bit scales and mins).
 * Needs N % 16 == 0, K % 256 == 0.
 */
PRISM_API int prism_q4k_pack(const uint8_t* raw, uint8_t* qv, uint8_t* meta, int64_t N, int64_t K, void* stream);

/*
 * W4A8 GEMM on packed Q4_K weights.  Replaces kernels/w4a8.py:353-366 (gemm, kind "q4k") and the native
 * startlux_prism::w4a8_gemm (csrc/w4a8_gemm.cu:887-961, schema :963-966); arithmetic of kernels/w4a8.py:14-22 /
 * gemm_ref (:177-199), per super-block b of 256 inputs in increasing b:
 *   acc  = sum_g sc[n,b,g] (xq . q)_g ;  mins = sum_g mn[n,b,g] S[m, 8b+g]          (int32, exact)
 *   t = RN(d[n,b] float(acc)); t = fma(-dmin[n,b], float(mins), t); y = fma(a[b,m], t, y)
 *   epi 0: bf16(y); epi 1: out = RN(out + y).
 * xq int8 [M, K]; a fp32, element (b, m) at a[b * a_sb + m] (a_sb = 0: one scale per token); xs int8 [K/256, M, 16]
 * (per super-block eight S & 63 then eight S >> 6); qv / meta from prism_q4k_pack; out row stride ldo.
 * kernel: -1 picks by M (2 up to 4 rows where it applies and N / 16 < 512, else 1 up to 16 rows, beyond 16 rows 0);
 * 0 the prefill tile kernel;
 * 1 the per-tile decode kernel (M <= 16; the tile kernel when its per-super-block terms, K/256 x M x 64 bytes, exceed
 * the 160 KB of LDS); 2 the balanced-grid decode kernel (M <= 16 with M (K + 32) + K M / 8 bytes of activation image
 * within LDS; equal shares of the weights per CU, running sums handed between workgroups through `workspace`).
 * workspace: for kernel 2, a zero-initialised device buffer of at least prism_w8a8_q8_0_packed_workspace_bytes(N, K)
 * bytes (the same size rule as the Q8_0 one), left zeroed by every call; may be null for the other kernels.  Calls
 * sharing one workspace must not overlap in time.  Needs K % 256 == 0, N % 16 == 0.
 */
PRISM_API int prism_w4a8_q4k_gemm(const int8_t* xq, const float* a, int64_t a_sb, const int8_t* xs, const uint8_t* qv,
                                  const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int64_t M,
                                  int64_t N, int64_t K, int epi, int kernel, void* workspace, int64_t workspace_bytes,
                                  void* stream);

/*
 * Repack Q6_K weights for the W4A8 kernels (the load-time step of kernels/w4a8.py:82-90, repack "q6k", which keeps
 * the values as int8 q - 32).  raw uint8 [N, K/256, 210] (GGUF block_q6_K: ql[128], qh[64], 16 int8 scales, fp16 d)
 * -> qv int8 [N/16][K/256][4][64][16] (per 16-row tile and super-block, lane slot l = row l % 16, q = l / 16; bytes
 * 8 u + t of chunk j: window w = 2 j + u of 32 inputs, input 32 w + 8 q + t) and meta uint8 [N/16][K/256][288]
 * (the 16 rows' 16 scales, then their fp16 d).  Needs N % 16 == 0, K % 256 == 0; raw needs no alignment.
 */
PRISM_API int prism_q6k_pack(const uint8_t* raw, uint8_t* qv, uint8_t* meta, int64_t N, int64_t K, void* stream);

/*
 * W4A8 GEMM on packed Q6_K weights.  Replaces kernels/w4a8.py:353-366 (gemm, kind "q6k") and the Q6_K branch of
 * startlux_prism::w4a8_gemm (csrc/w4a8_gemm.cu); arithmetic of kernels/w4a8.py:19-20 / gemm_ref (:193-197), per
 * super-block b in increasing b: acc = sum_h sc[n,b,h] (xq . q)_h over its 16 sub-blocks of 16 (int32, exact),
 * y = fma(a[b,m], RN(d[n,b] float(acc)), y); epi 0: bf16(y); epi 1: out = RN(out + y).  xq, a, a_sb, out, ldo,
 * n_rows and kernel as prism_w4a8_q4k_gemm (Q6_K has no mins: no activation sums), plus kernel 2: the stream decode
 * kernel (M <= 16), which the MI355X dispatch table picks for the shapes where it measured faster.
 */
PRISM_API int prism_w4a8_q6k_gemm(const int8_t* xq, const float* a, int64_t a_sb, const uint8_t* qv,
                                  const uint8_t* meta, void* out, int64_t ldo, const int32_t* n_rows, int64_t M,
                                  int64_t N, int64_t K, int epi, int kernel, void* stream);

/* -------------------------------------------------------------------------------------- fused producers */
/*
 * RMSNorm producer: y = RN(RN(h * r) * w), r = RN(1 / RN(sqrt(RN(RN(ss / HID) + eps)))), ss the sum of RN(h * h) in
 * a fixed order (a 256-thread workgroup's: each thread its inputs 8 (t + 256 c) + j in increasing order, the 64 lanes
 * of a wave by halving, the four waves left to right).  Replaces kernels/quant.py:418-431 (norm_q8, back 0: q int8
 * [M, HID] and s fp32 [M]) and :395-397 (norm_g, back 1: q, s [HID/256, M], xs [HID/256, M, 16] as
 * prism_quant_rows_g; back 2: one scale per row, s [M]).  h fp32 rows of stride ldh; output row i reads input row
 * rows[i] when rows is not null.  Rows >= *n_rows are not written.  Needs HID % 8 == 0 (% 256 for backs 1, 2).
 */
PRISM_API int prism_norm_quant(const float* h, int64_t ldh, const float* w, const int32_t* rows, int8_t* q, float* s,
                               int8_t* xs, const int32_t* n_rows, int64_t M, int64_t HID, float eps, int back,
                               void* stream);

/*
 * prism_norm_quant that first finishes a residual add deferred by prism_w8a8_pc_packed_gemm_split (norm_q8 with
 * `pending`, kernels/quant.py:418-431 and _fold_parts :129-141): per row r and column c, tot = the sum of the np
 * slots' parts[p part_stride + r ldp + c] (int32, exact), h = RN(h + RN(RN(float(tot) psa[r psa_sm]) psw[c])) (psw
 * fp32 [HID], fp16 when psw16), stored back to h; then the norm of the updated row.  psa may be s itself (a row reads
 * its scale before writing its own).  No row gather.  Needs what prism_norm_quant needs, ldp >= HID and
 * part_stride >= M ldp (multiples of 4), 1 <= np <= 64.
 */
PRISM_API int prism_norm_quant_fold(float* h, int64_t ldh, const float* w, int8_t* q, float* s, int8_t* xs,
                                    const int32_t* n_rows, int64_t M, int64_t HID, float eps, int back,
                                    const int32_t* parts, int64_t part_stride, int64_t ldp, int np, const float* psa,
                                    int64_t psa_sm, const void* psw, int psw16, void* stream);

/*
 * The deferred residual add alone, when no norm follows (kernels/quant.py:435-457 fold): h updated as in
 * prism_norm_quant_fold for rows < *n_rows.  Needs HID % 8 == 0, ldh % 4 == 0, M <= 65535.
 */
PRISM_API int prism_fold_parts(float* h, int64_t ldh, const int32_t* parts, int64_t part_stride, int64_t ldp, int np,
                               const float* psa, int64_t psa_sm, const void* psw, int psw16, const int32_t* n_rows,
                               int64_t M, int64_t HID, void* stream);

/*
 * SwiGLU producer: y = RN(RN(silu(g) * u) * inv_s) with silu(g) = RN(g / RN(1 + exp(-g))) (exp: Cody-Waite
 * reduction and a degree-7 Taylor series in fp32 fmas, this library's own).  gu [M, 2 FF] bf16 (fp32 when gu_f32),
 * row stride ldg, gate = columns 0 .. FF-1, up = FF .. 2 FF - 1; inv_s fp32 [FF] or null.  Replaces
 * kernels/quant.py:472-478 (swiglu_q8, back 0) and :403-406 (swiglu_g, back 1; back 2 one scale per row), outputs as
 * prism_norm_quant.  Needs FF % 8 == 0 (% 256 for backs 1, 2).
 */
PRISM_API int prism_swiglu_quant(const void* gu, int gu_f32, int64_t ldg, const float* inv_s, int8_t* q, float* s,
                                 int8_t* xs, const int32_t* n_rows, int64_t M, int64_t FF, int back, void* stream);

/*
 * Gated RMSNorm producer of the linear-attention output projection: per head of D values,
 * r = RN(1 / RN(sqrt(RN(RN(ss / D) + eps)))) with ss the head's sum of squares in a fixed order (8-value chunks in
 * increasing index, then the D / 8 chunk sums combined by halving), y = RN(RN(RN(o * r) * w[d]) * silu(z)), then
 * RN(y * inv_s) when inv_s is not null; quantized as prism_norm_quant.  o fp32 [M, HV D] (row stride ldo); z the
 * row's HV D gate values, bf16 (fp32 when z_f32) with row stride ldz (the caller passes the projection plus its
 * column offset); w fp32 [D]; inv_s fp32 [HV D] or null.  Replaces kernels/quant.py:460-469 (gated_norm_q8, back 0)
 * and :399-401 (gated_norm_g, back 1; back 2 one scale per row).  Needs D a power of two in 8 .. 512, HV D <= 32768
 * (% 256 for backs 1, 2).
 */
PRISM_API int prism_gated_norm_quant(const float* o, int64_t ldo, const void* z, int z_f32, int64_t ldz,
                                     const float* w, const float* inv_s, int8_t* q, float* s, int8_t* xs,
                                     const int32_t* n_rows, int64_t M, int64_t HV, int64_t D, float eps, int back,
                                     void* stream);

/* ------------------------------------------------------------------------------------------------ MXFP4 */
/* Element formats of MX operands (the MFMA format codes): e4m3 (OCP float8_e4m3fn) and e2m1 (fp4).
 * PRISM_MX_E4M3_PANELS: e4m3 activations in the panel layout (no counterpart in the reference, whose activations
 * are e2m1 row-major; the e4m3 activations are the C4 workload's): 16-row blocks of K / 128 chunks of 2 KB, byte
 * 1024 h + 16 (16 p + r) + i of chunk st of block b holding row 16 b + r, input 128 st + 64 h + 16 p + i.  The
 * buffer holds ceil(M / 16) blocks (16 K bytes each); the prefill tile kernel reads each 16-row step in one piece. */
enum { PRISM_MX_E4M3 = 0, PRISM_MX_E4M3_PANELS = 1, PRISM_MX_E2M1 = 4 };

/*
 * Quantize fp32 weights w [N, K] (row stride ldw) to MXFP4 in the device layout the GEMM reads: 32-input blocks,
 * e2m1 codes, one e8m0 scale each.  Replaces kernels/mxfp4.py:57-86 (pack; CPU there):
 *   mode 0 "max": e = ceil(log2(amax / 6)) clipped to +-127, codes by strict thresholds (midpoints toward zero);
 *   mode 1 "mse": of e and e - 1 the one with the smaller squared error (float32, numpy's summation order);
 *   mode 2 "ocp": e = floor(log2(amax)) - 2, codes nearest-even saturating at 6 (tests/quant_sim.py:66-72, the C4
 *                 weights).
 * Output q uint8 [N/16][K/128][64][16] (tile t, step s, lane 16 p + i: row 16 t + i, inputs 128 s + 32 p .. + 31,
 * low nibble first) and s uint8 [N/16][K/128][64] (e + 127).  Needs N % 16 == 0, K % 128 == 0.
 */
PRISM_API int prism_mxfp4_pack(const float* w, int64_t ldw, uint8_t* q, uint8_t* s, int64_t N, int64_t K, int mode,
                               void* stream);

/* Row-major MX4 (q [N, K/2], s [N, K/32]: kernels/mxfp4.py:25-30, the layout pack() and the engine's side files
 * hold) -> the device layout of prism_mxfp4_pack.  A byte permutation. */
PRISM_API int prism_mxfp4_repack(const uint8_t* q_rows, const uint8_t* s_rows, uint8_t* q, uint8_t* s, int64_t N,
                                 int64_t K, void* stream);

/*
 * Per-32 MX activation quantization of x [M, K] (bf16 bits, or fp32 when x_f32; row stride ldx), optionally times
 * inv [K] first.  fmt PRISM_MX_E2M1: replaces kernels/mxfp4.py:181-185 (quantize_act) and :173-178
 * (quantize_act_scaled): e = clip(ceil(log2(max(amax, 1e-30) / 6)), +-127), q uint8 [M, K/2].  fmt PRISM_MX_E4M3:
 * tests/quant_sim.py:75-81 (mxfp8, the C4 activations): e = floor(log2(max(amax, 1e-30))) - 8,
 * q = e4m3(clamp(x / 2^e, +-448)) nearest even, q uint8 [M, K]; fmt PRISM_MX_E4M3_PANELS: the same codes in the
 * panel layout (K % 128 == 0, q of ceil(M / 16) 16 K bytes).  s uint8 [M, K/32] = e + 127 (row-major always).
 * Rows >= *n_rows (when n_rows is not null) are not written.
 */
PRISM_API int prism_mxfp4_quant_act(const void* x, int x_f32, int64_t ldx, const float* inv, uint8_t* q, uint8_t* s,
                                    const int32_t* n_rows, int64_t M, int64_t K, int fmt, void* stream);

/*
 * MXFP4 GEMM out[m, n] = sum_k A[m, k] W[n, k] with fp32 accumulation.  Replaces kernels/mxfp4.py:292-317 (gemm,
 * the Triton _gemm_kernel :260-289 on tl.dot_scaled) and the C ABI mxfp4_gemm of csrc/mxfp4_gemm.cu:96.
 * aq / as: activations in fmt a_fmt (e4m3 [M, K] or e2m1 [M, K/2]) with e8m0 [M, K/32]; wq / ws: weights from
 * prism_mxfp4_pack / _repack.  epi 0: bf16 out; epi 1: out (fp32) = out + y.  Output row stride ldo.  n_rows may be
 * null (all M rows live).  Every kernel sums in the same order (128-input MFMA steps chained within 1024-input
 * segments, segment sums added left to right), so results do not depend on M or on the kernel.
 * kernel: -1 picks by M; 0 the tile kernel; 1 the decode kernel (M <= 64); 2 the split decode, which needs the
 * workspace of prism_mxfp4_gemm_ws (here: PRISM_ERR_ARG).  Needs N % 16 == 0, K % 128 == 0.
 * a_fmt PRISM_MX_E4M3_PANELS (activations from prism_mxfp4_quant_act in that format): the tile kernel only (kernel
 * -1 or 0; N K / 2 < 2^31), bits equal to the row-major e4m3 call's.
 */
PRISM_API int prism_mxfp4_gemm(const uint8_t* aq, const uint8_t* as, int a_fmt, const uint8_t* wq, const uint8_t* ws,
                               void* out, int64_t ldo, const int32_t* n_rows, int64_t M, int64_t N, int64_t K,
                               int epi, int kernel, void* stream);
/*
 * prism_mxfp4_gemm with a workspace (the same arguments and bits; no counterpart in the reference, whose gemm is one
 * Triton launch): kernel 2, the split decode (M <= 16, a_fmt PRISM_MX_E4M3), spreads the projection's (1024-input
 * segment, 16-row weight tile) units over up to 256 workgroups in segment-major order, so each workgroup copies only
 * one or two segments of the activation rows; the segment sums go to `work` and a second launch on the stream adds
 * each tile's sums left to right, as every kernel does.  kernel -1 takes it where it measured faster than the staged
 * decode and `work` is given.  work: device memory of at least prism_mxfp4_split_workspace_bytes(N, K) bytes,
 * 16-byte aligned, rewritten by every launch, or NULL.  Calls that overlap on one GPU must not share work.
 */
PRISM_API int prism_mxfp4_gemm_ws(const uint8_t* aq, const uint8_t* as, int a_fmt, const uint8_t* wq,
                                  const uint8_t* ws, void* out, int64_t ldo, const int32_t* n_rows, int64_t M,
                                  int64_t N, int64_t K, int epi, int kernel, void* work, int64_t work_bytes,
                                  void* stream);
/* Bytes of work the split decode needs for an N x K projection; 0 for shapes it does not take. */
PRISM_API int64_t prism_mxfp4_split_workspace_bytes(int64_t N, int64_t K);

/*
 * Peak probes (measurement tooling: the reference's bench/csrc/mma_peak.cu:14-70 and bench/csrc/l2_bw.cu:8 for
 * this GPU, no counterpart on the engine's path).  prism_probe_mfma launches `workgroups` workgroups of 4 waves,
 * each wave issuing `iters` x 4 independent MFMAs of one kind on register operands: 0 int8
 * (v_mfma_i32_32x32x32_i8), 1 fp8 e4m3 and 2 fp4 e2m1 (v_mfma_scale_f32_16x16x128_f8f6f4, unit scales), 3 bf16
 * (v_mfma_f32_32x32x16_bf16), 4 int8 with pseudo-random operands changing from one MFMA to the next (what a GEMM's
 * operands draw under the power limit), 5 e2m1 x e4m3 likewise; prism_probe_mfma_ops gives one instruction's operations (2 M N K).  prism_probe_read
 * streams `bytes` of `buf` (16-byte aligned) with `workgroups` workgroups of 512 threads, each a contiguous slice, 8
 * nontemporal 16-byte loads per lane in flight.  `sink` (device, >= workgroups elements) is written only on a value
 * the probes never produce.
 */
PRISM_API int prism_probe_mfma(int kind, int64_t workgroups, int64_t iters, float* sink, void* stream);
PRISM_API int64_t prism_probe_mfma_ops(int kind);
PRISM_API int prism_probe_read(const void* buf, int64_t bytes, int64_t workgroups, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PRISM_AMD_H */
