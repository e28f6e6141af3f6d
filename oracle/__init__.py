"""CPU oracle for StartLux-Prism's quantized linear-layer hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the
checker (or the timed CPU baseline), never as the thing measured or shipped.  The arithmetic lives in
prism_oracle.c (built by oracle/Makefile into oracle/_build/liboracle.so); this module wraps it with numpy.

Pinning (each function is checked by tests/test_oracle.py against something other than its own formula):
  fp16/bf16 conversions      numpy's float16 / a bit-level bf16 rounding of float64, exhaustive over patterns
  q8_0_quantize              numpy dequantisation round trip (|w - q d| <= d / 2), absmax element -> +-127,
                             the torch restatement in the product package (gguf_formats.as_q8) bit for bit
  quant_rows_i8 / _groups    special cases (zero row -> scale 1e-10/127, absmax -> +-127), numpy IEEE division
  w8a8_gemm                  int32 block sums vs brute-force int64 (numpy), fp32 result vs float64 within the
                             rounding bound, gk == K reducing to the per-channel formula, epi 1 = out + epi 0 value
  w8a8_gemm_reassoc          (this build's opt-in order, not the reference's) one element replayed with the pinned
                             fmaf, the float64 rounding bound, epilogues as w8a8_gemm's, and agreement with
                             w8a8_gemm's bf16 bits on all but a few outputs in 10^4
  fold_parts                 one slot holding numpy's int64 sums gives w8a8_gemm's gk = K, epi 1 residual bit for
                             bit; any split of those sums into slots gives the same bits
  q4k_quantize / dequant     an independent numpy decoder of the GGUF block_q4_K layout (ggml get_scale_min_k4)
  q4k_repack                 the W4 nibble order re-derived from the dequantised values
  quant_rows_g               per-32 sums vs numpy, split-sum reconstruction, scale special cases
  w4a8_gemm                  int32 super-block sums vs brute force, fmaf vs exact rational arithmetic
                             (fractions.Fraction), fp32 result vs float64 within the rounding bound
  mx_pack (max, mse)         the reference's exact-grid vector survives (tests/test_mxfp4.py:32-37), every code is
                             a nearest e2m1 value under the stated tie rule (brute force over the grid), the
                             scale is the smallest power of two putting amax/6 within the grid, "mse" never has a
                             larger squared error than "max"
  mx_pack (ocp), quant_act   scale exponents from numpy's log2 on the same values; e4m3 codes against torch's
                             float8_e4m3fn conversion over every representable input class
  mx_gemm                    float64 dot products against numpy's matmul of independently decoded operands
  expf                       within 2 ulp of float64 exp over the whole range, exact at 0, inf / 0 at the ends
  norm_quant, swiglu_quant   y within a few ulp of the float64 formulas; the quantized outputs equal the row / group
                             quantizers (quant_rows_i8, quant_rows_g) applied to the oracle's own y; the fixed-order
                             sum of squares against math.fsum within its error bound and against a hand-built case
                             whose result depends on the order
  Parity unpinned against the reference's bits for these producers: the reference computes rsqrt, exp and '/' with
  NVIDIA's approximate instructions in Triton's reduction order, so no specification of its bits exists.
Parity unpinned: none of the above is checked against the reference's own numbers, because the reference holds
no numeric fixtures for this path (its GEMM tests compare GPU kernels with each other on CUDA-seeded inputs).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

_i64 = ctypes.c_int64
_p = ctypes.c_void_p


def build():
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_bf16_to_float": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_float_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_q8_0_quantize": (None, [_p, _i64, _i64, _p, _p, ctypes.c_int]),
            "orc_quant_rows_i8": (None, [_p, _i64, _p, _i64, _i64, _i64, _p, _p, ctypes.c_int]),
            "orc_quant_rows_groups": (None, [_p, _i64, _i64, _i64, _i64, _p, _p, ctypes.c_int]),
            "orc_w8a8_block_sums": (None, [_p, _p, _i64, _i64, _i64, _i64, _p]),
            "orc_w8a8_gemm": (None, [_p, _p, _i64, _i64, _p, _p, ctypes.c_int, _i64, _i64, _i64, _i64,
                                     ctypes.c_int, _p, _i64, _i64, ctypes.c_int]),
            "orc_w8a8_gemm_reassoc": (None, [_p, _p, _i64, _p, _p, ctypes.c_int, _i64, _i64, _i64, ctypes.c_int, _p,
                                             _i64, _i64, ctypes.c_int]),
            "orc_fold_parts": (None, [_p, _i64, _p, _i64, _i64, ctypes.c_int, _p, _i64, _p, ctypes.c_int, _i64,
                                      _i64]),
            "orc_q4k_quantize": (None, [_p, _i64, _i64, _p, ctypes.c_int]),
            "orc_q4k_dequant": (None, [_p, _i64, _i64, _p]),
            "orc_q4k_repack": (None, [_p, _i64, _i64, _p, _p, _p, _p, _p]),
            "orc_quant_rows_g": (None, [_p, _i64, _i64, _i64, _i64, _p, _p, _p, ctypes.c_int]),
            "orc_w4a8_gemm": (None, [_p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, ctypes.c_int, _p,
                                     _i64, _i64, _p, _p, ctypes.c_int]),
            "orc_fmaf": (ctypes.c_double, [ctypes.c_float, ctypes.c_float, ctypes.c_float]),
            "orc_expf": (ctypes.c_float, [ctypes.c_float]),
            "orc_sumsq_fixed": (ctypes.c_float, [_p, _i64]),
            "orc_norm_quant": (None, [_p, _i64, _p, _p, _i64, ctypes.c_float, ctypes.c_int, _i64, _p, _p, _p,
                                      ctypes.c_int]),
            "orc_swiglu_quant": (None, [_p, _i64, _p, _i64, ctypes.c_int, _i64, _p, _p, _p, ctypes.c_int]),
            "orc_head_sumsq": (ctypes.c_float, [_p, _i64]),
            "orc_q6k_quantize": (None, [_p, _i64, _i64, _p, ctypes.c_int]),
            "orc_q6k_dequant": (None, [_p, _i64, _i64, _p]),
            "orc_q6k_repack": (None, [_p, _i64, _i64, _p, _p, _p]),
            "orc_w4a8_gemm_q6k": (None, [_p, _p, _i64, _p, _p, _p, _i64, _i64, _i64, ctypes.c_int, _p, _i64, _i64,
                                         _p, ctypes.c_int]),
            "orc_gated_norm_quant": (None, [_p, _p, _i64, _p, _p, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int,
                                            _i64, _p, _p, _p, ctypes.c_int]),
            "orc_e2m1_value": (ctypes.c_float, [ctypes.c_int]),
            "orc_e4m3_value": (ctypes.c_float, [ctypes.c_int]),
            "orc_e4m3_code": (ctypes.c_int, [ctypes.c_float]),
            "orc_mx_pack": (None, [_p, _i64, _i64, ctypes.c_int, _p, _p, ctypes.c_int]),
            "orc_mx_quant_act": (None, [_p, _p, _i64, _i64, ctypes.c_int, _i64, _p, _p, ctypes.c_int]),
            "orc_mx_gemm": (None, [_p, _p, ctypes.c_int, _p, _p, _i64, _i64, _i64, _p, _p, ctypes.c_int]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def _ptr(x):
    return None if x is None else x.ctypes.data


def _c(x, dtype):
    assert x.dtype == dtype, (x.dtype, dtype)
    assert x.flags["C_CONTIGUOUS"]
    return x


# ------------------------------------------------------------------------------------------------ formats
def bf16_bits(x):
    """fp32 array -> bf16 bit patterns (uint16), round to nearest even (the C conversion, vectorised in numpy)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_c(v):
    return lib().orc_float_to_bf16(float(v))


def f32_to_half_c(v):
    return lib().orc_float_to_half(float(v))


def half_to_f32_c(h):
    return lib().orc_half_to_float(int(h))


def fmaf(a, b, c):
    return lib().orc_fmaf(float(a), float(b), float(c))


# ------------------------------------------------------------------------------------------------ Q8_0 / W8A8
def q8_0_quantize(w, nthreads=0):
    """fp32 [N, K] -> (qs int8 [N, K], d fp16-bits uint16 [N, K/32]) (gguf_weights.py:121-133)."""
    w = _c(np.ascontiguousarray(w, np.float32), np.float32)
    N, K = w.shape
    qs = np.empty((N, K), np.int8)
    d = np.empty((N, K // 32), np.uint16)
    lib().orc_q8_0_quantize(_ptr(w), N, K, _ptr(qs), _ptr(d), nthreads)
    return qs, d


def quant_rows_i8(x_bf16, inv_s=None, live=None, nthreads=0):
    """bf16 bits uint16 [M, K] -> (q int8 [M, K], s fp32 [M]) (kernels/quant.py:287-309)."""
    x = _c(np.ascontiguousarray(x_bf16), np.uint16)
    M, K = x.shape
    live = M if live is None else live
    q = np.zeros((M, K), np.int8)
    s = np.zeros(M, np.float32)
    inv = None if inv_s is None else _c(np.ascontiguousarray(inv_s, np.float32), np.float32)
    lib().orc_quant_rows_i8(_ptr(x), K, _ptr(inv), M, K, live, _ptr(q), _ptr(s), nthreads)
    return q, s


def quant_rows_groups(x_bf16, gk, live=None, nthreads=0):
    """bf16 bits [M, K] -> (q int8 [M, K], s fp32 [M, K/gk]) (kernels/w8a8.py:101-112)."""
    x = _c(np.ascontiguousarray(x_bf16), np.uint16)
    M, K = x.shape
    live = M if live is None else live
    q = np.zeros((M, K), np.int8)
    s = np.zeros((M, K // gk), np.float32)
    lib().orc_quant_rows_groups(_ptr(x), M, K, gk, live, _ptr(q), _ptr(s), nthreads)
    return q, s


def w8a8_block_sums(a, w, gk):
    a = _c(np.ascontiguousarray(a), np.int8)
    w = _c(np.ascontiguousarray(w), np.int8)
    M, K = a.shape
    N = w.shape[0]
    P = np.empty((M, N, K // gk), np.int32)
    lib().orc_w8a8_block_sums(_ptr(a), _ptr(w), M, N, K, gk, _ptr(P))
    return P


def w8a8_gemm(a, a_s, w, w_s, gk, epi=0, out=None, live=None, nthreads=0):
    """(kernels/w8a8.py:64-85).  a int8 [M, K]; a_s fp32 [M] (per token) or [M, K/gk]; w int8 [N, K];
    w_s fp16 bits uint16 or fp32 [N, K/gk].  epi 0 -> bf16 bits uint16 [M, N] (rows >= live zero unless `out`
    given); epi 1 -> out fp32 [M, N] updated in place (out = out + y)."""
    a = _c(np.ascontiguousarray(a), np.int8)
    w = _c(np.ascontiguousarray(w), np.int8)
    M, K = a.shape
    N = w.shape[0]
    G = K // gk
    a_s = np.ascontiguousarray(a_s, np.float32)
    as_sm, as_sg = (1, 0) if a_s.ndim == 1 else (G, 1)
    ws16 = w_s.dtype == np.uint16
    w_s = np.ascontiguousarray(w_s)
    assert w_s.shape == (N, G)
    live = M if live is None else live
    if out is None:
        out = np.zeros((M, N), np.uint16 if epi == 0 else np.float32)
    assert out.dtype == (np.uint16 if epi == 0 else np.float32) and out.flags["C_CONTIGUOUS"]
    lib().orc_w8a8_gemm(_ptr(a), _ptr(a_s), as_sm, as_sg, _ptr(w), _ptr(w_s), int(ws16), M, N, K, gk, epi,
                        _ptr(out), out.shape[1], live, nthreads)
    return out


def w8a8_gemm_reassoc(a, a_s, w, w_s, gk, epi=0, out=None, live=None, nthreads=0):
    """w8a8_gemm's reassociated order (one activation scale per token, a_s fp32 [M]): per block y = fmaf(float(P),
    sw, y), then y = RN(y a_s[m]); not the reference's rounding sequence (the "reassoc" kernel's arithmetic)."""
    a = _c(np.ascontiguousarray(a), np.int8)
    w = _c(np.ascontiguousarray(w), np.int8)
    M, K = a.shape
    N = w.shape[0]
    a_s = _c(np.ascontiguousarray(a_s, np.float32).reshape(-1), np.float32)
    assert a_s.shape[0] >= M
    ws16 = w_s.dtype == np.uint16
    w_s = np.ascontiguousarray(w_s)
    assert w_s.shape == (N, K // gk)
    live = M if live is None else live
    if out is None:
        out = np.zeros((M, N), np.uint16 if epi == 0 else np.float32)
    assert out.dtype == (np.uint16 if epi == 0 else np.float32) and out.flags["C_CONTIGUOUS"]
    lib().orc_w8a8_gemm_reassoc(_ptr(a), _ptr(a_s), 1, _ptr(w), _ptr(w_s), int(ws16), N, K, gk, epi, _ptr(out),
                                out.shape[1], live, nthreads)
    return out


def fold_parts(h, parts, psa, psw, live=None):
    """(kernels/quant.py:129-141) h fp32 [M, HID] updated in place and returned: the deferred residual add of the
    int32 slots parts [np, M, HID] with activation scales psa fp32 [M] and weight scales psw fp32 / fp16 bits
    uint16 [HID]."""
    assert h.dtype == np.float32 and h.flags["C_CONTIGUOUS"]
    parts = np.ascontiguousarray(parts, np.int32)
    psa = np.ascontiguousarray(psa, np.float32).reshape(-1)
    psw16 = psw.dtype == np.uint16
    psw = np.ascontiguousarray(psw).reshape(-1)
    S, M, HID = parts.shape
    lib().orc_fold_parts(_ptr(h), h.shape[1], _ptr(parts), M * HID, HID, S, _ptr(psa), 1, _ptr(psw), int(psw16),
                         M if live is None else live, HID)
    return h


# ------------------------------------------------------------------------------------------------ Q4_K / W4A8
def q4k_quantize(w, nthreads=0):
    """fp32 [N, K] -> GGUF block_q4_K bytes uint8 [N, K/256, 144] (this build's own quantizer)."""
    w = _c(np.ascontiguousarray(w, np.float32), np.float32)
    N, K = w.shape
    out = np.empty((N, K // 256, 144), np.uint8)
    lib().orc_q4k_quantize(_ptr(w), N, K, _ptr(out), nthreads)
    return out


def q4k_dequant(blocks):
    blocks = _c(np.ascontiguousarray(blocks), np.uint8)
    N, NB = blocks.shape[:2]
    w = np.empty((N, NB * 256), np.float32)
    lib().orc_q4k_dequant(_ptr(blocks), N, NB * 256, _ptr(w))
    return w


def q4k_repack(blocks):
    """-> dict(q uint8 [N, K/2], sc uint8 [K/256, N, 8], mn, d fp32 [K/256, N], dm) (kernels/w4a8.py:70-81)."""
    blocks = _c(np.ascontiguousarray(blocks), np.uint8)
    N, NB = blocks.shape[:2]
    K = NB * 256
    r = dict(q=np.empty((N, K // 2), np.uint8), sc=np.empty((NB, N, 8), np.uint8), mn=np.empty((NB, N, 8), np.uint8),
             d=np.empty((NB, N), np.float32), dm=np.empty((NB, N), np.float32))
    lib().orc_q4k_repack(_ptr(blocks), N, K, _ptr(r["q"]), _ptr(r["sc"]), _ptr(r["mn"]), _ptr(r["d"]), _ptr(r["dm"]))
    return r


def quant_rows_g(x, group=256, live=None, nthreads=0):
    """fp32 [M, K] -> (xq int8 [M, K], a fp32 [K/group, M], xs int8 [K/256, M, 16]) (kernels/w4a8.py:144-155)."""
    x = _c(np.ascontiguousarray(x, np.float32), np.float32)
    M, K = x.shape
    live = M if live is None else live
    xq = np.zeros((M, K), np.int8)
    a = np.zeros((K // group, M), np.float32)
    xs = np.zeros((K // 256, M, 16), np.int8)
    lib().orc_quant_rows_g(_ptr(x), M, K, group, live, _ptr(xq), _ptr(a), _ptr(xs), nthreads)
    return xq, a, xs


def group_sums(xs):
    """xs int8 [K/256, M, 16] -> int32 [M, K/32] (kernels/w4a8.py:158-161)."""
    p = xs.transpose(1, 0, 2).reshape(xs.shape[1], -1, 2, 8).astype(np.int32)
    return (p[:, :, 0] + 64 * p[:, :, 1]).reshape(xs.shape[1], -1)


def w4a8_gemm(xq, a, xs, w4, epi=0, out=None, live=None, sums=False, nthreads=0):
    """(kernels/w4a8.py:177-199).  a fp32 [K/256, M] or [M] (one scale per token).  Returns bf16 bits [M, N]
    (epi 0) or the updated fp32 out (epi 1); with sums=True also (acc, mins) int32 [M, N, K/256]."""
    xq = _c(np.ascontiguousarray(xq), np.int8)
    M, K = xq.shape
    N = w4["q"].shape[0]
    a = np.ascontiguousarray(a, np.float32)
    a_sb = 0 if a.ndim == 1 else M
    xs = _c(np.ascontiguousarray(xs), np.int8)
    live = M if live is None else live
    if out is None:
        out = np.zeros((M, N), np.uint16 if epi == 0 else np.float32)
    acc = mins = None
    if sums:
        acc = np.zeros((M, N, K // 256), np.int32)
        mins = np.zeros((M, N, K // 256), np.int32)
    lib().orc_w4a8_gemm(_ptr(xq), _ptr(a), a_sb, _ptr(xs), _ptr(w4["q"]), _ptr(w4["sc"]), _ptr(w4["mn"]),
                        _ptr(w4["d"]), _ptr(w4["dm"]), M, N, K, epi, _ptr(out), out.shape[1], live, _ptr(acc),
                        _ptr(mins), nthreads)
    return (out, acc, mins) if sums else out


def q6k_quantize(w, nthreads=0):
    """fp32 [N, K] -> GGUF block_q6_K bytes uint8 [N, K/256, 210] (this build's own quantizer)."""
    w = _c(np.ascontiguousarray(w, np.float32), np.float32)
    N, K = w.shape
    out = np.empty((N, K // 256, 210), np.uint8)
    lib().orc_q6k_quantize(_ptr(w), N, K, _ptr(out), nthreads)
    return out


def q6k_dequant(blocks):
    blocks = _c(np.ascontiguousarray(blocks), np.uint8)
    N, NB = blocks.shape[:2]
    w = np.empty((N, NB * 256), np.float32)
    lib().orc_q6k_dequant(_ptr(blocks), N, NB * 256, _ptr(w))
    return w


def q6k_repack(blocks):
    """-> dict(kind "q6k", q int8 [N, K], sc int8 [K/256, N, 16], d fp32 [K/256, N]) (kernels/w4a8.py:82-90)."""
    blocks = _c(np.ascontiguousarray(blocks), np.uint8)
    N, NB = blocks.shape[:2]
    K = NB * 256
    r = dict(kind="q6k", q=np.empty((N, K), np.int8), sc=np.empty((NB, N, 16), np.int8), d=np.empty((NB, N), np.float32))
    lib().orc_q6k_repack(_ptr(blocks), N, K, _ptr(r["q"]), _ptr(r["sc"]), _ptr(r["d"]))
    return r


def w4a8_gemm_q6k(xq, a, w6, epi=0, out=None, live=None, sums=False, nthreads=0):
    """(kernels/w4a8.py:193-197).  a fp32 [K/256, M] or [M].  Returns bf16 bits [M, N] (epi 0) or the updated fp32
    out (epi 1); with sums=True also acc int32 [M, N, K/256]."""
    xq = _c(np.ascontiguousarray(xq), np.int8)
    M, K = xq.shape
    N = w6["q"].shape[0]
    a = np.ascontiguousarray(a, np.float32)
    a_sb = 0 if a.ndim == 1 else M
    live = M if live is None else live
    if out is None:
        out = np.zeros((M, N), np.uint16 if epi == 0 else np.float32)
    acc = np.zeros((M, N, K // 256), np.int32) if sums else None
    lib().orc_w4a8_gemm_q6k(_ptr(xq), _ptr(a), a_sb, _ptr(w6["q"]), _ptr(w6["sc"]), _ptr(w6["d"]), M, N, K, epi,
                            _ptr(out), out.shape[1], live, _ptr(acc), nthreads)
    return (out, acc) if sums else out


# ------------------------------------------------------------------------------------------------- MXFP4
MX_E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
MX_MODES = {"max": 0, "mse": 1, "ocp": 2}
MX_FMT = {"e4m3": 0, "e2m1": 4}


def e4m3_code(v):
    return int(lib().orc_e4m3_code(float(v)))


def e4m3_value(c):
    return float(lib().orc_e4m3_value(int(c)))


def mx_pack(w, mode="max", nthreads=0):
    """fp32 [N, K] -> (q uint8 [N, K/2] low nibble first, s uint8 [N, K/32]) in the engine's row-major MX4 layout
    (kernels/mxfp4.py:57-86; mode "ocp" = tests/quant_sim.py:66-72 with round-to-nearest-even codes)."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    q = np.zeros((N, K // 2), np.uint8)
    s = np.zeros((N, K // 32), np.uint8)
    lib().orc_mx_pack(w.ctypes.data, N, K, MX_MODES[mode], q.ctypes.data, s.ctypes.data, nthreads)
    return q, s


def mx_quant_act(x, fmt="e4m3", inv=None, live=None, nthreads=0):
    """fp32 (or bf16-valued fp32) [M, K] -> (q, s): fmt "e2m1" = kernels/mxfp4.py:124-146 (q [M, K/2]); "e4m3" =
    tests/quant_sim.py:75-81 (q [M, K]); s [M, K/32].  Rows >= live stay zero."""
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    f = MX_FMT[fmt]
    q = np.zeros((M, K if f == 0 else K // 2), np.uint8)
    s = np.zeros((M, K // 32), np.uint8)
    inv = None if inv is None else np.ascontiguousarray(inv, np.float32)
    lib().orc_mx_quant_act(x.ctypes.data, _ptr(inv), M, K, f, M if live is None else live, q.ctypes.data,
                           s.ctypes.data, nthreads)
    return q, s


def mx_gemm(aq, a_s, wq, ws, fmt=None, nthreads=0):
    """float64 value of the scaled MX product and the sum of |terms| (for error bounds): ([M, N], [M, N])."""
    aq = np.ascontiguousarray(aq, np.uint8)
    a_s = np.ascontiguousarray(a_s, np.uint8)
    wq = np.ascontiguousarray(wq, np.uint8)
    ws = np.ascontiguousarray(ws, np.uint8)
    N, K = wq.shape[0], wq.shape[1] * 2
    M = aq.shape[0]
    if fmt is None:
        fmt = "e4m3" if aq.shape[1] == K else "e2m1"
    y = np.zeros((M, N), np.float64)
    ya = np.zeros((M, N), np.float64)
    lib().orc_mx_gemm(aq.ctypes.data, a_s.ctypes.data, MX_FMT[fmt], wq.ctypes.data, ws.ctypes.data, M, N, K,
                      y.ctypes.data, ya.ctypes.data, nthreads)
    return y, ya


# ------------------------------------------------------------------------------------------ fused producers
BACKS = {"q8": 0, "g256": 1, "grow": 2}


def expf(x):
    return float(lib().orc_expf(float(x)))


def sumsq_fixed(y):
    y = np.ascontiguousarray(y, np.float32)
    return float(lib().orc_sumsq_fixed(y.ctypes.data, y.shape[0]))


def _outs(M, K, back):
    q = np.zeros((M, K), np.int8)
    if back == "q8":
        return q, np.zeros(M, np.float32), None
    s = np.zeros((K // 256, M) if back == "g256" else M, np.float32)
    return q, s, np.zeros((K // 256, M, 16), np.int8)


def norm_quant(h, w, eps, back="q8", rows=None, live=None, nthreads=0):
    """h fp32 [*, HID], w fp32 [HID] -> (q, s[, xs]) of rmsnorm(h) * w (kernels/quant.py:144-170, :354-366)."""
    h = np.ascontiguousarray(h, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    M = h.shape[0] if rows is None else len(rows)
    HID = h.shape[1]
    rows = None if rows is None else np.ascontiguousarray(rows, np.int32)
    q, s, xs = _outs(M, HID, back)
    lib().orc_norm_quant(h.ctypes.data, HID, w.ctypes.data, _ptr(rows), M, float(eps), BACKS[back],
                         M if live is None else live, q.ctypes.data, s.ctypes.data, _ptr(xs), nthreads)
    return (q, s) if xs is None else (q, s, xs)


def swiglu_quant(gu, inv_s=None, back="q8", live=None, nthreads=0):
    """gu fp32 [M, 2 FF] -> (q, s[, xs]) of silu(gate) * up (* inv_s) (kernels/quant.py:249-280, :384-393)."""
    gu = np.ascontiguousarray(gu, np.float32)
    M, FF = gu.shape[0], gu.shape[1] // 2
    inv_s = None if inv_s is None else np.ascontiguousarray(inv_s, np.float32)
    q, s, xs = _outs(M, FF, back)
    lib().orc_swiglu_quant(gu.ctypes.data, FF, _ptr(inv_s), M, BACKS[back], M if live is None else live,
                           q.ctypes.data, s.ctypes.data, _ptr(xs), nthreads)
    return (q, s) if xs is None else (q, s, xs)


def head_sumsq(y):
    y = np.ascontiguousarray(y, np.float32)
    return float(lib().orc_head_sumsq(y.ctypes.data, y.shape[0]))


def gated_norm_quant(o, z, w, eps, HV, D, inv_s=None, back="q8", live=None, nthreads=0):
    """o fp32 [M, HV D], z fp32 [M, >= HV D] (the gate columns), w fp32 [D] -> (q, s[, xs]) of the per-head RMSNorm
    of o times w times silu(z) (times inv_s) (kernels/quant.py:216-246, :349-365)."""
    o = np.ascontiguousarray(o, np.float32)
    z = np.ascontiguousarray(z, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    M, K = o.shape[0], HV * D
    assert o.shape[1] == K and z.shape[1] >= K and w.shape[0] == D
    inv_s = None if inv_s is None else np.ascontiguousarray(inv_s, np.float32)
    q, s, xs = _outs(M, K, back)
    lib().orc_gated_norm_quant(o.ctypes.data, z.ctypes.data, z.shape[1], w.ctypes.data, _ptr(inv_s), M, HV, D,
                               float(eps), BACKS[back], M if live is None else live, q.ctypes.data, s.ctypes.data,
                               _ptr(xs), nthreads)
    return (q, s) if xs is None else (q, s, xs)
