"""Activation producers: per-token int8 quantization for the W8A8 GEMM, and the W4A8 producer with per-32 sums.

Drop-in for StartLux-Prism kernels/quant.py's rows_q8 (:481-486) and rows_g (:409-411): same argument names,
meaning and buffers (the caller preallocates every output; `n` is a device int32 [1] live-row count).  The
tensor-parallel modes (mode 1/2/3, amax exchange, sync) are not part of this single-GPU build and raise.
"""
import torch

from . import _lib as L


def _live(n, T, dev):
    if n is None:
        return torch.tensor([T], dtype=torch.int32, device=dev)
    if n.dtype != torch.int32 or n.device != dev:
        raise ValueError("n must be a device int32 tensor on the tensors' device")
    return n


def rows_q8(x, inv_s, q, s, n, T, mode=0, amax=None, sync=None):
    """x bf16 [>=T, K] -> q int8 [>=T, K], s fp32 [>=T]: per row y = x * inv_s (inv_s fp32 [K] or None),
    scale = max(amax|y|, 1e-10) / 127, q = rint(y / scale) (IEEE divisions).  Rows >= n[0] untouched."""
    if mode != 0 or sync is not None:
        raise NotImplementedError("tensor-parallel quantization modes are not part of the single-GPU build")
    K = q.shape[1]
    if x.dtype != torch.bfloat16 or q.dtype != torch.int8 or s.dtype != torch.float32:
        raise TypeError("rows_q8: x bf16, q int8, s fp32")
    if x.shape[1] != K or x.stride(1) != 1 or not q.is_contiguous() or x.shape[0] < T or q.shape[0] < T or s.numel() < T:
        raise ValueError("rows_q8: shape mismatch")
    if inv_s is not None and (inv_s.dtype != torch.float32 or inv_s.numel() != K or not inv_s.is_contiguous()):
        raise ValueError("rows_q8: inv_s must be fp32 [K] contiguous")
    n = _live(n, T, x.device)
    L.call("prism_quant_rows_i8", L.ptr(x), x.stride(0), L.ptr(inv_s), L.ptr(q), L.ptr(s), L.ptr(n), T, K,
           L.stream_of(x))


def quant_rows(x, gk, n_rows=None):
    """x bf16 [M, K] -> (q int8 [M, K], s fp32 [M, K / gk]) with one scale per (row, gk inputs)
    (kernels/w8a8.py:264-271)."""
    M, K = x.shape
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise TypeError("quant_rows: x must be contiguous bf16")
    q = torch.empty(M, K, dtype=torch.int8, device=x.device)
    s = torch.empty(M, K // gk, dtype=torch.float32, device=x.device)
    n = _live(n_rows, M, x.device)
    L.call("prism_quant_rows_groups", L.ptr(x), L.ptr(q), L.ptr(s), L.ptr(n), M, K, gk, L.stream_of(x))
    return q, s


def rows_g(x, q, s, xs, n, T, group=256):
    """W4A8 producer: x bf16 [>=T, K] -> q int8 [>=T, K], s fp32 [K / group, M], xs int8 [K / 256, M, 16]
    (M = s.shape[1]).  group 256 is the reference's scale per 256 inputs; group K gives one scale per token
    (s then [1, M]).  Per 32 inputs the int32 sum S of q is stored as S & 63 then S >> 6."""
    K = q.shape[1]
    M = s.shape[1]
    if x.dtype != torch.bfloat16 or q.dtype != torch.int8 or s.dtype != torch.float32 or xs.dtype != torch.int8:
        raise TypeError("rows_g: x bf16, q int8, s fp32, xs int8")
    if s.shape[0] != K // group or tuple(xs.shape) != (K // 256, M, 16) or x.stride(1) != 1 or not q.is_contiguous():
        raise ValueError("rows_g: shape mismatch")
    if not (s.is_contiguous() and xs.is_contiguous()) or T > M:
        raise ValueError("rows_g: s and xs must be contiguous, T <= M")
    n = _live(n, T, x.device)
    L.call("prism_quant_rows_g", L.ptr(x), x.stride(0), L.ptr(q), L.ptr(s), L.ptr(xs), L.ptr(n), M, K, group,
           L.stream_of(x))
