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


# ---------------------------------------------------------------------------------------------- fused producers
# kernels/quant.py:144-170 / :418-431 (norm_q8), :249-280 / :472-478 (swiglu_q8), :354-366 / :395-397 (norm_g),
# :384-393 / :403-406 (swiglu_g), :216-246 / :460-469 (gated_norm_q8), :349-365 / :399-401 (gated_norm_g).  Arithmetic: IEEE fp32 throughout, rsqrt as 1 / sqrt (both correctly rounded),
# exp this library's own (Cody-Waite reduction, degree-7 Taylor series), the sum of squares in a fixed order; the
# reference's NVIDIA approximations (rsqrt.approx, ex2.approx, div.full) have no specification to match bit for bit.

def _rows_arg(n, T, dev):
    return _live(n, T, dev)


def _fold_args(h, parts, pending, T):
    """(parts, part stride, row stride, count, psa, psa row stride, psw, psw fp16) of a Deferred."""
    if pending.sync is not None:
        raise NotImplementedError("tensor-parallel deferred adds (Sync) are out of scope on one GPU")
    if pending.parts is not None:
        parts = pending.parts
    HID = h.shape[1]
    if parts is None or parts.dtype != torch.int32 or parts.dim() != 3 or parts.shape[0] < pending.n \
            or parts.shape[1] < T or parts.shape[2] < HID or parts.stride(2) != 1:
        raise ValueError("parts must be int32 [>= n, >= T, >= HID] with unit column stride")
    psa = pending.a_s
    if psa.dtype != torch.float32:
        raise TypeError("the deferred activation scales must be fp32")
    psw = pending.w_s.reshape(-1)
    if psw.dtype not in (torch.float32, torch.float16) or psw.numel() < HID or not psw.is_contiguous():
        raise ValueError("the deferred weight scales must be contiguous fp32 / fp16 [HID]")
    return (L.ptr(parts), parts.stride(0), parts.stride(1), int(pending.n), L.ptr(psa), psa.stride(0), L.ptr(psw),
            int(psw.dtype == torch.float16))


def norm_q8(h, w_over_s, q, s, n, T, eps, rows=None, parts=None, pending=None):
    """h fp32 [*, HID] -> q int8 [>=T, HID], s fp32 [>=T]: y = rmsnorm(h) * w_over_s, one scale per row.  rows int32
    [T] (optional): output row i from input row rows[i].  pending (w8a8.Deferred or None): a residual add deferred
    by a split-K projection, finished in h first (its own slots when it names them, else `parts`) and kept there
    (kernels/quant.py:418-431); the deferred projection's activation scales may be `s` itself."""
    HID = h.shape[1]
    if h.dtype != torch.float32 or w_over_s.dtype != torch.float32 or q.dtype != torch.int8 or s.dtype != torch.float32:
        raise TypeError("norm_q8: h fp32, w fp32, q int8, s fp32")
    if h.stride(1) != 1 or q.shape[1] != HID or not q.is_contiguous() or w_over_s.numel() != HID:
        raise ValueError("norm_q8: shape mismatch")
    if rows is not None and (rows.dtype != torch.int32 or rows.numel() < T):
        raise ValueError("norm_q8: rows must be int32 [T]")
    n = _rows_arg(n, T, h.device)
    if pending:
        if rows is not None:
            raise ValueError("norm_q8: a deferred add and a row gather together (the reference asserts rows is None)")
        L.call("prism_norm_quant_fold", L.ptr(h), h.stride(0), L.ptr(w_over_s.contiguous()), L.ptr(q), L.ptr(s), None,
               L.ptr(n), T, HID, float(eps), 0, *_fold_args(h, parts, pending, T), L.stream_of(h))
        return
    L.call("prism_norm_quant", L.ptr(h), h.stride(0), L.ptr(w_over_s.contiguous()), L.ptr(rows), L.ptr(q), L.ptr(s),
           None, L.ptr(n), T, HID, float(eps), 0, L.stream_of(h))


def fold(h, parts, pending, n, T):
    """Finish a deferred residual add (w8a8.Deferred) in h when no norm follows (kernels/quant.py:449-457)."""
    if not pending:
        return
    if h.dtype != torch.float32 or h.stride(1) != 1:
        raise TypeError("fold: h must be fp32 rows")
    n = _rows_arg(n, T, h.device)
    L.call("prism_fold_parts", L.ptr(h), h.stride(0), *_fold_args(h, parts, pending, T), L.ptr(n), T, h.shape[1],
           L.stream_of(h))


def _swiglu(gu, inv_s, q, s, xs, n, T, back):
    FF = q.shape[1]
    if gu.dtype not in (torch.bfloat16, torch.float32) or q.dtype != torch.int8 or s.dtype != torch.float32:
        raise TypeError("swiglu: gu bf16 or fp32, q int8, s fp32")
    if gu.stride(1) != 1 or gu.shape[1] < 2 * FF or not q.is_contiguous():
        raise ValueError("swiglu: gu [*, 2 FF] with unit column stride, q [*, FF] contiguous")
    if inv_s is not None and (inv_s.dtype != torch.float32 or inv_s.numel() != FF):
        raise ValueError("swiglu: inv_s fp32 [FF]")
    n = _rows_arg(n, T, gu.device)
    L.call("prism_swiglu_quant", L.ptr(gu), int(gu.dtype == torch.float32), gu.stride(0),
           L.ptr(None if inv_s is None else inv_s.contiguous()), L.ptr(q), L.ptr(s), L.ptr(xs), L.ptr(n), T, FF, back,
           L.stream_of(gu))


def swiglu_q8(gu, inv_s, q, s, n, T, mode=0, amax=None, sync=None):
    """gu [*, 2 FF] (bf16 GEMM output, or fp32) -> q int8 [>=T, FF], s fp32 [>=T]: y = silu(gate) * up * inv_s."""
    if mode != 0 or sync is not None:
        raise NotImplementedError("tensor-parallel quantization modes are not part of the single-GPU build")
    _swiglu(gu, inv_s, q, s, None, n, T, 0)


def _g_back(q, s, xs, group):
    K, M = q.shape[1], xs.shape[1]
    if xs.dtype != torch.int8 or tuple(xs.shape) != (K // 256, M, 16) or not xs.is_contiguous():
        raise ValueError("xs must be int8 [K / 256, M, 16]")
    if group == 256:
        if tuple(s.shape) != (K // 256, M):
            raise ValueError("s must be fp32 [K / 256, M]")
        return 1
    if group == K:
        if s.numel() != M:
            raise ValueError("s must be fp32 [1, M] (one scale per token)")
        return 2
    raise ValueError("group must be 256 or K")


def norm_g(h, w, q, s, xs, n, T, eps, group=256):
    """W4A8 producer of rmsnorm(h) * w: q int8 [>=T, HID], s fp32 [HID / group, M], xs int8 [HID / 256, M, 16]."""
    HID = h.shape[1]
    if h.dtype != torch.float32 or w.dtype != torch.float32 or h.stride(1) != 1 or q.shape[1] != HID:
        raise ValueError("norm_g: h fp32 [*, HID] with unit column stride, w fp32 [HID]")
    back = _g_back(q, s, xs, group)
    n = _rows_arg(n, T, h.device)
    L.call("prism_norm_quant", L.ptr(h), h.stride(0), L.ptr(w.contiguous()), None, L.ptr(q), L.ptr(s), L.ptr(xs),
           L.ptr(n), xs.shape[1], HID, float(eps), back, L.stream_of(h))


def swiglu_g(gu, q, s, xs, n, T, group=256):
    """W4A8 producer of silu(gate) * up: q int8 [>=T, FF], s fp32 [FF / group, M], xs int8 [FF / 256, M, 16]."""
    back = _g_back(q, s, xs, group)
    FF = q.shape[1]
    if gu.dtype not in (torch.bfloat16, torch.float32) or gu.stride(1) != 1 or gu.shape[1] < 2 * FF:
        raise ValueError("swiglu_g: gu [*, 2 FF] bf16 or fp32")
    n = _rows_arg(n, T, gu.device)
    L.call("prism_swiglu_quant", L.ptr(gu), int(gu.dtype == torch.float32), gu.stride(0), None, L.ptr(q), L.ptr(s),
           L.ptr(xs), L.ptr(n), xs.shape[1], FF, back, L.stream_of(gu))


def _gated(o, proj, z_off, w, inv_s, q, s, xs, n, T, cfg, back):
    HV, D = cfg.v_heads, cfg.gdn_dim
    if getattr(cfg, "v_heads_full", HV) != HV:
        raise NotImplementedError("tensor-parallel head shards are not part of the single-GPU build")
    K = HV * D
    if o.dtype != torch.float32 or o.stride(-1) != 1 or o.reshape(o.shape[0], -1).shape[1] != K:
        raise ValueError("gated norm: o fp32 [*, v_heads, gdn_dim], unit column stride")
    if proj.dtype not in (torch.bfloat16, torch.float32) or proj.stride(1) != 1 or proj.shape[1] < z_off + K:
        raise ValueError("gated norm: proj [*, >= z_off + v_heads gdn_dim] bf16 or fp32")
    if w.dtype != torch.float32 or w.numel() != D:
        raise ValueError("gated norm: w fp32 [gdn_dim]")
    if q.dtype != torch.int8 or q.shape[1] != K or not q.is_contiguous() or s.dtype != torch.float32:
        raise ValueError("gated norm: q int8 [*, v_heads gdn_dim] contiguous, s fp32")
    if inv_s is not None and (inv_s.dtype != torch.float32 or inv_s.numel() != K):
        raise ValueError("gated norm: inv_s fp32 [v_heads gdn_dim]")
    o2 = o.reshape(o.shape[0], K)
    z = proj[:, z_off:]
    M = T if back == 0 else xs.shape[1]
    n = _rows_arg(n, T, o.device)
    L.call("prism_gated_norm_quant", L.ptr(o2), o2.stride(0), L.ptr(z), int(proj.dtype == torch.float32),
           proj.stride(0), L.ptr(w.contiguous()), L.ptr(None if inv_s is None else inv_s.contiguous()), L.ptr(q),
           L.ptr(s), L.ptr(xs), L.ptr(n), M, HV, D, float(cfg.eps), back, L.stream_of(o))


def gated_norm_q8(o, proj, z_off, w, inv_s, q, s, n, T, cfg, mode=0, amax=None, sync=None):
    """o fp32 [*, v_heads, gdn_dim] (the linear-attention output), proj [*, P] (the gate z at columns z_off ..),
    w fp32 [gdn_dim] -> q int8 [>= T, v_heads gdn_dim], s fp32 [>= T]: y = rmsnorm per head (o) * w * silu(z) *
    inv_s, one scale per row.  cfg: eps, v_heads, gdn_dim."""
    if mode != 0 or sync is not None:
        raise NotImplementedError("tensor-parallel quantization modes are not part of the single-GPU build")
    _gated(o, proj, z_off, w, inv_s, q, s, None, n, T, cfg, 0)


def gated_norm_g(o, proj, z_off, w, q, s, xs, n, T, cfg, group=256):
    """W4A8 producer of the gated norm: q int8 [>= T, K], s fp32 [K / group, M], xs int8 [K / 256, M, 16]
    (K = v_heads gdn_dim)."""
    back = _g_back(q, s, xs, group)
    _gated(o, proj, z_off, w, None, q, s, xs, n, T, cfg, back)
