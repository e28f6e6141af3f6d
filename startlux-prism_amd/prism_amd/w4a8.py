"""W4A8 projections on gfx950: int8 activations x Q4_K weights on int8 MFMA.

Drop-in for StartLux-Prism kernels/w4a8.py's engine entry points: repack (:70-94), concat (:97-104), segments
(:107-120), seg_rows (:123-130), seg_width (:133-134), gemm_segs (:137-140) and gemm (:353-366), same argument names
and meaning.  Arithmetic (kernels/w4a8.py:14-22): per super-block b of 256 inputs, in increasing b,
acc = sum_g sc (xq . q)_g, mins = sum_g m S_g (int32, exact), t = RN(d float(acc)), t = fma(-dmin, float(mins), t),
y = fma(a[b, m], t, y); then bf16(y) or out += y.

W4 here holds the MFMA-native device layout made by repack.  Q4_K: a byte permutation of the GGUF block_q4_K bytes
(144 bytes per row and 256 inputs, no size overhead): qv uint8 [n/16, k/256, 2, 64, 16] (per 16-row tile and
super-block 2 KB of nibbles, each lane's 16 bytes unpacking to its MFMA operands) and meta uint8 [n/16, k/256, 16,
16] (per row the block's d, dmin and 12 bytes of 6-bit scales and mins).  Q6_K: the values as int8 q - 32, as the
reference's repack keeps them (kernels/w4a8.py:82-90): qv int8 [n/16, k/256, 4, 64, 16] (each lane's 16 bytes two
32-input MFMA operands) and meta uint8 [n/16, k/256, 288] (16 rows' 16 int8 scales, then their fp16 d).  Rows are
sliced and concatenated in whole 16-row tiles; a fused projection mixing the kinds is split into segments.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from . import _lib as L
from . import dispatch
from . import w8a8 as KW8
from .gguf_formats import KQuant, Q4_K_BYTES, Q6_K_BYTES, kquant_kind

QK_K = 256
# "stream": on Q6_K the per-tile stream kernel, on Q4_K the balanced-grid kernel (up to 16 rows, its activation image
# within LDS, with the device workspace of w8a8.workspace)
KERNELS = {"auto": -1, "tile": 0, "decode": 1, "stream": 2}


class W4(NamedTuple):
    kind: str               # "q4k" or "q6k"
    qv: torch.Tensor        # q4k: uint8 [n/16, k/256, 2, 64, 16]; q6k: int8 [n/16, k/256, 4, 64, 16]
    meta: torch.Tensor      # q4k: uint8 [n/16, k/256, 16, 16]; q6k: uint8 [n/16, k/256, 288]
    n: int
    k: int

    @property
    def shape(self):
        return (self.n, self.k)

    def rows(self, r0, r1):
        """Rows r0:r1 (multiples of 16): views of whole row tiles."""
        if r0 % 16 or r1 % 16:
            raise ValueError("W4 rows are sliced in whole 16-row tiles")
        return W4(self.kind, self.qv[r0 // 16:r1 // 16], self.meta[r0 // 16:r1 // 16], r1 - r0, self.k)

    def nbytes(self):
        return self.qv.numel() + self.meta.numel()

    # The reference W4's field names (kernels/w4a8.py:44-54), so its op call `w4a8_gemm(xq, a, xs, w.q, w.sc, w.mn,
    # w.d, w.dm, ...)` (kernels/w4a8.py:365) passes this layout through torch_ops unchanged: q the values, sc the
    # per-row meta bytes (scales, mins, d, dmin); mn and dm are not separate here (None), and d, which the schema
    # requires as a tensor, is the meta tensor again (not read).
    @property
    def q(self):
        return self.qv

    @property
    def sc(self):
        return self.meta

    @property
    def d(self):
        return self.meta

    @property
    def mn(self):
        return None

    @property
    def dm(self):
        return None


def _is_kquant(kq):
    """Duck type of a k-quant matrix: this build's gguf_formats.KQuant or the reference engine's own
    gguf_weights.KQuant (gguf_weights.py:100-112), both (raw uint8 [n, k/256, bytes], type, k)."""
    return all(hasattr(kq, f) for f in ("raw", "type", "k")) and isinstance(getattr(kq, "raw"), torch.Tensor)


def repack(kq) -> W4:
    """A KQuant (raw uint8 [n, k/256, 144] Q4_K or [n, k/256, 210] Q6_K, on the GPU; type the ggml id 12 / 14 as
    the reference's, or "q4k" / "q6k") -> W4."""
    if not _is_kquant(kq):
        raise ValueError(f"repack takes a k-quant matrix (raw, type, k), not {type(kq).__name__}")
    kind = kquant_kind(kq.type)
    raw = kq.raw.contiguous()
    n, k = raw.shape[0], int(kq.k)
    if raw.dim() != 3 or raw.shape[1] * QK_K != k:
        raise ValueError(f"raw must be [n, k/256, block bytes] with k = {k}")
    if n % 16:
        raise ValueError(f"{n} rows: the W4 device layout takes whole 16-row tiles")
    if kind == "q6k":
        if raw.dtype != torch.uint8 or raw.shape[-1] != Q6_K_BYTES:
            raise ValueError("raw Q6_K blocks expected")
        qv = torch.empty(n // 16, k // 256, 4, 64, 16, dtype=torch.int8, device=raw.device)
        meta = torch.empty(n // 16, k // 256, 288, dtype=torch.uint8, device=raw.device)
        L.call("prism_q6k_pack", L.ptr(raw), L.ptr(qv), L.ptr(meta), n, k, L.stream_of(raw))
        return W4("q6k", qv, meta, n, k)
    if raw.dtype != torch.uint8 or raw.shape[-1] != Q4_K_BYTES:
        raise ValueError("raw Q4_K blocks expected")
    qv = torch.empty(n // 16, k // 256, 2, 64, 16, dtype=torch.uint8, device=raw.device)
    meta = torch.empty(n // 16, k // 256, 16, 16, dtype=torch.uint8, device=raw.device)
    L.call("prism_q4k_pack", L.ptr(raw), L.ptr(qv), L.ptr(meta), n, k, L.stream_of(raw))
    return W4("q4k", qv, meta, n, k)


def concat(ws):
    """Row-concatenation of W4 matrices (a fused projection)."""
    if len({w.kind for w in ws}) != 1 or len({w.k for w in ws}) != 1:
        raise ValueError("cannot fuse different k-quant kinds or widths")
    return W4(ws[0].kind, torch.cat([w.qv for w in ws]), torch.cat([w.meta for w in ws]), sum(w.n for w in ws),
              ws[0].k)


def segments(kqs, device):
    """The KQuant matrices of a fused projection -> [(W4, first output column)], neighbours of one kind fused
    (kernels/w4a8.py:107-120).  Takes the reference engine's gguf_weights.KQuant as it is (engine/model.py:287)."""
    out, off = [], 0
    for kq in kqs:
        if not _is_kquant(kq):
            raise ValueError(f"the W4A8 path needs k-quant projections, not {type(kq).__name__}")
        w = repack(KQuant(kq.raw.to(device), kq.type, kq.k))
        if out and out[-1][0].kind == w.kind:
            out[-1] = (concat([out[-1][0], w]), out[-1][1])
        else:
            out.append((w, off))
        off += w.n
    return out


def seg_rows(segs, r0, r1):
    out = []
    for w, off in segs:
        a, b = max(r0, off), min(r1, off + w.n)
        if a < b:
            out.append((w.rows(a - off, b - off), a - r0))
    return out


def seg_width(segs):
    return max(off + w.n for w, off in segs)


def gemm_segs(xq, a, xs, segs, out, n_rows, epi=0, pdl=0):
    for w, off in segs:
        gemm(xq, a, xs, w, out[:, off:off + w.n], n_rows, epi, pdl=pdl)


def gemm(xq, a, xs, w: W4, out, n_rows, epi=0, cfg=None, pdl=0, kernel="auto"):
    """xq int8 [M, K]; a fp32 [K/256, M] (one scale per 256 inputs), [1, M] or [M] (one per token); xs int8
    [K/256, M, 16] split per-32 sums (Q4_K's mins; Q6_K does not read it) -> out (epi 0: bf16 [M, >= n]; epi 1: fp32,
    out += y).  n_rows: device int32 [1]; rows >= n_rows[0] untouched."""
    if epi not in (0, 1):
        raise NotImplementedError(f"epilogue {epi}")
    M, K = xq.shape
    if w.k != K or xq.dtype != torch.int8 or not xq.is_contiguous():
        raise ValueError("xq must be contiguous int8 [M, K] with K = w.k")
    if a.dtype != torch.float32:
        raise TypeError("a must be fp32")
    if a.dim() == 1 or a.shape[0] == 1:
        a_sb = 0
        if a.shape[-1] < M:
            raise ValueError("a too short")
    else:
        if a.shape[0] != K // QK_K or a.shape[1] < M or a.stride(1) != 1:
            raise ValueError("a must be [K/256, M]")
        a_sb = a.stride(0)
    want = torch.bfloat16 if epi == 0 else torch.float32
    if out.dtype != want or out.shape[0] < M or out.shape[1] < w.n or out.stride(1) != 1:
        raise ValueError(f"out must be {want} [>= {M}, >= {w.n}] with unit column stride")
    if kernel == "auto":             # the MI355X table's choice for the shape, where valid (dispatch.w4a8_kernel)
        c = dispatch.w4a8_kernel(w.kind, w.n, K, M)
        ok = c == "tile" or (c in ("decode", "stream") and M <= 16)
        kernel = c if ok else "auto"
    if w.kind == "q6k":              # no mins: xs is not read
        L.call("prism_w4a8_q6k_gemm", L.ptr(xq), L.ptr(a), a_sb, L.ptr(w.qv), L.ptr(w.meta), L.ptr(out),
               out.stride(0), L.ptr(n_rows), M, w.n, K, epi, KERNELS[kernel], L.stream_of(xq))
        return
    if xs.dtype != torch.int8 or tuple(xs.shape[::2]) != (K // QK_K, 16) or not xs.is_contiguous():
        raise ValueError("xs must be contiguous int8 [K/256, M, 16]")
    Mx = xs.shape[1]
    if Mx != M:
        raise ValueError("xs rows must equal xq rows")
    ws = KW8.workspace(xq.device) if M <= 16 and kernel in ("auto", "stream") else None
    if kernel == "stream" and ws is None:
        raise L.PrismError('kernel "stream" needs the device workspace, made outside graph capture: run one eager '
                           'call first')
    L.call("prism_w4a8_q4k_gemm", L.ptr(xq), L.ptr(a), a_sb, L.ptr(xs), L.ptr(w.qv), L.ptr(w.meta), L.ptr(out),
           out.stride(0), L.ptr(n_rows), M, w.n, K, epi, KERNELS[kernel], L.ptr(ws), 0 if ws is None else ws.numel(),
           L.stream_of(xq))
