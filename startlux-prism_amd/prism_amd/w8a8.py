"""W8A8 projections on gfx950: int8 x int8 MFMA GEMMs with per-group scales along K and fused epilogues.

Drop-in for StartLux-Prism kernels/w8a8.py's engine entry points (gemm :183-231, quant_rows :264-271,
weight_from_q8 :274-286) with the same argument names and meaning.  Arithmetic (kernels/w8a8.py:64-85): per group
g of gk inputs, in increasing g, P = sum a w (int32, exact) and y = RN(y + RN(RN(float(P) * a_s[m, g]) * w_s[n, g]));
epilogue 0 stores bf16(y), epilogue 1 adds y into an fp32 residual (out = RN(out + y)).  With gk = 32 the weights are
Q8_0's own int8 values and fp16 block scales; with gk = K the per-channel form.

Differences from the reference, by design of this single-GPU MI355X build:
  * w_s may be the Q8_0 fp16 scales themselves (torch.float16 [N, K/32]); the kernels widen them exactly, so the
    weight stream is 34 bytes per 32 weights instead of 36.
  * a_s may be fp32 [M] (or [M, 1]): one activation scale per token, broadcast over the groups.
  * The deferred split-K residual add (kernels/w8a8.py:200-204) is produced for per-channel packed weights only
    (PackedPC, epilogue 1, up to 64 rows, the decode kernel's domain, where K split over more workgroups feeds
    every CU): its int32 parts go to `slots` and gemm returns a Deferred for quant.norm_q8 / quant.fold, which give
    the residual the unsplit product's bits.  cfg / pdl are accepted and ignored.
  * Epilogue 2 (SwiGLU into int8, kernels/w8a8.py:86-98) runs as the product in fp32 (epilogue 1 into a zeroed
    buffer, so y exactly) followed by the SwiGLU quantizer over each tile's gate and up halves: the values of a fused
    epilogue, with the library's exact silu (quant.swiglu_q8), at the cost of one fp32 round trip of the product.
    Epilogue 3 (raw int32, tensor parallel) is gemm_i32.
"""
from typing import NamedTuple

import torch

from . import _lib as L
from . import dispatch
from .quant import quant_rows  # noqa: F401  (re-exported: kernels/w8a8.py:264)

KERNELS = {"auto": -1, "tile": 0, "decode": 1, "mid": 2, "reassoc": 3, "stream": 4}
# "stream" (packed Q8_0, 1..16 rows): the balanced decode kernel, whose workgroups take equal shares of the weight
# chunks and hand a split tile's running sums on through a small per-device workspace (workspace()).
# "reassoc" (packed Q8_0 only, by request, never chosen by "auto"): the prefill tile kernel with the per-token
# activation scale factored out of the block sum (y = fma(float(P), sw, y) per block, then y * a_s once), half the
# exact epilogue's vector work; not the reference's rounding order, so its bf16 outputs differ from the exact kernels'
# on a few outputs in 10^4, by at most 1 bf16 ulp plus 2 (K/32 + 2) 2^-24 sum |terms|.


class PackedQ8(NamedTuple):
    """Q8_0 weights [n, k] in the MFMA-native layout the packed kernels stream: qt int8 [n/16, k/64, 64, 16] (per
    16-row tile and block pair one 1 KB chunk, a wave's 16-byte-per-lane load), dt fp16 [n/16, k/64, 16, 2] (the
    chunk's block scales).  The same values and scales as the Q8_0 planes, permuted; made once at load by pack_q8."""
    qt: torch.Tensor
    dt: torch.Tensor
    n: int
    k: int

    @property
    def shape(self):
        return (self.n, self.k)


def pack_q8(qs, d):
    """Q8_0 planes (qs int8 [n, k], d fp16 [n, k/32], on the GPU) -> PackedQ8 (n % 16 == 0, k % 128 == 0, the packed
    GEMM's rule)."""
    n, k = qs.shape
    if qs.dtype != torch.int8 or d.dtype != torch.float16 or tuple(d.shape) != (n, k // 32):
        raise ValueError("pack_q8: qs int8 [n, k], d fp16 [n, k/32]")
    if not (qs.is_contiguous() and d.is_contiguous()):
        raise ValueError("pack_q8: contiguous planes expected")
    qt = torch.empty(n // 16, k // 64, 64, 16, dtype=torch.int8, device=qs.device)
    dt = torch.empty(n // 16, k // 64, 16, 2, dtype=torch.float16, device=qs.device)
    L.call("prism_q8_0_pack", L.ptr(qs), L.ptr(d), L.ptr(qt), L.ptr(dt), n, k, L.stream_of(qs))
    return PackedQ8(qt, dt, n, k)


class PackedPC(NamedTuple):
    """Per-channel (gk = K) int8 weights [n, k] in 1 KB chunks of 16 rows x 64 inputs (qt int8 [n/16, k/64, 64,
    16], lane slot l: row l % 16, inputs 16 (l / 16) .. + 15), with their per-channel scales ws (fp32 [n, 1]).  Made
    once at load by pack_i8 / weight_from_q8(q8, K); the decode kernels stream it as 1 KB chunks, and the prefill
    tile kernel loads each wave's MFMA fragments straight from them (a lane's 16 bytes are its operand)."""
    qt: torch.Tensor
    ws: torch.Tensor
    n: int
    k: int

    @property
    def shape(self):
        return (self.n, self.k)

    def __getitem__(self, key):
        """w[r0:r1]: the rows r0 .. r1 - 1 as a PackedPC view (no copy; r0 and r1 multiples of 16, whole 16-row
        chunks), the engine's row slice of a fused projection (engine/model.py:848-850: lw["qkv_q"][qn:]).  An integer
        index is the tuple's field."""
        if not isinstance(key, slice):
            return tuple.__getitem__(self, key)
        r0, r1, step = key.indices(self.n)
        if step != 1 or r0 % 16 or r1 % 16 or r1 <= r0:
            raise ValueError(f"PackedPC rows [{key.start}:{key.stop}]: whole 16-row chunks only")
        return PackedPC(self.qt[r0 // 16:r1 // 16], self.ws[r0:r1], r1 - r0, self.k)


def pack_i8(w, ws):
    """int8 [n, k] and scales [n] / [n, 1] (on the GPU) -> PackedPC (n % 16 == 0, k % 64 == 0).  The load-time step
    for the engine's smooth_quant output (engine/model.py:72-82): `wq, ws, extra = smooth_quant(...)` followed by
    `wq = pack_i8(wq, ws)` gives the operand the packed per-channel kernels read; the engine's calls
    `KW.gemm(xq, as_, wq, ws, ...)` and its row slices `wq[qn:]` then work unchanged (`ws` is then ignored: the
    scales travel in the PackedPC)."""
    n, k = w.shape
    if w.dtype != torch.int8 or not w.is_contiguous():
        raise ValueError("pack_i8: w must be contiguous int8 [n, k]")
    qt = torch.empty(n // 16, k // 64, 64, 16, dtype=torch.int8, device=w.device)
    L.call("prism_i8_pack", L.ptr(w), L.ptr(qt), n, k, L.stream_of(w))
    return PackedPC(qt, ws.reshape(n, 1).contiguous(), n, k)


class Deferred(NamedTuple):
    """A residual add left to the next kernel that reads the residual (quant.norm_q8 or quant.fold), as the
    reference's (kernels/w8a8.py:171-180): `n` int32 slots of partial sums, and the projection's activation and
    weight scales to apply to their total.  parts: the slots when they are not the reader's own `parts` buffer (this
    build always names them); sync: tensor-parallel readers, not used on one GPU."""
    n: int
    a_s: torch.Tensor
    w_s: torch.Tensor
    parts: torch.Tensor = None
    sync: object = None


def _scales_a(a_s, M, G):
    """-> (tensor, stride per row, stride per group) of the activation scales."""
    if a_s.dtype != torch.float32:
        raise TypeError("a_s must be fp32")
    if a_s.dim() == 1:
        if a_s.shape[0] < M:
            raise ValueError("a_s [M] too short")
        return a_s, a_s.stride(0), 0
    if a_s.shape[0] < M or a_s.shape[1] not in (1, G):
        raise ValueError(f"a_s must be [M], [M, 1] or [M, {G}], got {tuple(a_s.shape)}")
    return a_s, a_s.stride(0), (0 if a_s.shape[1] == 1 else a_s.stride(1))


def gemm(a, a_s, w, w_s, out, n_rows, gk, epi=0, outs=None, cfg=None, slots=None, pdl=False, kernel="auto"):
    """a int8 [M, K], a_s fp32 [M] / [M, 1] / [M, K/gk], w int8 [N, K], w_s fp16 or fp32 [N, K/gk] -> out
    (epi 0: bf16 [M, >=N] row stride out.stride(0); epi 1: fp32, out += y).  n_rows: device int32 [1], rows >=
    n_rows[0] untouched.  Returns None, or a Deferred when an epi 1 per-channel product split K into `slots` (int32
    [S, >= M, N]): then `out` is untouched and the residual add is finished by quant.norm_q8 / quant.fold."""
    if epi == 2:
        return _gemm_swiglu(a, a_s, w, w_s, out, outs, n_rows, gk, kernel)
    if epi not in (0, 1):
        raise NotImplementedError(f"epilogue {epi}: 0 (bf16 store), 1 (fp32 residual add), 2 (SwiGLU to int8); "
                                  "the raw int32 sums are gemm_i32")
    if isinstance(w, PackedQ8):
        return _gemm_packed(a, a_s, w, out, n_rows, gk, epi, kernel)
    if isinstance(w, PackedPC):
        if slots is not None and epi == 1 and gk == w.k:
            d = _gemm_pc_deferred(a, a_s, w, slots, n_rows, kernel)
            if d is not None:
                return d
        return _gemm_pc_packed(a, a_s, w, out, n_rows, gk, epi, kernel)
    if kernel == "reassoc":
        raise ValueError('kernel "reassoc" is the packed Q8_0 prefill tile kernel\'s (PackedQ8 weights)')
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K or a.dtype != torch.int8 or w.dtype != torch.int8:
        raise ValueError("a int8 [M, K] and w int8 [N, K] expected")
    if not (a.is_contiguous() and w.is_contiguous()):
        raise ValueError("a and w must be contiguous (K-major)")
    if gk <= 0 or K % gk:
        raise ValueError("gk must divide K")
    G = K // gk
    a_s, as_sm, as_sg = _scales_a(a_s, M, G)
    if G == 1 and w_s.dim() == 1 and w_s.shape[0] == N:
        w_s = w_s.view(N, 1)        # the engine's per-channel row scales, fp32 [N] (engine/model.py:72-82)
    if w_s.dtype not in (torch.float16, torch.float32) or tuple(w_s.shape) != (N, G) or not w_s.is_contiguous():
        raise ValueError(f"w_s must be contiguous fp16/fp32 [{N}, {G}]")
    want = torch.bfloat16 if epi == 0 else torch.float32
    if out.dtype != want or out.shape[0] < M or out.shape[1] < N or out.stride(1) != 1:
        raise ValueError(f"out must be {want} [>= {M}, >= {N}] with unit column stride")
    if n_rows.dtype != torch.int32:
        raise ValueError("n_rows must be int32")
    if gk == K:
        kernel = _tabled(kernel, N, K, M, gk)     # per channel on int8 planes: the same table as PackedPC
        if kernel == "split":
            kernel = "decode"                     # the split decode reads the packed chunks only
    L.call("prism_w8a8_gemm", L.ptr(a), L.ptr(a_s), as_sm, as_sg, L.ptr(w), L.ptr(w_s),
           int(w_s.dtype == torch.float16), L.ptr(out), out.stride(0), L.ptr(n_rows), M, N, K, gk, epi,
           KERNELS[kernel], L.stream_of(a))
    return None


def _tabled(kernel, N, K, M, gk, packed_q8=False):
    """kernel "auto": the MI355X table's choice for the shape (dispatch.w8a8_kernel) where it is valid at M."""
    if kernel == "reassoc" and not packed_q8:
        raise ValueError('kernel "reassoc" is the packed Q8_0 prefill tile kernel\'s; not for these weights')
    if kernel != "auto":
        return kernel
    c = dispatch.w8a8_kernel(N, K, M, gk)
    ok = c == "tile" or (c == "decode" and (M <= 64 or gk == K)) or (c == "mid" and gk == 32) or \
        (c == "stream" and packed_q8 and 1 <= M <= 16) or (c == "split" and gk == K and not packed_q8 and M <= 512)
    return c if ok else "auto"


_WS = {}
# the handoff words (the first 512 KB, the most any shape needs) and the prefill tile kernels' panel copy of the
# activations after them (ceil(M / 128) 128 K bytes; the library takes it from 1024 rows on projections at least
# 16384 wide)
Q8_HANDOFF_BYTES = 512 << 10
Q8_WS_BYTES = Q8_HANDOFF_BYTES + (96 << 20)


def workspace(dev):
    """The per-device workspace of the packed Q8_0 GEMM (the reference schema's `workspace`, allocated once per device
    as kernels/cuda_ext.py:138-143 does): the "stream" kernel's handoff words, zeroed once and left zeroed by every
    launch, then the prefill's panel copy of the activations.  None while a graph is
    being captured on a device that has none yet (its zero fill would be a graph node): "auto" then picks another
    kernel and "stream" raises."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _WS.get(idx)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        ws = torch.zeros(Q8_WS_BYTES, dtype=torch.uint8, device=torch.device("cuda", idx))
        torch.cuda.current_stream(idx).synchronize()
        _WS[idx] = ws
    return ws


def _gemm_packed(a, a_s, w, out, n_rows, gk, epi, kernel):
    M, K = a.shape
    asked = kernel
    kernel = _tabled(kernel, w.n, K, M, gk, packed_q8=True)
    if gk != 32 or (w.n, w.k) != (w.n, K) or w.k != K:
        raise ValueError("packed Q8_0 weights: gk must be 32 and K must match")
    if a.dtype != torch.int8 or not a.is_contiguous():
        raise ValueError("a must be contiguous int8 [M, K]")
    if a_s.dtype != torch.float32 or a_s.shape[0] < M or (a_s.dim() == 2 and a_s.shape[1] != 1):
        raise ValueError("packed kernels take one activation scale per token: a_s [M] or [M, 1]")
    want = torch.bfloat16 if epi == 0 else torch.float32
    if out.dtype != want or out.shape[0] < M or out.shape[1] < w.n or out.stride(1) != 1:
        raise ValueError(f"out must be {want} [>= {M}, >= {w.n}] with unit column stride")
    pan = M >= 1024 and w.n >= 16384 and kernel in ("auto", "tile", "reassoc") and \
        Q8_HANDOFF_BYTES + (M + 127) // 128 * 128 * K <= Q8_WS_BYTES
    ws = workspace(a.device) if (M <= 16 and kernel in ("auto", "decode", "stream")) or pan else None
    if kernel == "stream" and ws is None and asked == "auto":
        kernel = "auto"             # the table's pick needs the workspace; the library then picks without it
    if kernel == "stream" and ws is None:
        raise L.PrismError('kernel "stream" needs the device workspace, made outside graph capture: run one eager '
                           'call first')
    L.call("prism_w8a8_q8_0_packed_gemm", L.ptr(a), L.ptr(a_s), a_s.stride(0), L.ptr(w.qt), L.ptr(w.dt), L.ptr(out),
           out.stride(0), L.ptr(n_rows), M, w.n, K, epi, KERNELS[kernel], L.ptr(ws), 0 if ws is None else ws.numel(),
           L.stream_of(a))
    return None


_PCWS = {}
PC_WS_BYTES = 96 << 20        # as the reference's workspace (kernels/cuda_ext.py:20): the split decode's slots, or
                              # the tile kernel's panel copy of the activations


def pc_workspace(dev):
    """The per-device workspace of the per-channel GEMM: the split decode's int32 slots (kernel "split") or the tile
    kernel's panel copy of the activations (wide projections from 1024 rows), rewritten by every launch.  None while a graph is being captured on a device that has none yet: "auto" then picks another
    kernel and "split" raises."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _PCWS.get(idx)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        ws = torch.empty(PC_WS_BYTES, dtype=torch.uint8, device=torch.device("cuda", idx))
        _PCWS[idx] = ws
    return ws


_PC_KERNELS = {"auto": -1, "tile": 0, "decode": 1, "split": 2}


def _gemm_pc_packed(a, a_s, w, out, n_rows, gk, epi, kernel):
    M, K = a.shape
    asked = kernel
    kernel = _tabled(kernel, w.n, K, M, gk)
    if gk != K or w.k != K:
        raise ValueError("packed per-channel weights: gk must equal K and K must match")
    if a.dtype != torch.int8 or not a.is_contiguous():
        raise ValueError("a must be contiguous int8 [M, K]")
    if a_s.dtype != torch.float32 or a_s.shape[0] < M or (a_s.dim() == 2 and a_s.shape[1] != 1):
        raise ValueError("per-channel kernels take one activation scale per token: a_s [M] or [M, 1]")
    want = torch.bfloat16 if epi == 0 else torch.float32
    if out.dtype != want or out.shape[0] < M or out.shape[1] < w.n or out.stride(1) != 1:
        raise ValueError(f"out must be {want} [>= {M}, >= {w.n}] with unit column stride")
    if kernel not in _PC_KERNELS:
        raise ValueError(f"packed per-channel kernels: auto, tile, decode or split, not {kernel}")
    # the workspace: the split decode's slots (up to 512 rows), or the tile kernel's panel copy of the activations
    # (ceil(M / 16) 16 K bytes; the library takes it from 1024 rows on projections at least 16384 wide) where it fits
    use_ws = kernel == "split" or (kernel in ("auto", "tile") and
                                   (M <= 512 or (M + 15) // 16 * 16 * K <= PC_WS_BYTES))
    ws = pc_workspace(a.device) if use_ws else None
    if kernel == "split" and ws is None and asked == "auto":
        kernel = "auto"             # the table's pick needs the workspace; the library then picks without it
    if kernel == "split" and ws is None:
        raise L.PrismError('kernel "split" needs the device workspace, made outside graph capture: run one eager '
                           'call first')
    L.call("prism_w8a8_pc_packed_gemm_ws", L.ptr(a), L.ptr(a_s), a_s.stride(0), L.ptr(w.qt), L.ptr(w.ws),
           int(w.ws.dtype == torch.float16), L.ptr(out), out.stride(0), L.ptr(n_rows), M, w.n, K, epi,
           _PC_KERNELS[kernel], L.ptr(ws), 0 if ws is None else ws.numel(), L.stream_of(a))
    return None


# When a per-channel epilogue-1 product defers (the reference takes the split from its dispatch table,
# kernels/w8a8.py:199-204): measured on MI355X with the norm that finishes the add, splitting the decode kernel's K
# pays only for long K at 32-64 rows (5120 x 17408 at 64 rows: 57.4 -> 47.4 us for projection plus norm_q8; a tie at
# 16 rows; 10-40% slower at 1-4 rows or K <= 6144, where the slots' extra traffic and launch outweigh the spread).
# The count keeps the workgroups (two 16-row weight tiles each) within two per CU: 512.
def defer_split(M, N, K, S):
    """The number of K parts a deferred per-channel product uses with S slots available (1: do not defer)."""
    if M < 32 or M > 64 or K < 12288 or S < 2:
        return 1
    wgs = N // 32 if N % 32 == 0 else N // 16
    return max(1, min(4, S, 512 // max(1, wgs), K // (64 * 16)))


def _gemm_pc_deferred(a, a_s, w, slots, n_rows, kernel):
    M, K = a.shape
    if kernel not in ("auto", "decode"):
        return None
    if slots.dtype != torch.int32 or slots.dim() != 3 or slots.shape[1] < M or slots.shape[2] < w.n \
            or slots.stride(2) != 1:
        raise ValueError("slots must be int32 [S, >= M, >= N] with unit column stride")
    split = defer_split(M, w.n, K, slots.shape[0])
    if split < 2:
        return None
    if a.dtype != torch.int8 or not a.is_contiguous() or w.k != K:
        raise ValueError("a must be contiguous int8 [M, K] matching the weights")
    L.call("prism_w8a8_pc_packed_gemm_split", L.ptr(a), L.ptr(w.qt), L.ptr(slots), slots.stride(0), slots.stride(1),
           L.ptr(n_rows), M, w.n, K, split, L.stream_of(a))
    return Deferred(split, a_s, w.ws, slots)


def swiglu_tile(M, N, K):
    """The tile width BN of epilogue 2 for an M x N x K product: each BN-wide column tile holds BN / 2 gate columns
    then the matching up columns, and its SwiGLU output is quantized with one scale per row and tile.  The value the
    reference's tile choice gives epilogue 2 (kernels/w8a8.py:122-141, pick(M, N, K, 2)[1]), since the output format
    depends on it."""
    if N >= 8192:
        return 64 if M <= 64 else 128
    return 64 if K <= 4096 else 128


def interleave_gate_up(gate, up, bn):
    """Rows of gate [FF, K] and up [FF, K] -> [2 FF, K] in tiles of bn rows: bn / 2 gate rows, then the same up rows
    (kernels/w8a8.py:289-294), the weight order epilogue 2 reads."""
    FF, K = gate.shape
    h = bn // 2
    if FF % h or up.shape != gate.shape:
        raise ValueError("interleave_gate_up: gate and up [FF, K] with FF a multiple of bn / 2")
    return torch.stack([gate.reshape(FF // h, h, K), up.reshape(FF // h, h, K)], 1).reshape(2 * FF, K).contiguous()


def _gemm_swiglu(a, a_s, w, w_s, out, outs, n_rows, gk, kernel):
    """Epilogue 2 (kernels/w8a8.py:86-98): for every BN-wide tile t of the product y (BN = swiglu_tile(M, N, K)),
    act = silu(y[:, t BN + j]) * y[:, t BN + BN/2 + j], j < BN / 2, quantized per row and tile: outs[m, t] =
    RN(max(amax, 1e-10) / 127), out[m, t BN/2 + j] = rint(act / outs[m, t]).  out int8 [M, N / 2] contiguous, outs
    fp32 [M, N / BN] contiguous; rows >= n_rows untouched."""
    from . import quant as KQ
    M, K = a.shape
    N = w.n if isinstance(w, (PackedQ8, PackedPC)) else w.shape[0]
    BN = swiglu_tile(M, N, K)
    HB, nt = BN // 2, N // BN
    if N % BN:
        raise ValueError(f"epilogue 2: N ({N}) must be a multiple of the tile width {BN} (interleave_gate_up)")
    if out.dtype != torch.int8 or tuple(out.shape) != (M, N // 2) or not out.is_contiguous():
        raise ValueError(f"epilogue 2: out must be contiguous int8 [{M}, {N // 2}]")
    if outs is None or outs.dtype != torch.float32 or outs.numel() != M * nt or not outs.is_contiguous():
        raise ValueError(f"epilogue 2: outs must be contiguous fp32 [{M}, {nt}] (one scale per row and tile)")
    y = torch.empty(M, N, dtype=torch.float32, device=a.device).zero_()
    d = gemm(a, a_s, w, w_s, y, n_rows, gk, epi=1, kernel=kernel)
    assert d is None
    live = (n_rows * nt).to(torch.int32)
    KQ.swiglu_q8(y.view(M * nt, BN), None, out.view(M * nt, HB), outs.view(M * nt), live, M * nt)
    return None


def gemm_i32(a, a_s, w, w_s, slots, n_rows, max_split=4, pdl=False):
    """The int32 products a w^T without the scales (kernels/w8a8.py:234-262): split z's sums in slots[z] (int32
    [S, >= M, N]), returns the number of slots written.  On one GPU this is the deferred split's first half, used
    where the caller adds the parts itself; the reference's tensor-parallel callers add other ranks' parts too.
    w: per-channel packed weights (PackedPC).  a_s / w_s / pdl are accepted as the reference's and not used."""
    M, K = a.shape
    if not isinstance(w, PackedPC) or w.k != K:
        raise TypeError("gemm_i32 takes per-channel packed weights (PackedPC) matching a's K")
    if slots.dtype != torch.int32 or slots.dim() != 3 or slots.shape[1] < M or slots.shape[2] < w.n \
            or slots.stride(2) != 1:
        raise ValueError("slots must be int32 [S, >= M, >= N] with unit column stride")
    if a.dtype != torch.int8 or not a.is_contiguous():
        raise ValueError("a must be contiguous int8 [M, K]")
    split = max(1, min(max_split, slots.shape[0], defer_split(M, w.n, K, slots.shape[0])))
    L.call("prism_w8a8_pc_packed_gemm_split", L.ptr(a), L.ptr(w.qt), L.ptr(slots), slots.stride(0), slots.stride(1),
           L.ptr(n_rows), M, w.n, K, split, L.stream_of(a))
    return split


def weight_from_q8(q8, gk, smooth=None, packed=True):
    """Q8_0 matrix -> the GEMM's weight operands (kernels/w8a8.py:274-286).  gk == 32 keeps the Q8_0 values: by
    default as PackedQ8 (the MFMA-native layout; returned as (PackedQ8, None)), or with packed=False as the planes
    (int8 [N, K], fp16 [N, K/32]).  Otherwise the weights are requantized per gk inputs as the reference does
    (int8 [N, K], fp32 [N, K/gk]); for gk == K (per channel) on the GPU, by default packed as (PackedPC, None)."""
    if gk == 32 and smooth is None:
        if packed and q8.qs.is_cuda and q8.qs.shape[0] % 16 == 0 and q8.qs.shape[1] % 128 == 0:
            return pack_q8(q8.qs.contiguous(), q8.d.contiguous()), None
        return q8.qs.contiguous(), q8.d.contiguous()
    w = q8.dequant(torch.float32)
    if smooth is not None:
        w = w * smooth[None, :]
    N, K = w.shape
    g = w.view(N, K // gk, gk)
    s = g.abs().amax(-1).clamp_min(1e-10) / 127.0
    q = torch.round(g / s[..., None]).clamp(-127, 127).to(torch.int8).view(N, K)
    if gk == K and packed and q.is_cuda and N % 16 == 0 and K % 64 == 0:
        return pack_i8(q.contiguous(), s), None
    return q.contiguous(), s.contiguous()
