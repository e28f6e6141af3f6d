"""MXFP4 projections on gfx950: e2m1 weights with one e8m0 scale per 32 inputs, e4m3 or e2m1 activations with one
e8m0 scale per 32 inputs, fp32 accumulation on the scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4).

Drop-in for StartLux-Prism kernels/mxfp4.py (MX4 :23-37, pack :57-86, dequant_packed :89-101, quantize_act :181-185,
quantize_act_scaled :173-178, gemm :292-317) with the same names and argument meaning, plus the C4 workload's
activation format (quantize_act_fp8: per-32 e4m3 with e8m0 scales, tests/quant_sim.py:75-81).

Differences from the reference, by design of this MI355X build:
  * MX4.q / MX4.s live on the GPU in the MFMA operand order (q [n/16, k/128, 64, 16], s [n/16, k/128, 64]: per
    16-row tile and 128-input step one 1 KB operand chunk); to_rows() gives the row-major bytes back and from_rows()
    takes them (e.g. from the engine's MX4 side files).  pack() quantizes on the GPU.
  * gemm() accepts activations as e2m1 (a_q [M, K/2], the engine's W4A4) or e4m3 (a_q [M, K]); the format follows
    from a_q's width.  n_rows may be an int (as in the reference) or a device int32 tensor of live rows.
  * There is no CUTLASS branch: one accumulation order serves every M (128-input MFMA steps chained within
    1024-input segments, segment sums added left to right), so outputs are batch invariant by construction.
"""
from typing import NamedTuple

import torch

from . import _lib as L

QK = 32
E4M3, E4M3_PANELS, E2M1 = 0, 1, 4
MODES = {"max": 0, "mse": 1, "ocp": 2}
KERNELS = {"auto": -1, "tile": 0, "decode": 1, "split": 2}
SPLIT_WS_BYTES = 32 << 20     # the split decode's segment sums: 1 KB per (1024-input segment, 16-row tile)
_WS = {}


def split_workspace(dev):
    """The per-device workspace of the split decode (kernel "split"): its segment sums, rewritten by every launch, so
    calls that overlap in time on one GPU (on different streams) must not both take the split.  None while a graph
    is being captured on a device that has none yet: "auto" then picks another kernel and "split" raises."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _WS.get(idx)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        ws = torch.empty(SPLIT_WS_BYTES, dtype=torch.uint8, device=torch.device("cuda", idx))
        _WS[idx] = ws
    return ws


class MX4(NamedTuple):
    q: torch.Tensor          # uint8 [n/16, k/128, 64, 16] MFMA operand order
    s: torch.Tensor          # uint8 [n/16, k/128, 64] e8m0 exponents
    n: int
    k: int
    cs: torch.Tensor = None  # the reference's CUTLASS scale copy; unused here

    @property
    def shape(self):
        return (self.n, self.k)

    def rows(self, r0, r1):
        """Rows r0 .. r1 (multiples of 16) as a view."""
        if r0 % 16 or r1 % 16:
            raise ValueError("MX4.rows: row bounds must be multiples of 16")
        return MX4(self.q[r0 // 16:r1 // 16], self.s[r0 // 16:r1 // 16], r1 - r0, self.k)

    @property
    def nbytes(self):
        return self.q.numel() + self.s.numel()


def _dev(t):
    if t.is_cuda:
        return t.device
    return torch.device("cuda", torch.cuda.current_device())


def pack(w: torch.Tensor, mode: str = "max") -> MX4:
    """A [n, k] fp32/bf16 matrix -> MX4 on the GPU.  mode "max": scale 2^ceil(log2(amax/6)); "mse": the power of
    two among that and half of it with the smaller squared error; "ocp": 2^(floor(log2 amax) - 2) with nearest-even
    codes (the C4 weights).  n % 16 == 0, k % 128 == 0."""
    n, k = w.shape
    if n % 16 or k % 128:
        raise ValueError(f"mxfp4.pack: n % 16 == 0 and k % 128 == 0 needed, got {tuple(w.shape)}")
    wf = w.detach().to(device=_dev(w), dtype=torch.float32).contiguous()
    q = torch.empty(n // 16, k // 128, 64, 16, dtype=torch.uint8, device=wf.device)
    s = torch.empty(n // 16, k // 128, 64, dtype=torch.uint8, device=wf.device)
    L.call("prism_mxfp4_pack", L.ptr(wf), k, L.ptr(q), L.ptr(s), n, k, MODES[mode], L.stream_of(wf))
    return MX4(q, s, n, k)


def from_rows(q: torch.Tensor, s: torch.Tensor, n=None, k=None) -> MX4:
    """Row-major MX4 bytes (q uint8 [n, k/2], s uint8 [n, k/32]) -> MX4 in the device layout."""
    n = q.shape[0] if n is None else n
    k = q.shape[1] * 2 if k is None else k
    if n % 16 or k % 128 or tuple(q.shape) != (n, k // 2) or tuple(s.shape) != (n, k // 32):
        raise ValueError("mxfp4.from_rows: q [n, k/2], s [n, k/32] with n % 16 == 0, k % 128 == 0")
    dev = _dev(q)
    qr = q.to(dev).contiguous()
    sr = s.to(dev).contiguous()
    qo = torch.empty(n // 16, k // 128, 64, 16, dtype=torch.uint8, device=dev)
    so = torch.empty(n // 16, k // 128, 64, dtype=torch.uint8, device=dev)
    L.call("prism_mxfp4_repack", L.ptr(qr), L.ptr(sr), L.ptr(qo), L.ptr(so), n, k, L.stream_of(qr))
    return MX4(qo, so, n, k)


def to_rows(w: MX4):
    """MX4 -> row-major (q uint8 [n, k/2], s uint8 [n, k/32]): the inverse permutation of from_rows."""
    nt, ks = w.n // 16, w.k // 128
    q = w.q.view(nt, ks, 4, 16, 16).permute(0, 3, 1, 2, 4).reshape(w.n, w.k // 2)
    s = w.s.view(nt, ks, 4, 16).permute(0, 3, 1, 2).reshape(w.n, w.k // 32)
    return q.contiguous(), s.contiguous()


_LUT = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6], dtype=torch.float32)


def dequant_packed(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """Row-major e2m1 q [n, k/2] and e8m0 s [n, k/32] -> fp32 [n, k] on the CPU (kernels/mxfp4.py:89-101; for
    tests and tools)."""
    q = q.cpu().long()
    n, k2 = q.shape
    v = torch.empty(n, k2 * 2, dtype=torch.float32)
    v[:, 0::2] = _LUT[q & 15]
    v[:, 1::2] = _LUT[q >> 4]
    sc = torch.pow(2.0, s.cpu().float() - 127)
    return (v.view(n, -1, QK) * sc[..., None]).view(n, k2 * 2)


def _quant(x, inv, q, s, fmt, n_rows=None):
    n, k = x.shape
    if x.dtype not in (torch.bfloat16, torch.float32) or x.stride(1) != 1:
        raise ValueError("mxfp4 quantize: x bf16 or fp32 with unit inner stride")
    if fmt == E4M3 and q.dim() == 3:
        fmt, want, got = E4M3_PANELS, _panel_shape(n, k), tuple(q.shape)
        if not q.is_contiguous():
            raise ValueError("mxfp4 quantize: panel buffer must be contiguous (act_panels)")
    else:
        want, got = ((n, k) if fmt == E4M3 else (n, k // 2)), tuple(q.shape[-2:])
    if q.dtype != torch.uint8 or s.dtype != torch.uint8 or got != want or s.shape[-1] != k // QK:
        raise ValueError(f"mxfp4 quantize: q uint8 {want}, s uint8 [{n}, {k // QK}]")
    if inv is not None:
        inv = inv.to(torch.float32).contiguous()
    live = n_rows if isinstance(n_rows, torch.Tensor) else None
    L.call("prism_mxfp4_quant_act", L.ptr(x), int(x.dtype == torch.float32), x.stride(0), L.ptr(inv), L.ptr(q),
           L.ptr(s), L.ptr(live), n, k, fmt, L.stream_of(x))


def quantize_act(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor) -> None:
    """x [n, k] bf16/fp32 -> q uint8 [n, k/2] (e2m1), s uint8 [n, k/32].  q, s are the caller's buffers."""
    _quant(x, None, q, s, E2M1)


def quantize_act_scaled(x: torch.Tensor, inv: torch.Tensor, q: torch.Tensor, s: torch.Tensor) -> None:
    """x [n, k] * inv [k] -> q uint8 [n, k/2], s uint8 [n, k/32]."""
    _quant(x, inv, q, s, E2M1)


def quantize_act_fp8(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor, n_rows=None) -> None:
    """x [n, k] bf16/fp32 -> q uint8 [n, k] (e4m3), s uint8 [n, k/32] (the MXFP8 activations of the C4 workload).
    q may instead be a panel buffer from act_panels(n, k): the same codes in the layout the prefill kernel reads."""
    _quant(x, None, q, s, E4M3, n_rows)


def _panel_shape(n, k):
    return ((n + 15) // 16, k // 128, 2048)


def act_panels(n: int, k: int, device) -> torch.Tensor:
    """A buffer for n e4m3 activation rows of k inputs in the panel layout (PRISM_MX_E4M3_PANELS): uint8
    [ceil(n / 16), k / 128, 2048], chunk [b, st] holding rows 16 b .. 16 b + 15, inputs 128 st .. + 127 in the order
    the tile kernel's lanes load them.  gemm() takes it for a_q; only the prefill tile kernel reads it."""
    if k % 128:
        raise ValueError("act_panels: k must be a multiple of 128")
    return torch.empty(_panel_shape(n, k), dtype=torch.uint8, device=device)


def panels_to_rows(q: torch.Tensor, n: int) -> torch.Tensor:
    """The row-major e4m3 codes [n, k] of a panel buffer (a byte permutation, for checks)."""
    b, ks, _ = q.shape
    t = q.view(b, ks, 2, 4, 16, 16).permute(0, 4, 1, 2, 3, 5).reshape(b * 16, ks * 128)
    return t[:n]


def gemm(a_q, a_s, w: MX4, out, n_rows, epi=0, out_stride=None, kernel="auto"):
    """a_q uint8 [n_rows, k/2] (e2m1) or [n_rows, k] (e4m3), or an e4m3 panel buffer (act_panels; the tile kernel
    reads it, same bits); a_s uint8 [n_rows, k/32]; w MX4 [N, k].  epi=0 writes bf16 into `out`; epi=1 adds into the
    fp32 residual `out`.  n_rows: int, or a device int32 [1] of live rows (then the launch covers a_s.shape[0] rows)."""
    K, N = w.k, w.n
    if w.q.dim() != 4 or tuple(w.q.shape) != (N // 16, K // 128, 64, 16) or tuple(w.s.shape) != (N // 16, K // 128, 64):
        if w.q.dim() == 2:
            raise ValueError("mxfp4.gemm: w holds row-major bytes (q [n, k/2], as pack() of the reference or a side "
                             "file gives them); convert once at load with mxfp4.from_rows(q, s)")
        raise ValueError(f"mxfp4.gemm: w must be in the device layout (q uint8 [{N // 16}, {K // 128}, 64, 16])")
    if isinstance(n_rows, torch.Tensor):
        M, live = (a_s.shape[0] if a_q.dim() == 3 else a_q.shape[0]), n_rows
    else:
        M, live = int(n_rows), None
    if a_q.dim() == 3:
        if tuple(a_q.shape) != _panel_shape(M, K) or not a_q.is_contiguous():
            raise ValueError(f"mxfp4.gemm: panel activations must be act_panels({M}, {K})")
        if kernel not in ("auto", "tile"):
            raise ValueError("mxfp4.gemm: panel activations are read by the tile kernel only")
        fmt = E4M3_PANELS
    elif a_q.shape[1] == K:
        fmt = E4M3
    elif a_q.shape[1] * 2 == K:
        fmt = E2M1
    else:
        raise ValueError(f"mxfp4.gemm: a_q width {a_q.shape[1]} matches neither e4m3 ({K}) nor e2m1 ({K // 2})")
    if fmt != E4M3_PANELS and (a_q.stride(1) != 1 or a_q.stride(0) != a_q.shape[1]) or a_s.stride(0) != K // QK:
        raise ValueError("mxfp4.gemm: a_q and a_s must be row-major with packed rows")
    if epi == 0 and out.dtype != torch.bfloat16 or epi == 1 and out.dtype != torch.float32:
        raise ValueError("mxfp4.gemm: epi 0 writes bf16, epi 1 adds into fp32")
    ldo = out.stride(0) if out_stride is None else out_stride
    ws = split_workspace(a_q.device) if fmt == E4M3 and M <= 16 and kernel in ("auto", "split") else None
    if kernel == "split" and ws is None:
        raise L.PrismError('kernel "split" needs the device workspace, made outside graph capture: run one eager call '
                           'first')
    L.call("prism_mxfp4_gemm_ws", L.ptr(a_q), L.ptr(a_s), fmt, L.ptr(w.q), L.ptr(w.s), L.ptr(out), ldo, L.ptr(live),
           M, N, K, epi, KERNELS[kernel], L.ptr(ws), 0 if ws is None else ws.numel(), L.stream_of(a_q))


def cutlass_enabled():
    """kernels/mxfp4.py:227-228: the reference's SM120 CUTLASS path; there is none on MI355X (one kernel family
    serves every M), so False and the engine's load_mlp keeps its MX4 objects as they are."""
    return False


def cutlass_prepare(w):
    """kernels/mxfp4.py:231-242: the CUTLASS scale copy; nothing to prepare here, w is returned as it is."""
    return w
