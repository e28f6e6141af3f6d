"""The reference's torch op schemas for this path, registered over libprism_amd.so.

StartLux-Prism registers its CUDA GEMMs as `torch.ops.startlux_prism.*` (csrc/w8a8_gemm.cu:794-797,
csrc/w4a8_gemm.cu:963-966) and reaches them through kernels/cuda_ext.py:load() (:48-72), which returns
`torch.ops.startlux_prism`.  `load()` here registers the same three schemas, with the same argument names, order and
defaults, and returns the same namespace, so a caller written against the reference's ops (the engine's W4A8 call
`CX.load().w4a8_gemm(xq, a, xs, w.q, w.sc, w.mn, w.d, w.dm, out, n_rows, kind, epi, cfg, stages, pdl)`,
kernels/w4a8.py:365) runs unchanged.  The ops launch on torch's current stream, so they can be captured in a graph.

What the arguments mean on MI355X:
* `cfg`, `stages`, `pdl`, `sk_waves`, `grid`: tile and pipeline choices of the CUDA kernels.  They are accepted and
  not used; the MI355X dispatch table picks the kernel for the shape (prism_amd.dispatch).
* `w8a8_gemm` `w`: the reference's plain int8 [N, K], or the packed per-channel tiles of `w8a8.pack_i8` (int8
  [N/16, K/64, 64, 16], the faster kernels).  Split modes "atomic", "workspace" and "cluster" (0-2) give the bits of
  the unsplit product, as the reference's "workspace" and "cluster" do (its "atomic" is order dependent, so the
  unsplit bits are one of its possible results).  Mode "defer" (3) with `split > 1` or `slot_stride > 0` writes
  int32 partial sums into `split` slots `slot_stride` elements apart, as the reference does (csrc/w8a8_gemm.cu:
  741-744); the slots' sum is the exact int32 product whatever the K parts are.  That mode needs packed weights.
* `w4a8_gemm` `wq`, `wsc`: this build's repacked Q4_K / Q6_K device layout (`w4a8.W4.qv` and `.meta`, which W4
  also names `.q` and `.sc`).  `wmn`, `wd` and `wdm` are accepted and not read: the mins, d and dmin travel in
  `wsc`.  `kind` 0 is Q4_K, 1 is Q6_K.
"""
from __future__ import annotations

import torch

from . import w4a8 as KW4
from . import w8a8 as KW8

W8A8_SCHEMA = ("w8a8_gemm(Tensor a, Tensor sa, Tensor w, Tensor sw, Tensor(a!) out, Tensor n_rows, int epi, int cfg, "
               "int split, int stages, int mode=2, Tensor(b!)? workspace=None, Tensor(c!)? counters=None, "
               "int slot_stride=0, int pdl=0) -> ()")
W8A8_SK_SCHEMA = ("w8a8_gemm_sk(Tensor a, Tensor sa, Tensor w, Tensor sw, Tensor(a!) out, Tensor n_rows, "
                  "Tensor(b!) ws, Tensor(c!) counters, int epi, int cfg, int stages, int grid, int sk_waves, "
                  "int pdl=0) -> ()")
W4A8_SCHEMA = ("w4a8_gemm(Tensor a, Tensor a_s, Tensor xs, Tensor wq, Tensor wsc, Tensor? wmn, Tensor wd, "
               "Tensor? wdm, Tensor(a!) out, Tensor n_rows, int kind, int epi, int cfg, int stages, int pdl=0) -> ()")

SPLIT_DEFER = 3          # kernels/cuda_ext.py:122 SPLIT_MODES["defer"]

_lib = None


def _weights(w, sw):
    """The op's `w` / `sw` -> what w8a8.gemm takes: plain int8 [N, K] with fp32 [N], or PackedPC from the packed
    tiles."""
    if w.dim() == 2:
        return w, sw
    if w.dim() != 4 or tuple(w.shape[2:]) != (64, 16) or w.dtype != torch.int8:
        raise ValueError("w must be int8 [N, K] or the packed per-channel tiles int8 [N/16, K/64, 64, 16]")
    n, k = w.shape[0] * 16, w.shape[1] * 64
    if sw.numel() != n:
        raise ValueError(f"sw must hold {n} per-channel scales")
    return KW8.PackedPC(w, sw.reshape(n, 1), n, k), None


def _w8a8_gemm(a, sa, w, sw, out, n_rows, epi, cfg, split, stages, mode=2, workspace=None, counters=None,
               slot_stride=0, pdl=0):
    """csrc/w8a8_gemm.cu:737-766: a int8 [M, K], sa fp32 [M], w int8 [N, K] (or packed), sw fp32 [N] -> out."""
    M, K = a.shape
    if epi not in (0, 1):
        raise NotImplementedError(f"epilogue {epi}")
    ww, ws = _weights(w, sw)
    if mode == SPLIT_DEFER and (split > 1 or slot_stride > 0):
        if epi != 1 or out.dtype != torch.int32:
            raise ValueError("deferred split-K: epilogue 1 with int32 slots")
        if not isinstance(ww, KW8.PackedPC):
            raise NotImplementedError("deferred split-K takes the packed per-channel weights: pack them once at load "
                                      "with prism_amd.w8a8.pack_i8")
        if split > 1 and slot_stride < out.shape[0] * out.stride(0):
            raise ValueError("deferred slots overlap")
        S = max(1, int(split))
        stride = slot_stride if S > 1 else out.shape[0] * out.stride(0)
        slots = torch.as_strided(out, (S, out.shape[0], out.shape[1]), (stride, out.stride(0), 1))
        got = KW8.gemm_i32(a, sa, ww, None, slots, n_rows, max_split=S)
        if got != S:              # the slots' sum is what the reader takes: fill the parts the split did not use
            slots[got:S].zero_()
        return
    KW8.gemm(a, sa.reshape(-1), ww, ws, out, n_rows, K, epi)


def _w8a8_gemm_sk(a, sa, w, sw, out, n_rows, ws, counters, epi, cfg, stages, grid, sk_waves, pdl=0):
    """csrc/w8a8_gemm.cu's persistent stream-K launch: the same product, so the same bits as w8a8_gemm."""
    _w8a8_gemm(a, sa, w, sw, out, n_rows, epi, cfg, 1, stages)


def _w4a8_gemm(a, a_s, xs, wq, wsc, wmn, wd, wdm, out, n_rows, kind, epi, cfg, stages, pdl=0):
    """csrc/w4a8_gemm.cu: xq int8 [M, K], a fp32 [K/256, M], xs int8 [K/256, M, 16], the repacked weights -> out."""
    if kind not in (0, 1):
        raise ValueError("kind: 0 (Q4_K) or 1 (Q6_K)")
    name = "q4k" if kind == 0 else "q6k"
    planes = 2 if kind == 0 else 4
    if wq.dim() != 5 or wq.shape[2] != planes:
        raise ValueError(f"wq must be the repacked {name.upper()} values (w4a8.repack(...).qv)")
    w = KW4.W4(name, wq, wsc, wq.shape[0] * 16, a.shape[1])
    KW4.gemm(a, a_s, xs, w, out, n_rows, epi)


def load():
    """Register the schemas once per process and return `torch.ops.startlux_prism` (kernels/cuda_ext.py:48-72)."""
    global _lib
    if _lib is None:
        lib = torch.library.Library("startlux_prism", "FRAGMENT")
        for schema, fn in ((W8A8_SCHEMA, _w8a8_gemm), (W8A8_SK_SCHEMA, _w8a8_gemm_sk), (W4A8_SCHEMA, _w4a8_gemm)):
            lib.define(schema)
            lib.impl(schema.split("(", 1)[0], fn, "CUDA")
        _lib = lib
    return torch.ops.startlux_prism


def l2_prefetch(tensors, ctas=32):
    """kernels/cuda_ext.py:171-173 (the engine's optional weight prefetch on a side stream, engine/model.py:785-791):
    an L2 residency hint for the next layer's weights.  On MI355X each XCD's L2 is 4 MB and the 256 MB MALL behind it
    already keeps recently streamed weights, so this is a no-op; it exists so an engine with the option on runs."""
    return None
