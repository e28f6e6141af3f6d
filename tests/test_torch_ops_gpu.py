"""The reference's op calls, through torch.ops.startlux_prism as torch_ops.load() registers them, give the oracle's
bits: w8a8_gemm on plain and packed per-channel weights (epilogues 0 and 1, the split modes, the deferred int32
slots), w8a8_gemm_sk, and w4a8_gemm with the reference engine's argument list (kernels/w4a8.py:365) on Q4_K and Q6_K,
also inside a captured graph."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, rng, weights_f32

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _pc_case(M, N, K, seed):
    wf = torch.from_numpy(weights_f32(N, K, seed=seed))
    ws = wf.abs().amax(1).clamp_min(1e-8) / 127.0
    wq = torch.round(wf / ws[:, None]).clamp(-127, 127).to(torch.int8).contiguous()
    a, sa = O.quant_rows_i8(acts_bf16(M, K, seed=seed + 1))
    return a, sa, wq, ws


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_w8a8_gemm_op(dev, packed, mode):
    from prism_amd import torch_ops, w8a8 as KW
    ops = torch_ops.load()
    M, N, K = 37, 256, 3072
    a, sa, wq, ws = _pc_case(M, N, K, 600)
    want0 = O.w8a8_gemm(a, sa, wq.numpy(), ws.numpy().reshape(N, 1), K, epi=0)
    base = rng(603).standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm(a, sa, wq.numpy(), ws.numpy().reshape(N, 1), K, epi=1, out=base.copy())
    wd, wsd = wq.to(dev), ws.to(dev)
    if packed:
        wd = KW.pack_i8(wd, wsd).qt
    ad, sad = _t(a, dev), _t(sa, dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    out = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
    ops.w8a8_gemm(ad, sad, wd, wsd, out, n, 0, 3, 2 if mode else 1, 4, mode)
    h = _t(base, dev)
    ops.w8a8_gemm(ad, sad, wd, wsd, h, n, 1, 3, 2 if mode else 1, 4, mode)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), want0)
    assert np.array_equal(h.cpu().numpy(), want1)
    sk = torch.zeros_like(out)
    ops.w8a8_gemm_sk(ad, sad, wd, wsd, sk, n, torch.empty(1, device=dev), torch.empty(1, device=dev), 0, 3, 4, 256, 0)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(sk), want0)


@pytest.mark.parametrize("M,split", [(40, 1), (40, 3), (5, 2)])
def test_w8a8_gemm_op_deferred_slots(dev, M, split):
    """Mode "defer": `split` int32 slots, slot_stride apart, whose sum is the exact int32 product a w^T."""
    from prism_amd import torch_ops, w8a8 as KW
    ops = torch_ops.load()
    N, K = 128, 16384
    a, sa, wq, ws = _pc_case(M, N, K, 610)
    want = a.astype(np.int64) @ wq.numpy().astype(np.int64).T
    wd = KW.pack_i8(wq.to(dev), ws.to(dev)).qt
    slots = torch.full((max(split, 1), M, N), 12345, dtype=torch.int32, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    ops.w8a8_gemm(_t(a, dev), _t(sa, dev), wd, ws.to(dev), slots[0], n, 1, 0, split, 4, 3, None, None,
                  slots.stride(0) if split > 1 else M * N)
    torch.cuda.synchronize()
    got = slots.cpu().numpy().astype(np.int64).sum(0)
    assert np.array_equal(got, want)


def test_w8a8_gemm_op_deferred_needs_packed(dev):
    from prism_amd import torch_ops
    ops = torch_ops.load()
    a, sa, wq, ws = _pc_case(8, 64, 1024, 620)
    slots = torch.zeros(2, 8, 64, dtype=torch.int32, device=dev)
    n = torch.tensor([8], dtype=torch.int32, device=dev)
    with pytest.raises(NotImplementedError, match="pack_i8"):
        ops.w8a8_gemm(_t(a, dev), _t(sa, dev), wq.to(dev), ws.to(dev), slots[0], n, 1, 0, 2, 4, 3, None, None,
                      slots.stride(0))


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_w4a8_gemm_op_engine_call(dev, kind):
    """CX.load().w4a8_gemm(xq, a, xs, w.q, w.sc, w.mn, w.d, w.dm, out, n_rows, kind, epi, c, stages, pdl) verbatim,
    eager and replayed from a captured graph."""
    from prism_amd import torch_ops, w4a8 as KW4
    from prism_amd.gguf_formats import KQuant
    ops = torch_ops.load()
    M, N, K = 19, 96, 2048
    wf = weights_f32(N, K, seed=630)
    raw = O.q4k_quantize(wf) if kind == "q4k" else O.q6k_quantize(wf)
    w = KW4.repack(KQuant(torch.from_numpy(raw).to(dev), 12 if kind == "q4k" else 14, K))
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=631)), 256)
    if kind == "q4k":
        want = O.w4a8_gemm(xq, a, xs, O.q4k_repack(raw))
    else:
        want = O.w4a8_gemm_q6k(xq, a, O.q6k_repack(raw))
    xqd, ad, xsd = _t(xq, dev), _t(a, dev), _t(xs, dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    out = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
    k = 0 if w.kind == "q4k" else 1
    ops.w4a8_gemm(xqd, ad, xsd, w.q, w.sc, w.mn, w.d, w.dm, out, n, k, 0, 6, 4, 0)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), want)
    g_out = torch.zeros_like(out)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.w4a8_gemm(xqd, ad, xsd, w.q, w.sc, w.mn, w.d, w.dm, g_out, n, k, 0, 6, 4, 0)
    for _ in range(3):
        g_out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(g_out), want)
