"""The per-channel and packed Q8_0 tile kernels on the panel copy of the activations (from 1024 rows on projections
at least 16384 wide, per channel also M N >= 2^25, where the GEMM's workspace holds the copy): bit-exact against the oracle and
equal to the row-major tile kernel (the same call without a workspace), both epilogues, M not a multiple of 16 or
of the 128-row tile, live rows below M, N not a multiple of the column tile, calls back to back, and replays of a
captured graph."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import rng
from test_pc_split_gpu import _bits, _case, _t

pytestmark = pytest.mark.gpu


def _call(a, sa, pw, out, n, epi, ws):
    from prism_amd import _lib as L
    M, K = a.shape
    L.call("prism_w8a8_pc_packed_gemm_ws", L.ptr(a), L.ptr(sa), sa.stride(0), L.ptr(pw.qt), L.ptr(pw.ws),
           int(pw.ws.dtype == torch.float16), L.ptr(out), out.stride(0), L.ptr(n), M, pw.n, K, epi, 0, L.ptr(ws),
           0 if ws is None else ws.numel(), L.stream_of(a))


@pytest.mark.parametrize("M,N,K,live", [(2048, 16384, 512, 2048), (2100, 16400, 1024, 1999),
                                        (2049, 16640, 1536, 2049)])
def test_panels_bit_exact(dev, M, N, K, live):
    from prism_amd import w8a8 as KW
    a, sa, wq, ws, pw = _case(M, N, K, 900 + M, dev)
    want0 = O.w8a8_gemm(a, sa, wq, ws, K, epi=0, live=live, nthreads=16)
    base = rng(M + 3).standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm(a, sa, wq, ws, K, epi=1, out=base.copy(), live=live, nthreads=16)
    ad, sad = _t(a, dev), _t(sa, dev)
    n = torch.tensor([live], dtype=torch.int32, device=dev)
    wsp = KW.pc_workspace(dev)
    for w in (wsp, wsp, None):                        # panels twice back to back, then the row-major kernel
        out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
        _call(ad, sad, pw, out, n, 0, w)
        h = _t(base, dev)
        _call(ad, sad, pw, h, n, 1, w)
        torch.cuda.synchronize()
        got = _bits(out)
        assert np.array_equal(got[:live], want0[:live]) and (got[live:] == 7).all()
        assert np.array_equal(h.cpu().numpy(), want1)


def test_panels_graph_replay(dev):
    """KW.gemm's "auto" path at 2048 rows and N = 16384 takes the panel copy; in a captured graph with new activations
    between replays every replay equals the oracle."""
    from prism_amd import w8a8 as KW
    M, N, K = 2048, 16384, 512
    _, _, wq, ws, pw = _case(M, N, K, 31, dev)
    KW.pc_workspace(dev)
    ad = torch.empty(M, K, dtype=torch.int8, device=dev)
    sad = torch.empty(M, dtype=torch.float32, device=dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    KW.gemm(ad, sad, pw, None, out, n, K, epi=0)       # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        KW.gemm(ad, sad, pw, None, out, n, K, epi=0)
    for rep in range(3):
        a, sa = O.quant_rows_i8(O.bf16_bits(rng(50 + rep).standard_normal((M, K)).astype(np.float32)))
        ad.copy_(_t(a, dev))
        sad.copy_(_t(sa.reshape(-1), dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = O.w8a8_gemm(a, sa, wq, ws, K, epi=0, nthreads=16)
        assert np.array_equal(_bits(out), want), rep


def _q8_call(a, s, pw, out, n, epi, kernel, ws):
    from prism_amd import _lib as L
    M, K = a.shape
    L.call("prism_w8a8_q8_0_packed_gemm", L.ptr(a), L.ptr(s), s.stride(0), L.ptr(pw.qt), L.ptr(pw.dt), L.ptr(out),
           out.stride(0), L.ptr(n), M, pw.n, K, epi, kernel, L.ptr(ws), 0 if ws is None else ws.numel(),
           L.stream_of(a))


@pytest.mark.parametrize("M,N,K,live", [(1024, 16384, 256, 1024), (1100, 16400, 1024, 999)])
def test_q8_panels_bit_exact(dev, M, N, K, live):
    """The packed Q8_0 tile kernels (exact and reassociated) on the panel copy past the handoff words (128-row tiles): the oracle's
    bits (exact kernel), the row-major call's bits (both), both epilogues; the handoff words stay zero."""
    from _inputs import acts_bf16, q8_weights
    from prism_amd import w8a8 as KW
    qs, d = q8_weights(N, K, seed=M + 1)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=M + 2))
    pw = KW.pack_q8(_t(qs, dev), _t(d, dev).view(torch.float16))
    ad, sd = _t(a, dev), _t(s, dev)
    n = torch.tensor([live], dtype=torch.int32, device=dev)
    want0 = O.w8a8_gemm(a, s, qs, d, 32, epi=0, live=live, nthreads=16)
    base = rng(M).standard_normal((M, N)).astype(np.float32)
    wsq = KW.workspace(dev)
    for kernel in (0, 3):
        outs = []
        for w in (wsq, None):
            out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
            _q8_call(ad, sd, pw, out, n, 0, kernel, w)
            h = _t(base, dev)
            _q8_call(ad, sd, pw, h, n, 1, kernel, w)
            torch.cuda.synchronize()
            outs.append((_bits(out), h.cpu().numpy()))
        assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1]), kernel
        assert (outs[0][0][live:] == 7).all()
        if kernel == 0:
            assert np.array_equal(outs[0][0][:live], want0[:live])
    assert not wsq[:KW.Q8_HANDOFF_BYTES].any()
