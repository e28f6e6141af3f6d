"""The per-channel split decode (kernel "split": K in three parts writing their int32 sums to workspace slots, and a
second kernel adding them and applying the epilogue, the split-K of csrc/w8a8_gemm.cu:624-671): bit-exact
against the oracle and against the unsplit decode kernel, with four, two and one weight tiles per workgroup (N a
multiple of 64, of 32, of 16), both epilogues, live rows below M, calls back to back and replays of a captured graph
(the slots are rewritten by every launch)."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, rng, weights_f32

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _case(M, N, K, seed, dev):
    from prism_amd import w8a8 as KW
    wf = torch.from_numpy(weights_f32(N, K, seed=seed))
    ws = wf.abs().amax(1).clamp_min(1e-8) / 127.0
    wq = torch.round(wf / ws[:, None]).clamp(-127, 127).to(torch.int8).contiguous()
    a, sa = O.quant_rows_i8(acts_bf16(M, K, seed=seed + 1))
    pw = KW.pack_i8(wq.to(dev), ws.to(dev))
    return a, sa, wq.numpy(), ws.numpy().reshape(N, 1), pw


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("M,N,K,live", [(16, 5120, 5120, 16), (64, 5120, 17408, 64), (64, 5120, 17408, 41),
                                        (33, 2080, 4096, 33), (50, 1040, 1536, 29), (20, 256, 768, 20),
                                        (1, 512, 3072, 1), (4, 3072, 5120, 3), (200, 1024, 17408, 200),
                                        (512, 512, 4096, 300)])
def test_split_bit_exact(dev, M, N, K, live):
    from prism_amd import w8a8 as KW
    a, sa, wq, ws, pw = _case(M, N, K, 700 + M + N % 997, dev)
    want0 = O.w8a8_gemm(a, sa, wq, ws, K, epi=0, live=live, nthreads=16)
    base = rng(M + K).standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm(a, sa, wq, ws, K, epi=1, out=base.copy(), live=live, nthreads=16)
    ad, sad = _t(a, dev), _t(sa, dev)
    n = torch.tensor([live], dtype=torch.int32, device=dev)
    for rep in range(2):                               # back to back
        out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
        KW.gemm(ad, sad, pw, None, out, n, K, epi=0, kernel="split")
        h = _t(base, dev)
        KW.gemm(ad, sad, pw, None, h, n, K, epi=1, kernel="split")
        torch.cuda.synchronize()
        got = _bits(out)
        assert np.array_equal(got[:live], want0[:live]), rep
        assert (got[live:] == 7).all()
        assert np.array_equal(h.cpu().numpy(), want1), rep
    od = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    KW.gemm(ad, sad, pw, None, od, n, K, epi=0, kernel="decode")
    torch.cuda.synchronize()
    assert np.array_equal(_bits(od)[:live], got[:live])


def test_split_graph_replay(dev):
    """Captured once, replayed with new activations between replays: every replay equals the oracle."""
    from prism_amd import w8a8 as KW
    M, N, K = 64, 5120, 17408
    a, sa, wq, ws, pw = _case(M, N, K, 760, dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    ad, sad = _t(a, dev), _t(sa, dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    KW.gemm(ad, sad, pw, None, out, n, K, epi=0, kernel="split")    # eager first: the workspace exists
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            KW.gemm(ad, sad, pw, None, out, n, K, epi=0, kernel="split")
    for r in range(3):
        a2, sa2 = O.quant_rows_i8(acts_bf16(M, K, seed=770 + r))
        ad.copy_(_t(a2, dev))
        sad.copy_(_t(sa2, dev))
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), O.w8a8_gemm(a2, sa2, wq, ws, K, epi=0, nthreads=16)), r


def test_split_refuses_large_m(dev):
    """Beyond 512 rows the split is refused; "auto" there takes the unsplit kernels."""
    from prism_amd import _lib as L
    from prism_amd import w8a8 as KW
    M, N, K = 528, 512, 1024
    a, sa, wq, ws, pw = _case(M, N, K, 780, dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    with pytest.raises((L.PrismError, ValueError)):
        KW.gemm(_t(a, dev), _t(sa, dev), pw, None, out, n, K, epi=0, kernel="split")
    KW.gemm(_t(a, dev), _t(sa, dev), pw, None, out, n, K, epi=0)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), O.w8a8_gemm(a, sa, wq, ws, K, epi=0, nthreads=16))


@pytest.mark.parametrize("M,N,K,live,kernel", [(16, 5120, 5120, 16, "decode"), (8, 3072, 9216, 8, "decode"),
                                               (12, 5120, 17408, 9, "split"), (16, 1040, 1600, 16, "decode"),
                                               (7, 512, 4096, 7, "decode"), (16, 5120, 6144, 13, "split")])
def test_staged_decode_bit_exact(dev, M, N, K, live, kernel):
    """The decode kernel with its activation rows staged in LDS (8-16 rows, a grid within the CUs; K not a multiple
    of the 1 KB row piece included), unsplit and split, against the oracle; 7 rows take the unstaged form."""
    from prism_amd import w8a8 as KW
    a, sa, wq, ws, pw = _case(M, N, K, 900 + M + N % 991, dev)
    want0 = O.w8a8_gemm(a, sa, wq, ws, K, epi=0, live=live, nthreads=16)
    base = rng(M + N).standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm(a, sa, wq, ws, K, epi=1, out=base.copy(), live=live, nthreads=16)
    ad, sad = _t(a, dev), _t(sa, dev)
    n = torch.tensor([live], dtype=torch.int32, device=dev)
    out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    KW.gemm(ad, sad, pw, None, out, n, K, epi=0, kernel=kernel)
    h = _t(base, dev)
    KW.gemm(ad, sad, pw, None, h, n, K, epi=1, kernel=kernel)
    torch.cuda.synchronize()
    got = _bits(out)
    assert np.array_equal(got[:live], want0[:live]) and (got[live:] == 7).all()
    assert np.array_equal(h.cpu().numpy(), want1)
