"""W8A8 epilogue 2 (kernels/w8a8.py:86-98, SwiGLU into int8): for each BN-wide column tile (BN from the reference's
tile choice, w8a8.swiglu_tile) the gate half and the up half of the fp32 product give act = silu(gate) * up,
quantized with one scale per row and tile.  Bit-exact against the oracle's fp32 product and its SwiGLU quantizer
(the library's exact silu), on packed Q8_0, packed per-channel and plain int8 weights, with live rows below M; and
with weights built by interleave_gate_up, against separate gate and up products."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, q8_weights, weights_f32

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _pc_weights(N, K, seed):
    wf = torch.from_numpy(weights_f32(N, K, seed=seed))
    ws = wf.abs().amax(1).clamp_min(1e-8) / 127.0
    wq = torch.round(wf / ws[:, None]).clamp(-127, 127).to(torch.int8).contiguous()
    return wq, ws


def _expect(y, M, N, BN, live):
    """The oracle's epilogue 2 of an fp32 product y [M, N]."""
    nt, HB = N // BN, BN // 2
    q, s = O.swiglu_quant(y.reshape(M * nt, BN), back="q8", live=live * nt, nthreads=16)
    return q.reshape(M, nt * HB), s.reshape(M, nt)


def _run(dev, a, sa, w, ws, gk, M, N, live):
    from prism_amd import w8a8 as KW
    BN = KW.swiglu_tile(M, N, a.shape[1])
    out = torch.full((M, N // 2), 77, dtype=torch.int8, device=dev)
    outs = torch.full((M, N // BN), -1.0, dtype=torch.float32, device=dev)
    n = torch.tensor([live], dtype=torch.int32, device=dev)
    assert KW.gemm(_t(a, dev), _t(sa, dev), w, ws, out, n, gk, epi=2, outs=outs) is None
    torch.cuda.synchronize()
    return out.cpu().numpy(), outs.cpu().numpy(), BN


@pytest.mark.parametrize("kind,M,N,K,live", [("q8", 16, 256, 512, 13), ("pc", 100, 8192, 1024, 100),
                                             ("plain", 40, 8192, 5120, 29), ("q8", 300, 16384, 2048, 300)])
def test_epi2_bit_exact(dev, kind, M, N, K, live):
    from prism_amd import w8a8 as KW
    a, sa = O.quant_rows_i8(acts_bf16(M, K, seed=M + K))
    zero = np.zeros((M, N), np.float32)
    if kind == "q8":
        qs, d = q8_weights(N, K, seed=N + 1)
        w, ws, gk = KW.pack_q8(_t(qs, dev), _t(d, dev).view(torch.float16)), None, 32
        y = O.w8a8_gemm(a, sa, qs, d, 32, epi=1, out=zero.copy(), live=live, nthreads=16)
    else:
        wq, wsc = _pc_weights(N, K, seed=N + 2)
        gk = K
        if kind == "pc":
            w, ws = KW.pack_i8(wq.to(dev), wsc.to(dev)), None
        else:
            w, ws = wq.to(dev), wsc.to(dev)
        y = O.w8a8_gemm(a, sa, wq.numpy(), wsc.numpy().reshape(N, 1), K, epi=1, out=zero.copy(), live=live,
                        nthreads=16)
    got_q, got_s, BN = _run(dev, a, sa, w, ws, gk, M, N, live)
    want_q, want_s = _expect(y, M, N, BN, live)
    assert np.array_equal(got_q[:live], want_q[:live])
    assert np.array_equal(got_s[:live].view(np.uint32), want_s[:live].view(np.uint32))
    assert (got_q[live:] == 77).all() and (got_s[live:] == -1.0).all()


def test_epi2_interleaved_gate_up(dev):
    """Weights from interleave_gate_up(gate, up, BN): tile t's output is SwiGLU of gate columns t BN/2 .. and the
    same up columns of separate products."""
    from prism_amd import w8a8 as KW
    M, FF, K = 24, 4096, 768
    N = 2 * FF
    BN = KW.swiglu_tile(M, N, K)
    gq, gs = _pc_weights(FF, K, seed=5)
    uq, us = _pc_weights(FF, K, seed=6)
    w = KW.interleave_gate_up(gq, uq, BN)
    wsc = KW.interleave_gate_up(gs.view(FF, 1), us.view(FF, 1), BN).view(N)
    a, sa = O.quant_rows_i8(acts_bf16(M, K, seed=7))
    got_q, got_s, _ = _run(dev, a, sa, KW.pack_i8(w.to(dev), wsc.to(dev)), None, K, M, N, M)
    zero = np.zeros((M, FF), np.float32)
    yg = O.w8a8_gemm(a, sa, gq.numpy(), gs.numpy().reshape(FF, 1), K, epi=1, out=zero.copy(), nthreads=16)
    yu = O.w8a8_gemm(a, sa, uq.numpy(), us.numpy().reshape(FF, 1), K, epi=1, out=zero.copy(), nthreads=16)
    HB, nt = BN // 2, N // BN
    gu = np.concatenate([yg.reshape(M, nt, HB), yu.reshape(M, nt, HB)], axis=2).reshape(M * nt, BN)
    q, s = O.swiglu_quant(gu, back="q8", nthreads=16)
    assert np.array_equal(got_q, q.reshape(M, FF))
    assert np.array_equal(got_s.view(np.uint32), s.reshape(M, nt).view(np.uint32))
