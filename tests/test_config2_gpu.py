"""Benchmark config 2 (the Q8_0 decode sweep) at its real shapes, and the decode rows of configs 3 and 4 at full N.

Config 2: M in {1, 4, 16, 64} x (K, N) in {(5120, 5120), (17408, 5120)}, Q8_0 gk = 32, full N.  Every packed kernel
("auto" -- the MI355X table's choice, the one bench.py times --, "decode", "mid", "tile", and "stream" up to 16
rows) must give the oracle's bits
in both epilogues, and one live-row count below M per K leaves the rows past it untouched, as the reference's
tests/test_cuda_gemm.py:24-29 runs its every-config matrix on the real projection shapes.  Configs 3 and 4 at M = 16:
the whole N (13824 Q4_K rows, 5120 MXFP4 rows), through the kernel "auto" picks and the decode kernel."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import MX_ACC_REL, acts_bf16, q8_weights, rng, weights_f32

pytestmark = pytest.mark.gpu

C2 = [(M, K) for K in (5120, 17408) for M in (1, 4, 16, 64)]
N2 = 5120
_W = {}


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _bits(out):
    return out.view(torch.int16).cpu().numpy().view(np.uint16)


def _packed(dev, K):
    """Config 2's weights for one K (N = 5120), quantized once per session: (qs, d, PackedQ8)."""
    if K not in _W:
        from prism_amd import w8a8 as KW
        qs, d = q8_weights(N2, K, seed=200 + K)
        pw = KW.pack_q8(_t(qs, dev), _t(d, dev).view(torch.float16))
        _W.clear()
        _W[K] = (qs, d, pw)
    return _W[K]


@pytest.mark.parametrize("M,K", C2)
def test_config2_every_kernel_bit_exact(dev, M, K):
    from prism_amd import w8a8 as KW
    qs, d, pw = _packed(dev, K)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=300 + M + K))
    live = {1: 1, 4: 4, 16: 11, 64: 37}[M] if K == 17408 else M      # one live < M case per K (M >= 16)
    if K == 5120 and M == 64:
        live = 50
    want0 = O.w8a8_gemm(a, s, qs, d, 32, epi=0, live=live, nthreads=16)
    base = rng(M + K).standard_normal((M, N2)).astype(np.float32)
    want1 = O.w8a8_gemm(a, s, qs, d, 32, epi=1, out=base.copy(), live=live, nthreads=16)
    ad, sd, n = _t(a, dev), _t(s, dev), torch.tensor([live], dtype=torch.int32, device=dev)
    for kernel in ("auto", "decode", "mid", "tile") + (("stream",) if M <= 16 else ()):
        print(f"config 2 M={M} K={K} live={live} kernel={kernel}", flush=True)
        out = torch.full((M, N2), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
        KW.gemm(ad, sd, pw, None, out, n, 32, epi=0, kernel=kernel)
        o1 = _t(base, dev).clone()
        KW.gemm(ad, sd, pw, None, o1, n, 32, epi=1, kernel=kernel)
        torch.cuda.synchronize()
        got = _bits(out)
        assert np.array_equal(got[:live], want0[:live]), kernel
        assert (got[live:] == 7).all(), kernel
        assert np.array_equal(o1.cpu().numpy(), want1), kernel


def test_config3_decode_full_n(dev):
    """Config 3 at M = 16: K = 5120, all N = 13824 Q4_K rows, one activation scale per token."""
    from prism_amd import gguf_formats as GF
    from prism_amd import w4a8 as KW4
    M, K, N = 16, 5120, 13824
    blocks = O.q4k_quantize(weights_f32(N, K, seed=403), nthreads=16)
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=404)), K)
    want = O.w4a8_gemm(xq, a[0].copy(), xs, O.q4k_repack(blocks), nthreads=16)
    w = KW4.repack(GF.KQuant(_t(blocks, dev), GF.GGML_Q4_K, K))
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    for kernel in ("auto", "decode", "stream"):
        print(f"config 3 M=16 full N kernel={kernel}", flush=True)
        out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
        KW4.gemm(_t(xq, dev), _t(a, dev), _t(xs, dev), w, out, n, kernel=kernel)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), want), kernel


def test_config4_decode_full_n(dev):
    """Config 4 at M = 16: K = N = 5120 (all rows), e2m1 OCP weights x e4m3 activations, within the fp32 bound of the
    oracle's float64 value and 1e-2 relative error; "auto" and "decode" give the same bits."""
    from prism_amd import mxfp4 as MX
    M, K, N = 16, 5120, 5120
    mw = MX.pack(_t(weights_f32(N, K, seed=405), dev), "ocp")
    x = _t(acts_bf16(M, K, seed=406).view(np.int16), dev).view(torch.bfloat16)
    aq = torch.empty(M, K, dtype=torch.uint8, device=dev)
    asc = torch.empty(M, K // 32, dtype=torch.uint8, device=dev)
    MX.quantize_act_fp8(x, aq, asc)
    outs = {}
    for kernel in ("auto", "decode"):
        print(f"config 4 M=16 full N kernel={kernel}", flush=True)
        out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
        MX.gemm(aq, asc, mw, out, M, kernel=kernel)
        torch.cuda.synchronize()
        outs[kernel] = _bits(out)
    assert np.array_equal(outs["auto"], outs["decode"])
    wq, ws = (t.cpu().numpy() for t in MX.to_rows(mw))
    y64, yabs = O.mx_gemm(aq.cpu().numpy(), asc.cpu().numpy(), wq, ws, nthreads=16)
    got = O.bf16_to_f32(outs["decode"]).astype(np.float64)
    assert (np.abs(got - y64) <= 2.0 ** -8 * np.abs(y64) + MX_ACC_REL * yabs + 1e-30).all()
    assert np.linalg.norm(got - y64) / np.linalg.norm(y64) < 1e-2
