"""A seeded sweep of random shapes through every GEMM kernel and weight format, bit for bit against the CPU oracle
(MXFP4: within its fp32 bound): rows, live rows, N, K, the epilogue and the kernel are drawn per case, so shape edges
(a single row, a partial tile, live < M, K at the smallest step) meet every kernel rather than only the hand-picked
cases of the per-format tests.  PRISM_SWEEP_BASE=<n> draws another set of cases (the default set is n = 0)."""
import os

import numpy as np
import pytest
import torch

import oracle as O
from _inputs import MX_ACC_REL, acts_bf16, q6k_random_blocks, rng, weights_f32

pytestmark = pytest.mark.gpu
BASE = 100000 * int(os.environ.get("PRISM_SWEEP_BASE", "0"))


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _n(v, dev):
    return torch.tensor([v], dtype=torch.int32, device=dev)


def _draw(g, kmul, kmax, nmax=640):
    M = int(g.choice([1, 2, 3, 5, 8, 13, 16, 17, 31, 40, 64, 65, 100, 130]))
    live = int(g.integers(1, M + 1))
    N = 16 * int(g.integers(1, nmax // 16 + 1))
    K = kmul * int(g.integers(1, kmax // kmul + 1))
    return M, live, N, K, int(g.integers(0, 2))


def _out(dev, M, N, epi, base):
    if epi == 0:
        return torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    return _t(base, dev).clone()


def _check(out, want, live, epi):
    if epi == 0:
        got = out.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got[:live], want[:live]) and (got[live:] == 7).all()
    else:
        assert np.array_equal(out.cpu().numpy().view(np.int32), want.view(np.int32))


@pytest.mark.parametrize("case", range(12))
def test_w8a8_q8_0_random(dev, case):
    from prism_amd import gguf_formats as GF
    from prism_amd import w8a8 as KW
    g = rng(1000 + case + BASE)
    M, live, N, K, epi = _draw(g, 128, 4096)
    kernel = str(g.choice(["tile", "mid"] + (["decode"] if M <= 64 else [])))
    qs, d = O.q8_0_quantize(weights_f32(N, K, seed=case + BASE))
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=case + 1 + BASE))
    base = g.standard_normal((M, N)).astype(np.float32)
    want = O.w8a8_gemm(a, s, qs, d, 32, epi=epi, out=None if epi == 0 else base.copy(), live=live)
    pw = KW.pack_q8(_t(qs, dev), _t(d.view(np.int16), dev).view(torch.float16))
    out = _out(dev, M, N, epi, base)
    KW.gemm(_t(a, dev), _t(s, dev), pw, None, out, _n(live, dev), 32, epi=epi, kernel=kernel)
    torch.cuda.synchronize()
    _check(out, want, live, epi)


@pytest.mark.parametrize("case", range(10))
def test_w8a8_per_channel_random(dev, case):
    from prism_amd import w8a8 as KW
    g = rng(2000 + case + BASE)
    M, live, N, K, epi = _draw(g, 64, 6144)
    kernel = str(g.choice(["tile", "decode"] + (["split"] if K >= 768 else [])))
    w = g.integers(-127, 128, (N, K)).astype(np.int8)
    a = g.integers(-127, 128, (M, K)).astype(np.int8)
    sa = (g.random(M) * 0.02).astype(np.float32)
    sw = (g.random(N) * 0.01).astype(np.float32)
    base = g.standard_normal((M, N)).astype(np.float32)
    want = O.w8a8_gemm(a, sa, w, sw.reshape(N, 1), K, epi=epi, out=None if epi == 0 else base.copy(), live=live)
    pw = KW.pack_i8(_t(w, dev), _t(sw, dev))
    out = _out(dev, M, N, epi, base)
    KW.gemm(_t(a, dev), _t(sa, dev), pw, None, out, _n(live, dev), K, epi=epi, kernel=kernel)
    torch.cuda.synchronize()
    _check(out, want, live, epi)


@pytest.mark.parametrize("case", range(10))
def test_w4a8_q4k_random(dev, case):
    from prism_amd import gguf_formats as GF
    from prism_amd import w4a8 as KW4
    g = rng(3000 + case + BASE)
    M, live, N, K, epi = _draw(g, 256, 6144)
    kernel = str(g.choice(["tile"] + (["decode", "stream"] if M <= 16 else [])))
    group = int(g.choice([256, K]))
    blocks = O.q4k_quantize(weights_f32(N, K, seed=case + 7 + BASE))
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=case + 8 + BASE)), group)
    ao = a if group == 256 else a[0].copy()
    base = g.standard_normal((M, N)).astype(np.float32)
    want = O.w4a8_gemm(xq, ao, xs, O.q4k_repack(blocks), epi=epi, out=None if epi == 0 else base.copy(), live=live)
    w = KW4.repack(GF.KQuant(_t(blocks, dev), GF.GGML_Q4_K, K))
    out = _out(dev, M, N, epi, base)
    KW4.gemm(_t(xq, dev), _t(a, dev), _t(xs, dev), w, out, _n(live, dev), epi=epi, kernel=kernel)
    torch.cuda.synchronize()
    _check(out, want, live, epi)


@pytest.mark.parametrize("case", range(10))
def test_w4a8_q6k_random(dev, case):
    from prism_amd import gguf_formats as GF
    from prism_amd import w4a8 as KW4
    g = rng(4000 + case + BASE)
    M, live, N, K, epi = _draw(g, 256, 6144)
    kernel = str(g.choice(["tile"] + (["decode", "stream"] if M <= 16 else [])))
    blocks = q6k_random_blocks(N, K // 256, seed=case + 9 + BASE)
    xq, a, _ = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=case + 10 + BASE)), 256)
    base = g.standard_normal((M, N)).astype(np.float32)
    want = O.w4a8_gemm_q6k(xq, a, O.q6k_repack(blocks), epi=epi, out=None if epi == 0 else base.copy(), live=live)
    w = KW4.repack(GF.KQuant(_t(blocks, dev), GF.GGML_Q6_K, K))
    out = _out(dev, M, N, epi, base)
    xs = torch.zeros(K // 256, M, 16, dtype=torch.int8, device=dev)
    KW4.gemm(_t(xq, dev), _t(a, dev), xs, w, out, _n(live, dev), epi=epi, kernel=kernel)
    torch.cuda.synchronize()
    _check(out, want, live, epi)


@pytest.mark.parametrize("case", range(8))
def test_mxfp4_random(dev, case):
    from prism_amd import mxfp4 as MX
    g = rng(5000 + case + BASE)
    M, live, N, K, _ = _draw(g, 128, 4096)
    kernel = str(g.choice(["tile"] + (["decode"] if M <= 64 else []) + (["split"] if M <= 16 else [])))
    w = weights_f32(N, K, seed=case + 11 + BASE)
    x = acts_bf16(M, K, seed=case + 12 + BASE)
    mw = MX.pack(_t(w, dev), "ocp")
    aq = torch.empty(M, K, dtype=torch.uint8, device=dev)
    asc = torch.empty(M, K // 32, dtype=torch.uint8, device=dev)
    MX.quantize_act_fp8(_t(x.view(np.int16), dev).view(torch.bfloat16), aq, asc)
    out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    MX.gemm(aq, asc, mw, out, _n(live, dev), kernel=kernel)
    torch.cuda.synchronize()
    wq, ws = (t.cpu().numpy() for t in MX.to_rows(mw))
    y64, yabs = O.mx_gemm(aq.cpu().numpy()[:live], asc.cpu().numpy()[:live], wq, ws)
    got = out.float().cpu().numpy()[:live].astype(np.float64)
    assert (np.abs(got - y64) <= 2.0 ** -8 * np.abs(y64) + MX_ACC_REL * yabs + 1e-30).all()
    assert (out.view(torch.int16).cpu().numpy()[live:] == 7).all()
