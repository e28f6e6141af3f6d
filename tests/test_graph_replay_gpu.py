"""One captured HIP graph serves every batch size: each GEMM family is captured once with a device row count, then
replayed for live in {1, 7, M - 1, M} with the count rewritten on the device between replays.  After every replay
the live rows equal the oracle bit for bit (MXFP4: the same bits as an eager launch, which its own tests bound against
the oracle) and rows >= live keep the sentinel, as the reference's tests/test_cuda_gemm.py:149-169 checks its
captured decode steps.  The quantizer that feeds the projection rides in the same graph."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import MX_ACC_REL, acts_bf16, q8_weights, rng, weights_f32

pytestmark = pytest.mark.gpu

M = 48


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _replay(dev, run, out, n_rows, check, sentinel):
    """Capture run() once; for each live count: write n_rows, reset out, replay, check."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()                                      # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for live in (1, 7, M - 1, M, 7):
        print(f"replay live={live}", flush=True)
        n_rows.fill_(live)
        out.copy_(sentinel)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check(live)
    del g


def test_q8_0_packed_and_quantizer(dev):
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    N, K = 256, 2048
    qs, d = q8_weights(N, K, seed=11)
    pw = KW.pack_q8(_t(qs, dev), _t(d, dev).view(torch.float16))
    xb = acts_bf16(M, K, seed=12)
    x = _t(xb.view(np.int16), dev).view(torch.bfloat16)
    q = torch.zeros(M, K, dtype=torch.int8, device=dev)
    s = torch.zeros(M, dtype=torch.float32, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    rq, rs = O.quant_rows_i8(xb)
    want = O.w8a8_gemm(rq, rs, qs, d, 32, epi=0)
    for kernel in ("auto", "decode", "mid", "tile", "stream"):
        rows = 16 if kernel == "stream" else M          # the balanced decode kernel serves up to 16 rows
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        sentinel = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)

        def run(rows=rows, kernel=kernel, out=out):
            KQ.rows_q8(x, None, q, s, n, M)
            KW.gemm(q[:rows], s[:rows], pw, None, out, n, 32, kernel=kernel)

        def check(live, rows=rows, kernel=kernel, out=out):
            got = _bits(out)
            lv = min(live, rows)
            assert np.array_equal(got[:lv], want[:lv]), (kernel, live)
            assert (got[lv:] == 7).all(), (kernel, live)

        _replay(dev, run, out, n, check, sentinel)


def test_per_channel_packed_and_plain(dev):
    from prism_amd import w8a8 as KW
    N, K = 320, 1536
    g = rng(13)
    w = g.integers(-127, 128, (N, K), dtype=np.int8)
    sw = (g.random(N) * 1e-3).astype(np.float32)
    a = g.integers(-127, 128, (M, K), dtype=np.int8)
    sa = (g.random(M) * 1e-2).astype(np.float32)
    want = O.w8a8_gemm(a, sa, w, sw.reshape(N, 1), K, epi=0)
    ad, sad, n = _t(a, dev), _t(sa, dev), torch.tensor([M], dtype=torch.int32, device=dev)
    pw = KW.pack_i8(_t(w, dev), _t(sw, dev))
    wd, swd = _t(w, dev), _t(sw, dev)
    for name, W, WS, kernel in (("packed", pw, None, "auto"), ("packed", pw, None, "tile"),
                                ("packed", pw, None, "decode"), ("plain", wd, swd, "auto")):
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        sentinel = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)

        def run():
            KW.gemm(ad, sad, W, WS, out, n, K, kernel=kernel)

        def check(live):
            got = _bits(out)
            assert np.array_equal(got[:live], want[:live]), (name, kernel, live)
            assert (got[live:] == 7).all(), (name, kernel, live)

        _replay(dev, run, out, n, check, sentinel)


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_w4a8(dev, kind):
    from prism_amd import gguf_formats as GF
    from prism_amd import quant as KQ
    from prism_amd import w4a8 as KW4
    N, K = 192, 2048
    wf = weights_f32(N, K, seed=14)
    blocks = O.q4k_quantize(wf) if kind == "q4k" else O.q6k_quantize(wf)
    w = KW4.repack(GF.KQuant(_t(blocks, dev), kind, K))
    xb = acts_bf16(M, K, seed=15)
    x = _t(xb.view(np.int16), dev).view(torch.bfloat16)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    rq, ra, rxs = O.quant_rows_g(O.bf16_to_f32(xb), 256)
    want = (O.w4a8_gemm(rq, ra, rxs, O.q4k_repack(blocks)) if kind == "q4k" else
            O.w4a8_gemm_q6k(rq, ra, O.q6k_repack(blocks)))
    kernels = ("auto", "decode", "tile", "stream")
    for kernel in kernels:
        rows = M if kernel in ("auto", "tile") else 16     # the decode / stream kernels serve up to 16 rows
        xq = torch.zeros(rows, K, dtype=torch.int8, device=dev)
        a = torch.zeros(K // 256, rows, dtype=torch.float32, device=dev)
        xs = torch.zeros(K // 256, rows, 16, dtype=torch.int8, device=dev)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        sentinel = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)

        def run(rows=rows, kernel=kernel, xq=xq, a=a, xs=xs, out=out):
            KQ.rows_g(x[:rows], xq, a, xs, n, rows)
            KW4.gemm(xq, a, xs, w, out, n, kernel=kernel)

        def check(live, rows=rows, kernel=kernel, out=out):
            got = _bits(out)
            lv = min(live, rows)
            assert np.array_equal(got[:lv], want[:lv]), (kind, kernel, live)
            assert (got[lv:] == 7).all(), (kind, kernel, live)

        _replay(dev, run, out, n, check, sentinel)


def test_mxfp4(dev):
    from prism_amd import mxfp4 as MX
    N, K = 256, 2048
    mw = MX.pack(_t(weights_f32(N, K, seed=16), dev), "ocp")
    x = _t(acts_bf16(M, K, seed=17).view(np.int16), dev).view(torch.bfloat16)
    aq = torch.zeros(M, K, dtype=torch.uint8, device=dev)
    asc = torch.zeros(M, K // 32, dtype=torch.uint8, device=dev)
    MX.quantize_act_fp8(x, aq, asc)
    ref = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    MX.gemm(aq, asc, mw, ref, M, kernel="tile")
    torch.cuda.synchronize()
    want = _bits(ref)
    wq, ws = (t.cpu().numpy() for t in MX.to_rows(mw))
    y64, yabs = O.mx_gemm(aq.cpu().numpy(), asc.cpu().numpy(), wq, ws)
    got = O.bf16_to_f32(want).astype(np.float64)
    assert (np.abs(got - y64) <= 2.0 ** -8 * np.abs(y64) + MX_ACC_REL * yabs + 1e-30).all()
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    for kernel in ("auto", "decode", "tile"):
        rows = 16 if kernel == "decode" else M
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        sentinel = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)

        def run(rows=rows, kernel=kernel):
            MX.gemm(aq[:rows], asc[:rows], mw, out, n, kernel=kernel)

        def check(live, rows=rows, kernel=kernel):
            g = _bits(out)
            lv = min(live, rows)
            assert np.array_equal(g[:lv], want[:lv]), (kernel, live)
            assert (g[lv:] == 7).all(), (kernel, live)

        _replay(dev, run, out, n, check, sentinel)
