"""The headline configurations at their full sizes (benchmark configs 1, 3 and 4), checked through properties that do
not depend on the size: rows sampled from every 128-row tile (and the last row) equal the CPU oracle bit for bit
(MXFP4: within its fp32 bound), and the decode kernel run on a 16-row batch of the same rows gives the same bits as the
full prefill (batch invariance, kernels/w8a8.py:14-17).  Configs 1, 3 and 4 (and config 3's shape on Q6_K) are also
checked whole: every output against the oracle."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import MX_ACC_REL, acts_bf16, rng, weights_f32

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _rows(M, seed):
    g = rng(seed)
    r = [128 * t + int(g.integers(0, 128)) for t in range(M // 128)] + [0, M - 1]
    return np.array(sorted(set(min(x, M - 1) for x in r)), np.int64)


def _bits(out):
    return out.view(torch.int16).cpu().numpy().view(np.uint16)


def test_config1_q8_0_prefill_full_size(dev):
    """Config 1: M = 8192, K = 5120, N = 27648, Q8_0 gk = 32, bf16 out."""
    from prism_amd import gguf_formats as GF
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    M, K, N = 8192, 5120, 27648
    g = torch.Generator(device=dev)
    g.manual_seed(101)
    q8 = GF.quantize_q8_0(torch.randn(N, K, generator=g, device=dev) * 0.02)
    pw, _ = KW.weight_from_q8(q8, 32)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    q = torch.empty(M, K, dtype=torch.int8, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    KQ.rows_q8(x, None, q, s, n, M)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    KW.gemm(q, s, pw, None, out, n, 32, kernel="tile")
    torch.cuda.synchronize()
    rows = _rows(M, 1)
    qs, d = q8.qs.cpu().numpy(), q8.d.view(torch.int16).cpu().numpy().view(np.uint16)
    qa, sa = q.cpu().numpy()[rows], s.cpu().numpy()[rows]
    want = O.w8a8_gemm(qa, sa, qs, d, 32, epi=0, nthreads=16)
    assert np.array_equal(_bits(out)[rows], want)
    # the reassociated kernel at the same size: its own order's bits, and the exact kernel's on nearly every output
    ora = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    KW.gemm(q, s, pw, None, ora, n, 32, kernel="reassoc")
    torch.cuda.synchronize()
    got = _bits(ora)[rows]
    assert np.array_equal(got, O.w8a8_gemm_reassoc(qa, sa, qs, d, 32, epi=0, nthreads=16))
    assert (got == want).mean() > 0.999
    sub = rows[:16]
    o16 = torch.empty(16, N, dtype=torch.bfloat16, device=dev)
    KW.gemm(_t(qa[:16], dev), _t(sa[:16], dev), pw, None, o16, torch.tensor([16], dtype=torch.int32, device=dev),
            32, kernel="decode")
    torch.cuda.synchronize()
    assert np.array_equal(_bits(o16), _bits(out)[sub])


def test_config1_q8_0_prefill_every_row(dev):
    """Config 1 checked whole: the per-token quantizer's q and s on all 8192 rows of bf16 activations against the
    oracle's, then every one of the 8192 x 27648 outputs of the exact prefill kernel, fed the oracle's own quantized
    rows, against the oracle's GEMM (16 threads, about 9 s)."""
    from prism_amd import gguf_formats as GF
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    M, K, N = 8192, 5120, 27648
    g = torch.Generator(device=dev)
    g.manual_seed(102)
    q8 = GF.quantize_q8_0(torch.randn(N, K, generator=g, device=dev) * 0.02)
    pw, _ = KW.weight_from_q8(q8, 32)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    q = torch.empty(M, K, dtype=torch.int8, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    KQ.rows_q8(x, None, q, s, n, M)
    torch.cuda.synchronize()
    qa, sa = O.quant_rows_i8(x.view(torch.int16).cpu().numpy().view(np.uint16), nthreads=16)
    assert np.array_equal(q.cpu().numpy(), qa)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sa.view(np.uint32))
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    KW.gemm(_t(qa, dev), _t(sa, dev), pw, None, out, n, 32, kernel="tile")
    torch.cuda.synchronize()
    qs, d = q8.qs.cpu().numpy(), q8.d.view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.w8a8_gemm(qa, sa, qs, d, 32, epi=0, nthreads=16)
    got = _bits(out)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} outputs differ, first at {bad[:4].tolist()}"


def test_config1_per_channel_prefill_full_size(dev):
    """The per-channel projection (weight_from_q8(q8, K), the engine's production operand) at config 1's shape, the
    per-channel prefill line of the bench: every output bit-exact against the oracle, and the 16-row decode kernel
    on sampled rows gives the same bits."""
    from prism_amd import gguf_formats as GF
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    M, K, N = 8192, 5120, 27648
    g = torch.Generator(device=dev)
    g.manual_seed(103)
    q8 = GF.quantize_q8_0(torch.randn(N, K, generator=g, device=dev) * 0.02)
    pw, _ = KW.weight_from_q8(q8, K)
    del q8
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    q = torch.empty(M, K, dtype=torch.int8, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    KQ.rows_q8(x, None, q, s, n, M)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    KW.gemm(q, s, pw, None, out, n, K, kernel="tile")
    torch.cuda.synchronize()
    rows = _rows(M, 3)
    # the packed chunks back to rows: qt[t, c, l, b] is row 16 t + l % 16, input 64 c + 16 (l / 16) + b
    w = pw.qt.view(N // 16, K // 64, 4, 16, 16).permute(0, 3, 1, 2, 4).reshape(N, K).cpu().numpy()
    sw = pw.ws.float().cpu().numpy().reshape(N, 1)
    qall, sall = q.cpu().numpy(), s.cpu().numpy()
    want = O.w8a8_gemm(qall, sall, w, sw, K, epi=0, nthreads=16)      # every row
    assert np.array_equal(_bits(out), want)
    qa, sa = qall[rows], sall[rows]
    sub = rows[:16]
    o16 = torch.empty(16, N, dtype=torch.bfloat16, device=dev)
    KW.gemm(_t(qa[:16], dev), _t(sa[:16], dev), pw, None, o16, torch.tensor([16], dtype=torch.int32, device=dev),
            K, kernel="decode")
    torch.cuda.synchronize()
    assert np.array_equal(_bits(o16), _bits(out)[sub])


def test_config3_q4k_prefill_full_size(dev):
    """Config 3: M = 2048, K = 5120, N = 13824, Q4_K W4A8, one activation scale per token."""
    from prism_amd import gguf_formats as GF
    from prism_amd import w4a8 as KW4
    M, K, N = 2048, 5120, 13824
    blocks = O.q4k_quantize(weights_f32(N, K, seed=103), nthreads=16)
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=104)), K, nthreads=16)
    w = KW4.repack(GF.KQuant(_t(blocks, dev), GF.GGML_Q4_K, K))
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    KW4.gemm(_t(xq, dev), _t(a, dev), _t(xs, dev), w, out, n, kernel="tile")
    torch.cuda.synchronize()
    rows = _rows(M, 3)
    W = O.q4k_repack(blocks)
    want = O.w4a8_gemm(xq, a[0].copy(), xs, W, nthreads=16)      # every row
    assert np.array_equal(_bits(out), want)
    sub = rows[:16]
    o16 = torch.empty(16, N, dtype=torch.bfloat16, device=dev)
    KW4.gemm(_t(xq[sub], dev), _t(a[:, sub], dev), _t(xs[:, sub], dev), w, o16,
             torch.tensor([16], dtype=torch.int32, device=dev), kernel="decode")
    torch.cuda.synchronize()
    assert np.array_equal(_bits(o16), _bits(out)[sub])


def test_config3_shape_q6k_prefill_full_size(dev):
    """Config 3's shape on Q6_K weights (M = 2048, K = 5120, N = 13824, the bench's c3_q6k prefill line): every
    output bit-exact against the oracle, and the decode kernel's 16 rows equal the prefill's."""
    from prism_amd import gguf_formats as GF
    from prism_amd import w4a8 as KW4
    M, K, N = 2048, 5120, 13824
    blocks = O.q6k_quantize(weights_f32(N, K, seed=106), nthreads=16)
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=107)), K, nthreads=16)
    w = KW4.repack(GF.KQuant(_t(blocks, dev), GF.GGML_Q6_K, K))
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    KW4.gemm(_t(xq, dev), _t(a, dev), _t(xs, dev), w, out, n, kernel="tile")
    torch.cuda.synchronize()
    want = O.w4a8_gemm_q6k(xq, a[0].copy(), O.q6k_repack(blocks), nthreads=16)
    assert np.array_equal(_bits(out), want)
    sub = _rows(M, 6)[:16]
    o16 = torch.empty(16, N, dtype=torch.bfloat16, device=dev)
    KW4.gemm(_t(xq[sub], dev), _t(a[:, sub], dev), _t(xs[:, sub], dev), w, o16,
             torch.tensor([16], dtype=torch.int32, device=dev), kernel="decode")
    torch.cuda.synchronize()
    assert np.array_equal(_bits(o16), _bits(out)[sub])


def test_config4_mxfp4_prefill_full_size(dev):
    """Config 4: M = 4096, K = N = 5120, e2m1 weights (OCP scales) x e4m3 activations; within the fp32 bound of the
    exact value, and the decode kernel's 16 rows equal the tile kernel's."""
    from prism_amd import mxfp4 as MX
    M, K, N = 4096, 5120, 5120
    g = torch.Generator(device=dev)
    g.manual_seed(105)
    mw = MX.pack(torch.randn(N, K, generator=g, device=dev) * 0.02, "ocp")
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    aq = torch.empty(M, K, dtype=torch.uint8, device=dev)
    asc = torch.empty(M, K // 32, dtype=torch.uint8, device=dev)
    MX.quantize_act_fp8(x, aq, asc)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    MX.gemm(aq, asc, mw, out, M, kernel="tile")
    torch.cuda.synchronize()
    rows = _rows(M, 5)
    wq, ws = (t.cpu().numpy() for t in MX.to_rows(mw))
    y64, yabs = O.mx_gemm(aq.cpu().numpy(), asc.cpu().numpy(), wq, ws, nthreads=16)      # every row
    got = out.float().cpu().numpy().astype(np.float64)
    assert (np.abs(got - y64) <= 2.0 ** -8 * np.abs(y64) + MX_ACC_REL * yabs + 1e-30).all()
    sub = rows[:16]
    o16 = torch.empty(16, N, dtype=torch.bfloat16, device=dev)
    MX.gemm(aq[_t(sub, dev)].contiguous(), asc[_t(sub, dev)].contiguous(), mw, o16, 16, kernel="decode")
    torch.cuda.synchronize()
    assert np.array_equal(_bits(o16), _bits(out)[sub])
