"""GPU parity of the per-token activation quantizer and the Q8_0 / per-channel W8A8 GEMM against the CPU oracle.

Bit-exact throughout: int8 values and fp32 scales of the quantizer; the int32 block sums (checked through outputs
whose fp32 arithmetic is exact); bf16 outputs and fp32 residual adds of every kernel (decode and tile), for the
benchmark's config 0 (M = 16, K = N = 4096) and ragged / live-row / odd-K cases, as the reference's
tests/test_cuda_gemm.py checks every kernel config against one set of bits."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, half_integer_rows, q8_weights, rng

pytestmark = pytest.mark.gpu


def _t(x, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t if dtype is None else t.view(dtype)


def _live(n, dev):
    return torch.tensor([n], dtype=torch.int32, device=dev)


@pytest.mark.parametrize("M,K,live", [(16, 4096, 16), (5, 5120, 3), (33, 17408, 33), (1, 256, 1), (64, 128, 50)])
def test_rows_q8_bit_exact(dev, M, K, live):
    from prism_amd import quant as KQ
    x = acts_bf16(M, K, seed=M * 7 + K)
    if M > 2:
        x[1] = 0
        x[2, 3] = O.bf16_bits(np.array([77.0], np.float32))[0]
    xd = _t(x, dev, torch.bfloat16)
    q = torch.full((M, K), 99, dtype=torch.int8, device=dev)
    s = torch.full((M,), -1.0, dtype=torch.float32, device=dev)
    KQ.rows_q8(xd, None, q, s, _live(live, dev), M)
    rq, rs = O.quant_rows_i8(x, live=live)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy()[:live], rq[:live])
    assert np.array_equal(s.cpu().numpy()[:live], rs[:live])
    assert (q[live:] == 99).all() and (s[live:] == -1).all()          # rows >= live untouched
    inv = (rng(K).random(K).astype(np.float32) + 0.5)
    KQ.rows_q8(xd, _t(inv, dev), q, s, _live(live, dev), M)
    rq, rs = O.quant_rows_i8(x, inv_s=inv, live=live)
    assert np.array_equal(q.cpu().numpy()[:live], rq[:live]) and np.array_equal(s.cpu().numpy()[:live], rs[:live])


def test_rows_q8_half_integers(dev):
    """Quotients on and beside half-integers (exact ties at scales 1 and 2^-5): the quantizer's reciprocal product
    falls back to the exact division there, and the bits stay the oracle's RN(y / s) rounded to even."""
    from prism_amd import quant as KQ
    x = half_integer_rows(1024)
    M, K = x.shape
    q = torch.zeros((M, K), dtype=torch.int8, device=dev)
    s = torch.zeros((M,), dtype=torch.float32, device=dev)
    KQ.rows_q8(_t(x, dev, torch.bfloat16), None, q, s, _live(M, dev), M)
    rq, rs = O.quant_rows_i8(x, live=M)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)
    assert (np.abs(rq[0, 1:].astype(np.int32)) % 2 == 0).all()       # row 0: every tie went to the even neighbour
    q2, s2 = KQ.quant_rows(_t(x, dev, torch.bfloat16), 32)
    rq2, rs2 = O.quant_rows_groups(x, 32)
    assert np.array_equal(q2.cpu().numpy(), rq2) and np.array_equal(s2.cpu().numpy(), rs2)


@pytest.mark.parametrize("gk", [32, 64, 256, 1024, 96])
def test_quant_rows_groups_bit_exact(dev, gk):
    from prism_amd import quant as KQ
    K = 3072 if gk == 96 else 4096
    x = acts_bf16(7, K, seed=gk)
    q, s = KQ.quant_rows(_t(x, dev, torch.bfloat16), gk)
    rq, rs = O.quant_rows_groups(x, gk)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)


def _gemm(dev, a, s, qs, d, gk, epi, kernel, live=None, out0=None, ldo=None, as_group=False):
    from prism_amd import w8a8 as KW
    M, K = a.shape
    N = qs.shape[0]
    live = M if live is None else live
    ad, wd = _t(a, dev), _t(qs, dev)
    sd = _t(s, dev)
    wsd = _t(d, dev, torch.float16) if d.dtype == np.uint16 else _t(d, dev)
    ldo = N if ldo is None else ldo
    if epi == 0:
        out = torch.full((M, ldo), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    else:
        out = _t(out0, dev).clone()
    KW.gemm(ad, sd, wd, wsd, out, _live(live, dev), gk, epi=epi, kernel=kernel)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kernel", ["decode", "tile"])
def test_config0_bit_exact(dev, kernel):
    """Benchmark config 0: M = 16, K = N = 4096, Q8_0 gk = 32, per-token scales, bf16 out."""
    qs, d = q8_weights(4096, 4096, seed=0)
    a, s = O.quant_rows_i8(acts_bf16(16, 4096, seed=100))
    want = O.w8a8_gemm(a, s, qs, d, 32, epi=0)
    got = _gemm(dev, a, s, qs, d, 32, 0, kernel)
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), want)


CASES = [  # (M, N, K, live)
    (1, 16, 32, 1), (3, 48, 96, 2), (16, 256, 512, 16), (17, 64, 4096, 17), (33, 128, 1024, 20), (64, 80, 2048, 64),
    (100, 272, 640, 77), (130, 256, 1024, 130), (256, 384, 5120, 256),
]


@pytest.mark.parametrize("M,N,K,live", CASES)
def test_gemm_cases_bit_exact(dev, M, N, K, live):
    qs, d = q8_weights(N, K, seed=N + K)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=M + K))
    want0 = O.w8a8_gemm(a, s, qs, d, 32, epi=0, live=live)
    base = rng(M * N).standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm(a, s, qs, d, 32, epi=1, out=base.copy(), live=live)
    kernels = ["tile"] + (["decode"] if M <= 64 else [])
    for kernel in kernels:
        got0 = _gemm(dev, a, s, qs, d, 32, 0, kernel, live=live).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got0[:live], want0[:live]), kernel
        assert (got0[live:] == 7).all(), kernel                       # rows >= live untouched
        got1 = _gemm(dev, a, s, qs, d, 32, 1, kernel, live=live, out0=base).cpu().numpy()
        assert np.array_equal(got1, want1), kernel
    # fp32 weight scales (the reference's w_s) give the same bits
    dfl = d.view(np.float16).astype(np.float32)
    got = _gemm(dev, a, s, qs, dfl, 32, 0, "tile", live=live).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got[:live], want0[:live])


@pytest.mark.parametrize("kernel", ["decode", "tile"])
def test_strided_out_and_per_group_activation_scales(dev, kernel):
    M, N, K = 24, 96, 768
    qs, d = q8_weights(N, K, seed=5)
    x = acts_bf16(M, K, seed=6)
    a, s = O.quant_rows_groups(x, 32)                       # one scale per (row, 32 inputs)
    want = O.w8a8_gemm(a, s, qs, d, 32, epi=0)
    got = _gemm(dev, a, s, qs, d, 32, 0, kernel, ldo=N + 32)
    g = got.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(g[:, :N], want) and (g[:, N:] == 7).all()


def test_int32_block_sums_exact(dev):
    """With unit scales the fp32 arithmetic is exact, so the output is the int32 sum itself: K = 32 gives one
    block's sum, gk = K the whole-row sum (|P| < 2^24)."""
    g = rng(3)
    for K, gk in ((32, 32), (1024, 1024), (64, 32)):
        a = g.integers(-127, 128, (40, K), dtype=np.int8)
        w = g.integers(-127, 128, (64, K), dtype=np.int8)
        ones_a = np.ones(40, np.float32)
        ones_w = np.ones((64, K // gk), np.float32)
        P = a.astype(np.int64) @ w.astype(np.int64).T
        for kernel in (["tile", "decode"] if gk == 32 else ["tile"]):
            got = _gemm(dev, a, ones_a, w, ones_w, gk, 1, kernel, out0=np.zeros((40, 64), np.float32)).cpu().numpy()
            assert np.array_equal(got.astype(np.int64), P), (K, gk, kernel)


@pytest.mark.parametrize("M,N,K,live", [(16, 128, 4096, 16), (200, 256, 5120, 200), (64, 64, 256, 64),
                                         (300, 528, 1024, 290), (513, 272, 2048, 513), (1, 64, 128, 1), (33, 48, 5120, 30),
                                         (64, 272, 17408, 64)])
def test_per_channel_gk_equals_k(dev, M, N, K, live):
    """gk = K (the engine's per-channel weights): one epilogue per output, bf16 and residual-add epilogues, live rows,
    ragged tiles in both directions, fp32 and fp16 weight scales."""
    g = rng(K + M)
    a = g.integers(-127, 128, (M, K), dtype=np.int8)
    w = g.integers(-127, 128, (N, K), dtype=np.int8)
    sa = (g.random(M) * 1e-2).astype(np.float32)
    sw = (g.random((N, 1)) * 1e-3).astype(np.float32)
    want = O.w8a8_gemm(a, sa, w, sw, K, epi=0, live=live)
    base = g.standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm(a, sa, w, sw, K, epi=1, out=base.copy(), live=live)
    sw16 = sw.astype(np.float16)
    want16 = O.w8a8_gemm(a, sa, w, sw16.astype(np.float32), K, epi=0, live=live)
    for kernel in ("tile", "decode"):                  # decode: 64 rows per workgroup, grid rows beyond
        got = _gemm(dev, a, sa, w, sw, K, 0, kernel, live=live).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got[:live], want[:live]), kernel
        assert (got[live:] == 7).all(), kernel
        got1 = _gemm(dev, a, sa, w, sw, K, 1, kernel, live=live, out0=base).cpu().numpy()
        assert np.array_equal(got1, want1), kernel
        got16 = _gemm(dev, a, sa, w, sw16, K, 0, kernel, live=live).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got16[:live], want16[:live]), kernel
    # the packed per-channel layout (weight_from_q8's gk = K operand): same bits from both kernels
    from prism_amd import w8a8 as KW
    pw = KW.pack_i8(_t(w, dev), _t(sw, dev))
    for kernel in ("tile", "decode"):
        out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
        KW.gemm(_t(a, dev), _t(sa, dev), pw, None, out, _live(live, dev), K, epi=0, kernel=kernel)
        o1 = _t(base, dev).clone()
        KW.gemm(_t(a, dev), _t(sa, dev), pw, None, o1, _live(live, dev), K, epi=1, kernel=kernel)
        torch.cuda.synchronize()
        got = out.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got[:live], want[:live]), ("packed", kernel)
        assert np.array_equal(o1.cpu().numpy(), want1), ("packed", kernel)


@pytest.mark.parametrize("K", [64, 192, 320, 384, 448, 832])
def test_per_channel_packed_stage_counts(dev, K):
    """The packed per-channel tile kernel walks K in 64-input stages, unrolled by six with the register rings indexed
    by stage mod 6 and the loads two stages ahead clamped at the end: stage counts 1, 3, 5, 6, 7 and 13, with ragged
    rows and columns (528 = 2 x 256 + 16) and live rows, both epilogues, bit-exact against the oracle."""
    from prism_amd import w8a8 as KW
    M, N, live = 150, 528, 140
    g = rng(K + 77)
    a = g.integers(-127, 128, (M, K), dtype=np.int8)
    w = g.integers(-127, 128, (N, K), dtype=np.int8)
    sa = (g.random(M) * 1e-2).astype(np.float32)
    sw = (g.random((N, 1)) * 1e-3).astype(np.float32)
    base = g.standard_normal((M, N)).astype(np.float32)
    want = O.w8a8_gemm(a, sa, w, sw, K, epi=0, live=live)
    want1 = O.w8a8_gemm(a, sa, w, sw, K, epi=1, out=base.copy(), live=live)
    pw = KW.pack_i8(_t(w, dev), _t(sw, dev))
    out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    KW.gemm(_t(a, dev), _t(sa, dev), pw, None, out, _live(live, dev), K, epi=0, kernel="tile")
    o1 = _t(base, dev).clone()
    KW.gemm(_t(a, dev), _t(sa, dev), pw, None, o1, _live(live, dev), K, epi=1, kernel="tile")
    torch.cuda.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got[:live], want[:live]) and (got[live:] == 7).all()
    assert np.array_equal(o1.cpu().numpy(), want1)
    # row-major int8 weights (prism_w8a8_gemm, the LDS tile kernel) at the same stage counts
    got = _gemm(dev, a, sa, w, sw, K, 0, "tile", live=live).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got[:live], want[:live]) and (got[live:] == 7).all()
    assert np.array_equal(_gemm(dev, a, sa, w, sw, K, 1, "tile", live=live, out0=base).cpu().numpy(), want1)


def test_pack_i8_layout(dev):
    """prism_i8_pack: lane slot l of chunk (t, j) holds row 16 t + l % 16, inputs 64 j + 16 q .. + 15 (q = l / 16),
    checked over the whole tensor against a numpy reshape."""
    from prism_amd import w8a8 as KW
    N, K = 32, 256
    w = rng(4).integers(-127, 128, (N, K), dtype=np.int8)
    pw = KW.pack_i8(_t(w, dev), torch.ones(N, device=dev))
    torch.cuda.synchronize()
    want = w.reshape(N // 16, 16, K // 64, 4, 16).transpose(0, 2, 3, 1, 4).reshape(N // 16, K // 64, 64, 16)
    assert np.array_equal(pw.qt.cpu().numpy(), want)


def test_repeat_runs_identical(dev):
    qs, d = q8_weights(512, 2048, seed=9)
    a, s = O.quant_rows_i8(acts_bf16(48, 2048, seed=10))
    outs = [_gemm(dev, a, s, qs, d, 32, 0, k).view(torch.int16).cpu() for k in ("decode", "tile", "decode", "tile")]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_bad_arguments_raise(dev):
    from prism_amd import w8a8 as KW
    from prism_amd._lib import PrismError
    a = torch.zeros(4, 48, dtype=torch.int8, device=dev)       # K = 48: not a multiple of 32
    w = torch.zeros(16, 48, dtype=torch.int8, device=dev)
    with pytest.raises((PrismError, ValueError)):
        KW.gemm(a, torch.ones(4, device=dev), w, torch.ones(16, 1, device=dev), torch.empty(4, 16, dtype=torch.bfloat16,
                device=dev), _live(4, dev), 48)
    with pytest.raises(NotImplementedError):
        KW.gemm(a, torch.ones(4, device=dev), w, torch.ones(16, 1, device=dev), torch.empty(4, 16, dtype=torch.bfloat16,
                device=dev), _live(4, dev), 48, epi=3)
    with pytest.raises(ValueError):            # epilogue 2 needs int8 out [M, N / 2] and the per-tile scales
        KW.gemm(a, torch.ones(4, device=dev), w, torch.ones(16, 1, device=dev), torch.empty(4, 16, dtype=torch.bfloat16,
                device=dev), _live(4, dev), 48, epi=2)


# ------------------------------------------------------------------------------------------------ packed layout
def _np_pack(qs, d):
    N, K = qs.shape
    r = qs.reshape(N // 16, 16, K // 64, 2, 4, 8)          # [nt, row, pair, half, q, 8]
    qt = r.transpose(0, 2, 4, 1, 3, 5).reshape(N // 16, K // 64, 64, 16)
    dt = d.reshape(N // 16, 16, K // 64, 2).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(qt), np.ascontiguousarray(dt)


def test_pack_q8_layout(dev):
    from prism_amd import w8a8 as KW
    qs, d = q8_weights(64, 512, seed=31)
    p = KW.pack_q8(_t(qs, dev), _t(d, dev, torch.float16))
    torch.cuda.synchronize()
    qt, dt = _np_pack(qs, d)
    assert np.array_equal(p.qt.cpu().numpy(), qt)
    assert np.array_equal(p.dt.view(torch.int16).cpu().numpy().view(np.uint16), dt)


def _packed_gemm(dev, a, s, qs, d, epi, kernel, live=None, out0=None, ldo=None):
    from prism_amd import w8a8 as KW
    M, K = a.shape
    N = qs.shape[0]
    live = M if live is None else live
    pw = KW.pack_q8(_t(qs, dev), _t(d, dev, torch.float16))
    ldo = N if ldo is None else ldo
    if epi == 0:
        out = torch.full((M, ldo), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    else:
        out = _t(out0, dev).clone()
    KW.gemm(_t(a, dev), _t(s, dev), pw, None, out, _live(live, dev), 32, epi=epi, kernel=kernel)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kernel", ["decode", "mid", "tile"])
def test_packed_config0_bit_exact(dev, kernel):
    qs, d = q8_weights(4096, 4096, seed=0)
    a, s = O.quant_rows_i8(acts_bf16(16, 4096, seed=100))
    want = O.w8a8_gemm(a, s, qs, d, 32, epi=0)
    got = _packed_gemm(dev, a, s, qs, d, 0, kernel)
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), want)


PCASES = [  # (M, N, K, live)
    (1, 16, 128, 1), (2, 48, 384, 2), (4, 256, 5120, 3), (7, 64, 1024, 7), (16, 128, 4096, 16), (17, 64, 640, 9),
    (33, 96, 1280, 33), (64, 32, 2048, 60), (100, 272, 640, 77), (256, 384, 5120, 256), (130, 128, 17408, 129),
]


@pytest.mark.parametrize("M,N,K,live", PCASES)
def test_packed_cases_bit_exact(dev, M, N, K, live):
    qs, d = q8_weights(N, K, seed=N + 3 * K)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=M + 5 * K))
    want0 = O.w8a8_gemm(a, s, qs, d, 32, epi=0, live=live)
    base = rng(M * N + 1).standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm(a, s, qs, d, 32, epi=1, out=base.copy(), live=live)
    for kernel in ["tile", "mid"] + (["decode"] if M <= 64 else []):     # mid: any M
        got0 = _packed_gemm(dev, a, s, qs, d, 0, kernel, live=live).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got0[:live], want0[:live]), kernel
        assert (got0[live:] == 7).all(), kernel
        got1 = _packed_gemm(dev, a, s, qs, d, 1, kernel, live=live, out0=base).cpu().numpy()
        assert np.array_equal(got1, want1), kernel


@pytest.mark.parametrize("M,N,K,live", [(1, 16, 128, 1), (33, 96, 1280, 33), (130, 272, 640, 100),
                                         (256, 384, 5120, 256), (300, 528, 2048, 290)])
def test_packed_reassoc_bit_exact(dev, M, N, K, live):
    """The reassociated prefill kernel ("reassoc", not the reference's order) equals the oracle's restatement of its
    order bit for bit, in both epilogues and with live rows."""
    qs, d = q8_weights(N, K, seed=N + 7 * K)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=M + 9 * K))
    want0 = O.w8a8_gemm_reassoc(a, s, qs, d, 32, epi=0, live=live)
    base = rng(M * N + 3).standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm_reassoc(a, s, qs, d, 32, epi=1, out=base.copy(), live=live)
    got0 = _packed_gemm(dev, a, s, qs, d, 0, "reassoc", live=live).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got0[:live], want0[:live]) and (got0[live:] == 7).all()
    got1 = _packed_gemm(dev, a, s, qs, d, 1, "reassoc", live=live, out0=base).cpu().numpy()
    assert np.array_equal(got1, want1)


def test_reassoc_only_for_packed_q8(dev):
    from prism_amd import w8a8 as KW
    a = torch.zeros(4, 128, dtype=torch.int8, device=dev)
    w = torch.zeros(16, 128, dtype=torch.int8, device=dev)
    out = torch.empty(4, 16, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        KW.gemm(a, torch.ones(4, device=dev), w, torch.ones(16, 4, device=dev), out, _live(4, dev), 32,
                kernel="reassoc")
    pw = KW.pack_i8(w, torch.ones(16, device=dev))
    with pytest.raises(ValueError):
        KW.gemm(a, torch.ones(4, device=dev), pw, None, out, _live(4, dev), 128, kernel="reassoc")


SCASES = [  # (M, N, K, live): tiles below, at and above the 256-workgroup grid; ragged shares of a tile
    (1, 16, 128, 1), (3, 80, 640, 2), (4, 4096, 1024, 4), (16, 4112, 256, 16), (9, 5120, 5120, 7),
    (16, 5120, 384, 12), (5, 8192, 2048, 5), (2, 27648, 640, 2), (16, 1360, 17408, 16),
]


@pytest.mark.parametrize("M,N,K,live", SCASES)
def test_packed_stream_bit_exact(dev, M, N, K, live):
    """The balanced decode kernel ("stream"): a tile split between two workgroups gets its running sums handed over,
    so every output equals the oracle bit for bit, in both epilogues, on repeated launches, and the workspace is left
    zeroed for the next launch."""
    from prism_amd import w8a8 as KW
    qs, d = q8_weights(N, K, seed=N + 11 * K)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=M + 13 * K))
    want0 = O.w8a8_gemm(a, s, qs, d, 32, epi=0, live=live, nthreads=16)
    base = rng(M * N + 5).standard_normal((M, N)).astype(np.float32)
    want1 = O.w8a8_gemm(a, s, qs, d, 32, epi=1, out=base.copy(), live=live, nthreads=16)
    for rep in range(2):
        got0 = _packed_gemm(dev, a, s, qs, d, 0, "stream", live=live).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got0[:live], want0[:live]), rep
        assert (got0[live:] == 7).all(), rep
        got1 = _packed_gemm(dev, a, s, qs, d, 1, "stream", live=live, out0=base).cpu().numpy()
        assert np.array_equal(got1, want1), rep
    ws = KW.workspace(dev)[:KW.Q8_HANDOFF_BYTES]       # the handoff words (the prefill's panel copy follows them)
    torch.cuda.synchronize()
    assert int(ws.count_nonzero()) == 0
