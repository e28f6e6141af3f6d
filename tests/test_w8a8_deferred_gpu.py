"""GPU parity of the deferred split-K residual add (kernels/w8a8.py:200-204 with kernels/quant.py:129-171, 418-457):
the split GEMM's slots add up to the exact int32 sums (numpy brute force), and the residual finished by quant.fold or
quant.norm_q8 has the bits of the unsplit epilogue-1 product (this build's own kernel and the CPU oracle), for every
split count, live rows, fp16 and fp32 weight scales, and activation scales that are the norm's own output."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import rng

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _n(v, dev):
    return torch.tensor([v], dtype=torch.int32, device=dev)


def _case(dev, M, N, K, seed, ws16=False):
    from prism_amd import w8a8 as KW
    g = rng(seed)
    a = g.integers(-127, 128, (M, K)).astype(np.int8)
    w = g.integers(-127, 128, (N, K)).astype(np.int8)
    sa = (g.random(M) * 0.02).astype(np.float32)
    sw = (g.random(N) * 0.01).astype(np.float16 if ws16 else np.float32)
    h = (g.standard_normal((M, N)) * 3).astype(np.float32)
    pw = KW.pack_i8(_t(w, dev), _t(sw, dev))
    return a, w, sa, sw, h, pw


@pytest.mark.parametrize("M,N,K,split", [(1, 5120, 5120, 4), (4, 512, 17408, 3), (16, 1024, 2048, 2),
                                         (64, 256, 4096, 16), (80, 128, 1024, 5), (3, 48, 128, 2)])
def test_split_slots_sum_to_exact_products(dev, M, N, K, split):
    from prism_amd import _lib as L
    a, w, _, _, _, pw = _case(dev, M, N, K, M + N + K)
    live = max(1, M - 1)
    slots = torch.full((split, M + 2, N), 7, dtype=torch.int32, device=dev)
    at = _t(a, dev)
    L.call("prism_w8a8_pc_packed_gemm_split", L.ptr(at), L.ptr(pw.qt), L.ptr(slots), slots.stride(0),
           slots.stride(1), L.ptr(_n(live, dev)), M, N, K, split, L.stream_of(at))
    torch.cuda.synchronize()
    got = slots.cpu().numpy().astype(np.int64)
    P = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(got[:, :live].sum(0), P[:live])
    KP = K // 64
    for z in range(split):                                 # part z covers its own chunks only
        c0, c1 = KP * z // split * 64, KP * (z + 1) // split * 64
        Pz = a[:live, c0:c1].astype(np.int64) @ w[:, c0:c1].astype(np.int64).T
        assert np.array_equal(got[z, :live], Pz)
    assert (got[:, live:] == 7).all()


@pytest.mark.parametrize("M,N,K,ws16", [(1, 5120, 5120, False), (4, 5120, 17408, True), (16, 2048, 5120, False),
                                        (64, 1024, 6144, True), (7, 96, 2048, False)])
def test_fold_matches_unsplit_product(dev, M, N, K, ws16, monkeypatch):
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    monkeypatch.setattr(KW, "defer_split", lambda M_, N_, K_, S_: min(S_, 3))
    a, w, sa, sw, h, pw = _case(dev, M, N, K, 3 * M + N + K, ws16)
    at, st = _t(a, dev), _t(sa, dev)
    n = _n(M, dev)
    ref = _t(h, dev)
    assert KW.gemm(at, st, pw, None, ref, n, K, epi=1) is None
    slots = torch.zeros(4, M, N, dtype=torch.int32, device=dev)
    hd = _t(h, dev)
    d = KW.gemm(at, st, pw, None, hd, n, K, epi=1, slots=slots)
    assert isinstance(d, KW.Deferred) and d.n == 3
    torch.cuda.synchronize()
    assert np.array_equal(hd.cpu().numpy(), h)                # the residual waits for the reader
    KQ.fold(hd, None, d, n, M)
    torch.cuda.synchronize()
    want = O.w8a8_gemm(a, sa, w, (sw.view(np.uint16) if ws16 else sw).reshape(N, 1), K, epi=1, out=h.copy())
    assert np.array_equal(ref.cpu().numpy().view(np.int32), want.view(np.int32))
    assert np.array_equal(hd.cpu().numpy().view(np.int32), want.view(np.int32))


@pytest.mark.parametrize("M,HID,K,live,alias", [(1, 5120, 17408, 1, False), (16, 5120, 5120, 13, True),
                                                (64, 2048, 6144, 64, False), (5, 1024, 2048, 5, True)])
def test_norm_q8_finishes_the_deferred_add(dev, M, HID, K, live, alias, monkeypatch):
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    monkeypatch.setattr(KW, "defer_split", lambda M_, N_, K_, S_: min(S_, 1 + M_ % 3 + 1))
    a, w, sa, sw, h, pw = _case(dev, M, HID, K, M + HID + K + 1)
    g = rng(HID + live)
    nw = (0.5 + g.random(HID)).astype(np.float32)
    at = _t(a, dev)
    n = _n(live, dev)
    slots = torch.zeros(3, M, HID, dtype=torch.int32, device=dev)
    hd = _t(h, dev)
    q = torch.full((M, HID), 5, dtype=torch.int8, device=dev)
    s = _t(sa, dev) if alias else torch.zeros(M, dtype=torch.float32, device=dev)
    st = s if alias else _t(sa, dev)                        # alias: the projection's scales are the norm's output s
    d = KW.gemm(at, st, pw, None, hd, n, K, epi=1, slots=slots)
    assert isinstance(d, KW.Deferred)
    KQ.norm_q8(hd, _t(nw, dev), q, s, n, M, 1e-6, pending=d)
    torch.cuda.synchronize()
    hf = O.fold_parts(h.copy(), (a.astype(np.int64) @ w.astype(np.int64).T)[None].astype(np.int32), sa, sw,
                      live=live)
    assert np.array_equal(hd.cpu().numpy().view(np.int32), hf.view(np.int32))
    rq, rs = O.norm_quant(hf, nw, 1e-6, "q8", live=live)
    assert np.array_equal(q.cpu().numpy()[:live], rq[:live]) and np.array_equal(s.cpu().numpy()[:live], rs[:live])
    assert (q.cpu().numpy()[live:] == 5).all()


def test_deferral_policy(dev):
    """The measured rule: long K at 32-64 rows defers (three parts for a 5120-wide projection), everything else runs
    unsplit and returns None with the residual updated."""
    from prism_amd import w8a8 as KW
    assert KW.defer_split(64, 5120, 17408, 4) == 3 and KW.defer_split(32, 5120, 17408, 8) == 3
    assert KW.defer_split(16, 5120, 17408, 4) == 1 and KW.defer_split(64, 5120, 5120, 4) == 1
    assert KW.defer_split(96, 5120, 17408, 4) == 1 and KW.defer_split(64, 5120, 17408, 1) == 1
    a, w, sa, sw, h, pw = _case(dev, 96, 256, 1024, 5)
    slots = torch.zeros(4, 96, 256, dtype=torch.int32, device=dev)
    out = _t(h, dev)
    assert KW.gemm(_t(a, dev), _t(sa, dev), pw, None, out, _n(96, dev), 1024, epi=1, slots=slots) is None
    torch.cuda.synchronize()
    want = O.w8a8_gemm(a, sa, w, sw.reshape(-1, 1), 1024, epi=1, out=h.copy())
    assert np.array_equal(out.cpu().numpy().view(np.int32), want.view(np.int32))


def test_gemm_i32_slots(dev):
    """gemm_i32: the written slots add up to the exact int32 products (numpy int64), one slot where the deferral rule
    does not split."""
    from prism_amd import w8a8 as KW
    for M, K in ((64, 17408), (8, 2048)):
        a, w, sa, sw, h, pw = _case(dev, M, 5120 if M == 64 else 256, K, M + K)
        N = w.shape[0]
        slots = torch.zeros(4, M, N, dtype=torch.int32, device=dev)
        n = KW.gemm_i32(_t(a, dev), _t(sa, dev), pw, pw.ws, slots, _n(M, dev))
        torch.cuda.synchronize()
        assert n == KW.defer_split(M, N, K, 4) or (n == 1 and KW.defer_split(M, N, K, 4) == 1)
        got = slots.cpu().numpy().astype(np.int64)[:n].sum(0)
        assert np.array_equal(got, a.astype(np.int64) @ w.astype(np.int64).T)
