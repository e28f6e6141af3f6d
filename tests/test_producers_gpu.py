"""GPU parity of the fused producers (norm_q8, norm_g, swiglu_q8, swiglu_g, gated_norm_q8, gated_norm_g) against the
CPU oracle, bit for bit: int8 values, scales and split per-32 sums, at the engine's shapes (HID 5120, FF 17408, 48
value heads of 128), with gathered rows, live rows, bf16 and fp32 gate inputs, the smoothing factor, and both
workgroup sizes of the SwiGLU and gated-norm kernels (1024 threads up to 64 rows, 256 beyond)."""
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


@pytest.mark.parametrize("M,HID,live,gather", [(16, 5120, 16, False), (33, 4096, 30, True), (1, 256, 1, False),
                                               (200, 2048, 200, False)])
def test_norm_q8_bit_exact(dev, M, HID, live, gather):
    from prism_amd import quant as KQ
    g = rng(HID + M)
    h = (g.standard_normal((M + 5, HID)) * 2).astype(np.float32)
    h[1] = 0.0
    w = (0.3 + g.random(HID)).astype(np.float32)
    rows = g.permutation(M + 5)[:M].astype(np.int32) if gather else None
    q = torch.full((M, HID), 5, dtype=torch.int8, device=dev)
    s = torch.zeros(M, dtype=torch.float32, device=dev)
    KQ.norm_q8(_t(h, dev), _t(w, dev), q, s, _n(live, dev), M, 1e-6, rows=None if rows is None else _t(rows, dev))
    torch.cuda.synchronize()
    rq, rs = O.norm_quant(h if gather else h[:M], w, 1e-6, "q8", rows=rows, live=live)
    assert np.array_equal(q.cpu().numpy()[:live], rq[:live]) and np.array_equal(s.cpu().numpy()[:live], rs[:live])
    assert (q.cpu().numpy()[live:] == 5).all()


@pytest.mark.parametrize("group", ["g256", "grow"])
def test_norm_g_bit_exact(dev, group):
    from prism_amd import quant as KQ
    M, HID = 24, 5120
    g = rng(7)
    h = (g.standard_normal((M, HID)) * 2).astype(np.float32)
    w = (0.3 + g.random(HID)).astype(np.float32)
    q = torch.zeros(M, HID, dtype=torch.int8, device=dev)
    s = torch.zeros((HID // 256, M) if group == "g256" else (1, M), dtype=torch.float32, device=dev)
    xs = torch.zeros(HID // 256, M, 16, dtype=torch.int8, device=dev)
    KQ.norm_g(_t(h, dev), _t(w, dev), q, s, xs, _n(M, dev), M, 1e-5, group=256 if group == "g256" else HID)
    torch.cuda.synchronize()
    rq, rs, rxs = O.norm_quant(h, w, 1e-5, group)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy().reshape(rs.shape), rs)
    assert np.array_equal(xs.cpu().numpy(), rxs)


@pytest.mark.parametrize("M,FF,live,f32,smooth", [(16, 17408, 16, False, True), (5, 13824, 4, False, False),
                                                  (64, 1024, 64, True, True), (3, 264, 3, False, True),
                                                  (100, 13824, 97, False, True)])
def test_swiglu_q8_bit_exact(dev, M, FF, live, f32, smooth):
    from prism_amd import quant as KQ
    g = rng(FF + M)
    gu = (g.standard_normal((M, 2 * FF)) * 3).astype(np.float32)
    gu[0, :3] = [-120.0, 95.0, 0.0]
    inv = (0.5 + g.random(FF)).astype(np.float32) if smooth else None
    if f32:
        gud = _t(gu, dev)
    else:
        bits = O.bf16_bits(gu)
        gu = O.bf16_to_f32(bits)
        gud = _t(bits.view(np.int16), dev).view(torch.bfloat16)
    q = torch.full((M, FF), 5, dtype=torch.int8, device=dev)
    s = torch.zeros(M, dtype=torch.float32, device=dev)
    KQ.swiglu_q8(gud, None if inv is None else _t(inv, dev), q, s, _n(live, dev), M)
    torch.cuda.synchronize()
    rq, rs = O.swiglu_quant(gu, inv, "q8", live=live)
    assert np.array_equal(q.cpu().numpy()[:live], rq[:live]) and np.array_equal(s.cpu().numpy()[:live], rs[:live])
    assert (q.cpu().numpy()[live:] == 5).all()


@pytest.mark.parametrize("group", ["g256", "grow"])
def test_swiglu_g_bit_exact(dev, group):
    from prism_amd import quant as KQ
    M, FF = 16, 13824
    g = rng(9)
    bits = O.bf16_bits((g.standard_normal((M, 2 * FF)) * 3).astype(np.float32))
    q = torch.zeros(M, FF, dtype=torch.int8, device=dev)
    s = torch.zeros((FF // 256, M) if group == "g256" else (1, M), dtype=torch.float32, device=dev)
    xs = torch.zeros(FF // 256, M, 16, dtype=torch.int8, device=dev)
    KQ.swiglu_g(_t(bits.view(np.int16), dev).view(torch.bfloat16), q, s, xs, _n(M, dev), M,
                group=256 if group == "g256" else FF)
    torch.cuda.synchronize()
    rq, rs, rxs = O.swiglu_quant(O.bf16_to_f32(bits), None, group)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy().reshape(rs.shape), rs)
    assert np.array_equal(xs.cpu().numpy(), rxs)


class _Cfg:
    def __init__(self, hv, d, eps=1e-6):
        self.v_heads, self.gdn_dim, self.eps = hv, d, eps


@pytest.mark.parametrize("M,HV,D,live,f32,smooth", [(16, 48, 128, 13, False, True), (1, 32, 128, 1, False, True),
                                                    (40, 16, 64, 40, True, False), (7, 4, 256, 7, False, True),
                                                    (3, 3, 8, 3, True, True), (80, 48, 128, 77, False, True)])
def test_gated_norm_q8_bit_exact(dev, M, HV, D, live, f32, smooth):
    from prism_amd import quant as KQ
    K, zoff = HV * D, 3 * 128
    g = rng(K + M)
    o = (g.standard_normal((M, HV, D)) * 2).astype(np.float32)
    o[0, 1] = 0.0
    proj = (g.standard_normal((M, zoff + K + 64)) * 3).astype(np.float32)
    proj[0, zoff:zoff + 3] = [-120.0, 95.0, 0.0]
    w = (0.5 + g.random(D)).astype(np.float32)
    inv = (0.5 + g.random(K)).astype(np.float32) if smooth else None
    if f32:
        pd = _t(proj, dev)
    else:
        bits = O.bf16_bits(proj)
        proj = O.bf16_to_f32(bits)
        pd = _t(bits.view(np.int16), dev).view(torch.bfloat16)
    q = torch.full((M, K), 5, dtype=torch.int8, device=dev)
    s = torch.zeros(M, dtype=torch.float32, device=dev)
    KQ.gated_norm_q8(_t(o, dev), pd, zoff, _t(w, dev), None if inv is None else _t(inv, dev), q, s, _n(live, dev), M,
                     _Cfg(HV, D))
    torch.cuda.synchronize()
    rq, rs = O.gated_norm_quant(o.reshape(M, K), proj[:, zoff:], w, 1e-6, HV, D, inv_s=inv, back="q8", live=live)
    assert np.array_equal(q.cpu().numpy()[:live], rq[:live]) and np.array_equal(s.cpu().numpy()[:live], rs[:live])
    assert (q.cpu().numpy()[live:] == 5).all()


@pytest.mark.parametrize("group", ["g256", "grow"])
def test_gated_norm_g_bit_exact(dev, group):
    from prism_amd import quant as KQ
    M, HV, D = 16, 48, 128
    K, zoff = HV * D, 1024
    g = rng(11)
    o = (g.standard_normal((M, HV, D)) * 2).astype(np.float32)
    bits = O.bf16_bits((g.standard_normal((M, zoff + K)) * 3).astype(np.float32))
    w = (0.5 + g.random(D)).astype(np.float32)
    q = torch.zeros(M, K, dtype=torch.int8, device=dev)
    s = torch.zeros((K // 256, M) if group == "g256" else (1, M), dtype=torch.float32, device=dev)
    xs = torch.zeros(K // 256, M, 16, dtype=torch.int8, device=dev)
    KQ.gated_norm_g(_t(o, dev), _t(bits.view(np.int16), dev).view(torch.bfloat16), zoff, _t(w, dev), q, s, xs,
                    _n(M, dev), M, _Cfg(HV, D), group=256 if group == "g256" else K)
    torch.cuda.synchronize()
    rq, rs, rxs = O.gated_norm_quant(o.reshape(M, K), O.bf16_to_f32(bits)[:, zoff:], w, 1e-6, HV, D, back=group)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy().reshape(rs.shape), rs)
    assert np.array_equal(xs.cpu().numpy(), rxs)
