"""Pins the oracle's fused producers (orc_expf, orc_sumsq_fixed, orc_head_sumsq, orc_norm_quant, orc_swiglu_quant,
orc_gated_norm_quant) to things other than their own formulas: float64 exp, math.fsum, hand-built sums whose value
depends on the reduction order, the float64 RMSNorm / SwiGLU / gated-norm values (every quantized output within half
a quantization step of them), closed-form rows, a gated norm that reduces exactly to norm_quant, and the split-sum
layout of the W4A8 operands."""
import math

import numpy as np
import pytest

import oracle as O
from _inputs import rng


def _ulp(v):
    return np.spacing(np.float32(abs(v))).astype(np.float64)


def test_expf_within_two_ulp_of_float64():
    g = rng(31)
    xs = np.concatenate([g.uniform(-87.0, 88.7, 20000), g.uniform(-1, 1, 5000), [0.0, 1.0, -1.0, 88.7, -87.3]])
    for x in xs.astype(np.float32):
        got = O.expf(x)
        want = math.exp(float(x))
        assert abs(got - want) <= 2 * _ulp(want), (x, got, want)
    assert O.expf(0.0) == 1.0
    assert O.expf(100.0) == math.inf and O.expf(-110.0) == 0.0


def test_sumsq_fixed_order_and_bound():
    y = np.zeros(256, np.float32)
    y[0], y[8], y[24] = 4096.0, 1.0, 1.0      # threads 0, 1 and 3: the tree adds 1 + 1 before 2^24, a running sum not
    assert O.sumsq_fixed(y) == 2.0 ** 24 + 2.0
    assert np.float32(np.float32(2.0 ** 24) + np.float32(1.0)) + np.float32(1.0) == 2.0 ** 24
    g = rng(32)
    for K in (256, 5120, 17408):
        v = g.standard_normal(K).astype(np.float32)
        exact = math.fsum(float(t) * float(t) for t in v)
        assert abs(O.sumsq_fixed(v) - exact) <= K * 2.0 ** -23 * exact


def _check_dequant(q, s, y64, back, K):
    """Every quantized value lies within half a step (plus the rounding of y itself) of the float64 value."""
    M = q.shape[0]
    if back == "g256":
        sc = np.repeat(s.T, 256, axis=1)
    else:
        sc = np.repeat(np.asarray(s).reshape(M, 1), K, axis=1)
    err = np.abs(q.astype(np.float64) * sc - y64)
    assert (err <= 0.5 * sc + 4 * 2.0 ** -24 * np.abs(y64) + 1e-30).all()


@pytest.mark.parametrize("back", ["q8", "g256", "grow"])
def test_norm_quant_against_float64(back):
    g = rng(33)
    M, HID, eps = 9, 1024, 1e-6
    h = g.standard_normal((M, HID)).astype(np.float32) * 3
    h[2] = 0.0
    h[3] = 0.5
    w = (0.5 + g.random(HID)).astype(np.float32)
    out = O.norm_quant(h, w, eps, back)
    q, s = out[0], out[1]
    hd = h.astype(np.float64)
    y64 = hd / np.sqrt((hd * hd).mean(1, keepdims=True) + eps) * w
    _check_dequant(q, s, y64, back, HID)
    assert (q[2] == 0).all()                                   # zero row: y = 0, scale 1e-10/127
    if back == "q8":
        assert s[2] == np.float32(1e-10) / np.float32(127)
    if back != "q8":
        xs = out[2]
        S = q.astype(np.int32).reshape(M, HID // 32, 32).sum(-1)
        got = (xs[:, :, :8].astype(np.int32) + 64 * xs[:, :, 8:].astype(np.int32)).transpose(1, 0, 2).reshape(M, -1)
        assert np.array_equal(got, S)
    # gather: output row i from input row rows[i]
    rows = np.array([4, 0, 8], np.int32)
    og = O.norm_quant(h, w, eps, back, rows=rows)
    full = O.norm_quant(h[rows], w, eps, back)
    assert np.array_equal(og[0], full[0]) and np.array_equal(og[1], full[1])


@pytest.mark.parametrize("back", ["q8", "g256", "grow"])
def test_swiglu_quant_against_float64(back):
    g = rng(34)
    M, FF = 7, 768
    gu = (g.standard_normal((M, 2 * FF)) * 4).astype(np.float32)
    gu[0, :4] = [-120.0, 120.0, 0.0, -0.0]
    inv = (0.5 + g.random(FF)).astype(np.float32) if back == "q8" else None
    out = O.swiglu_quant(gu, inv, back)
    q, s = out[0], out[1]
    gd, ud = gu[:, :FF].astype(np.float64), gu[:, FF:].astype(np.float64)
    y64 = gd / (1 + np.exp(-gd)) * ud * (1.0 if inv is None else inv)
    _check_dequant(q, s, y64, back, FF)


def test_head_sumsq_order_and_bound():
    y = np.zeros(128, np.float32)
    y[0], y[8], y[72] = 4096.0, 1.0, 1.0      # chunks 0, 1, 9 of 16: the first halving adds chunk 9 to chunk 1 (1 + 1)
    assert O.head_sumsq(y) == 2.0 ** 24 + 2.0  # before 2^24 joins; a running sum would give 2^24
    g = rng(35)
    for D in (8, 64, 128, 512):
        v = g.standard_normal(D).astype(np.float32)
        exact = math.fsum(float(t) * float(t) for t in v)
        assert abs(O.head_sumsq(v) - exact) <= D * 2.0 ** -23 * exact


@pytest.mark.parametrize("back", ["q8", "g256", "grow"])
def test_gated_norm_quant_against_float64(back):
    g = rng(36)
    M, HV, D, eps = 6, 8, 128, 1e-6
    o = (g.standard_normal((M, HV * D)) * 2).astype(np.float32)
    o[1, :D] = 0.0                                             # a zero head
    z = (g.standard_normal((M, HV * D + 32)) * 3).astype(np.float32)
    w = (0.5 + g.random(D)).astype(np.float32)
    inv = (0.5 + g.random(HV * D)).astype(np.float32) if back == "q8" else None
    out = O.gated_norm_quant(o, z, w, eps, HV, D, inv_s=inv, back=back)
    q, s = out[0], out[1]
    od = o.astype(np.float64).reshape(M, HV, D)
    zd = z[:, :HV * D].astype(np.float64).reshape(M, HV, D)
    y64 = od / np.sqrt((od * od).mean(2, keepdims=True) + eps) * w * (zd / (1 + np.exp(-zd)))
    y64 = y64.reshape(M, HV * D) * (1.0 if inv is None else inv)
    _check_dequant(q, s, y64, back, HV * D)
    assert (q[1, :D] == 0).all()


def test_gated_norm_one_head_with_unit_gate_is_norm_quant():
    """z = 128: exp(-128) underflows, silu(z) = 128 exactly; with one head of D = 128 the chunk-halving sum equals
    the row sum's order, so q is norm_quant's and every scale is 128 x its scale."""
    g = rng(37)
    M, D = 5, 128
    o = (g.standard_normal((M, D)) * 2).astype(np.float32)
    w = (0.5 + g.random(D)).astype(np.float32)
    z = np.full((M, D), 128.0, np.float32)
    assert O.expf(-128.0) == 0.0
    for back in ("q8", "grow"):
        if back == "grow":
            o2, z2, w2 = np.tile(o, 2), np.tile(z, 2), w        # two identical heads: D 128, row 256
            gq = O.gated_norm_quant(o2, z2, w2, 1e-6, 2, D, back=back)
            nq = O.norm_quant(o, w, 1e-6, "q8")
            assert np.array_equal(gq[0], np.tile(nq[0], 2))
            assert np.array_equal(gq[1], nq[1] * np.float32(128.0))
        else:
            gq = O.gated_norm_quant(o, z, w, 1e-6, 1, D, back=back)
            nq = O.norm_quant(o, w, 1e-6, back)
            assert np.array_equal(gq[0], nq[0]) and np.array_equal(gq[1], nq[1] * np.float32(128.0))
