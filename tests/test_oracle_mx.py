"""Pins the oracle's MXFP4 functions (oracle/prism_oracle.c, orc_mx_* / orc_e4m3_*) to things other than their own
formulas: torch's float8_e4m3fn conversion, the reference's exact-grid vector (tests/test_mxfp4.py:32-37), nearest-
value brute force over the e2m1 grid, numpy's float32 log2 / squared-error sums on the same values (the reference
computes its scales and the "mse" choice with numpy, kernels/mxfp4.py:65-85), and numpy float64 matmuls of operands
decoded here independently."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, rng, weights_f32

GRID = np.array([0, .5, 1, 1.5, 2, 3, 4, 6], np.float64)


def _e4m3_lut():
    return torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy().astype(np.float64)


def _decode_e2m1_rows(q):
    v = np.empty((q.shape[0], q.shape[1] * 2), np.float64)
    lut = np.concatenate([GRID, -GRID])
    v[:, 0::2] = lut[q & 15]
    v[:, 1::2] = lut[q >> 4]
    return v


def _scaled(v, s):
    return (v.reshape(v.shape[0], -1, 32) * np.exp2(s.astype(np.float64) - 127)[..., None]).reshape(v.shape)


# ------------------------------------------------------------------------------------------------ e4m3 codes
def test_e4m3_code_matches_torch():
    lut = _e4m3_lut()
    finite = np.array([c for c in range(256) if np.isfinite(lut[c])])
    vals = lut[finite]
    mags = np.unique(np.abs(vals))
    mids = (mags[1:] + mags[:-1]) / 2                          # exact ties between neighbours
    g = rng(11)
    x = np.concatenate([vals, mids, -mids, g.uniform(-448, 448, 4000), g.standard_normal(4000) * 0.01,
                        g.standard_normal(2000) * 2.0 ** -9, [0.0, -0.0, 448.0, -448.0, 2.0 ** -10, -2.0 ** -10]])
    x = x.astype(np.float32)
    want = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([O.e4m3_code(v) for v in x], np.uint8)
    assert np.array_equal(got, want)
    for c in finite:                                           # and the decoder agrees with torch's
        assert O.e4m3_value(int(c)) == lut[c] or (lut[c] == 0 and O.e4m3_value(int(c)) == 0)


# ------------------------------------------------------------------------------------------------ weight pack
def test_pack_exact_grid_vector_survives():
    """tests/test_mxfp4.py:32-37: a row of exact grid values dequantizes to itself."""
    w = np.array([[0.0, 0.5, -0.5, 1.0, -1.0, 1.5, 2.0, 3.0, 4.0, 6.0] * 3 + [0.0, 0.5]], np.float32)
    for mode in ("max", "mse", "ocp"):
        q, s = O.mx_pack(w, mode)
        assert np.array_equal(_scaled(_decode_e2m1_rows(q), s), w.astype(np.float64)), mode


@pytest.mark.parametrize("mode", ["max", "ocp"])
def test_pack_codes_are_nearest_with_the_tie_rule(mode):
    w = weights_f32(64, 512, seed=12)
    ties = np.array([.25, .75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0] * 4, np.float32)   # amax 6: scale 1 in both modes
    w[0, :32] = ties
    w[1, :32] = -ties
    q, s = O.mx_pack(w, mode)
    e = s.astype(np.int64) - 127
    amax = np.abs(w.reshape(64, -1, 32)).max(-1).astype(np.float64)
    if mode == "max":   # smallest power of two with amax / 6 <= 2^e, and numpy's formula on the same values
        r = np.maximum(amax, 1e-30) / 6
        assert (r <= np.exp2(e)).all() and (r > np.exp2(e - 1)).all()
        ref = np.ceil(np.log2(np.maximum(w.reshape(64, -1, 32).__abs__().max(-1), np.float32(1e-30)) / 6.0))
        assert np.array_equal(e, ref.astype(np.int64))
    else:               # 2^(floor(log2 amax) - 2), numpy's log2 on the same values
        ref = np.floor(np.log2(np.maximum(np.abs(w.reshape(64, -1, 32)).max(-1), np.float32(1e-30)))) - 2
        assert np.array_equal(e, ref.astype(np.int64))
    a = np.abs(w.astype(np.float64)) / np.repeat(np.exp2(e), 32, axis=1)
    mag = np.concatenate([q & 7, (q >> 4) & 7], 1).reshape(64, 2, -1).transpose(0, 2, 1).reshape(64, -1)
    d = np.abs(np.minimum(a, 6.0)[..., None] - GRID)            # distance to every grid value
    best = d.min(-1)
    assert np.allclose(d[np.arange(64)[:, None], np.arange(a.shape[1]), mag], best, rtol=0, atol=0)
    # ties: "max" rounds the midpoint toward zero, "ocp" to the even code
    want = [0, 1, 2, 3, 4, 5, 6, 7] if mode == "max" else [0, 2, 2, 4, 4, 6, 6, 7]
    assert list(mag[0, :8]) == want and list(mag[1, :8]) == want
    sign = np.concatenate([q & 8, (q >> 4) & 8], 1).reshape(64, 2, -1).transpose(0, 2, 1).reshape(64, -1)
    assert ((sign != 0) == ((w < 0) & (mag != 0))).all()      # no negative zero in packed weights


def test_pack_mse_matches_numpy_choice():
    """kernels/mxfp4.py:69-84: numpy's float32 squared errors pick between 2^e and 2^(e-1)."""
    w = weights_f32(48, 1024, seed=13)
    w[:, ::7] *= 3.0
    q, s = O.mx_pack(w, "mse")
    q0, s0 = O.mx_pack(w, "max")
    b = w.reshape(48, -1, 32)
    lut = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    errs = []
    for e in (s0.astype(np.int64) - 127, s0.astype(np.int64) - 128):
        sc = np.exp2(e).astype(np.float32)
        a = np.abs(b) / sc[..., None]
        c = ((a > .25).astype(int) + (a > .75) + (a > 1.25) + (a > 1.75) + (a > 2.5) + (a > 3.5) + (a > 5.0))
        c = np.where((b < 0) & (c != 0), c | 8, c)
        v = lut[c] * sc[..., None]
        errs.append(((v - b) ** 2).sum(axis=2))
    pick = np.where(errs[1] < errs[0], s0.astype(np.int64) - 1, s0.astype(np.int64))
    assert np.array_equal(s.astype(np.int64), pick)
    assert (s != s0).any() and (s == s0).any()                   # both outcomes occur


# ------------------------------------------------------------------------------------------------ activations
def test_quant_act_e4m3_matches_torch_mxfp8():
    """tests/quant_sim.py:75-81 in torch: s = 2^(floor(log2 amax) - 8), q = e4m3(clamp(x / s, +-448))."""
    xb = acts_bf16(9, 1024, seed=14)
    xb[0, :32] = 0
    xb[1, 32:64] = O.bf16_bits(np.full(32, 3e-39, np.float32))
    x = O.bf16_to_f32(xb)
    q, s = O.mx_quant_act(x, "e4m3")
    t = torch.from_numpy(x).reshape(9, -1, 32)
    amax = t.abs().amax(-1, keepdim=True).clamp_min(1e-30)
    e = torch.floor(torch.log2(amax)) - 8
    want_q = (t / torch.exp2(e)).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).reshape(9, -1).numpy()
    assert np.array_equal(s.astype(np.int64) - 127, e[..., 0].numpy().astype(np.int64))
    assert np.array_equal(q, want_q)


def test_quant_act_e2m1_rules():
    """kernels/mxfp4.py:110-146: e = ceil(log2(amax / 6)), codes nearest (midpoints toward zero), and the sign bit on
    every negative input (also for code 0, unlike pack)."""
    xb = acts_bf16(7, 512, seed=15)
    xb[2, :32] = O.bf16_bits(np.array([.25, -.25, .75, -1.25, 1.75, 2.5, -3.5, 5.0] * 4, np.float32) * 1)
    xb[2, 31] = O.bf16_bits(np.array([6.0], np.float32))[0]
    x = O.bf16_to_f32(xb)
    inv = (1.0 + rng(16).random(512)).astype(np.float32)
    for scaled in (False, True):
        xs = x * inv if scaled else x
        q, s = O.mx_quant_act(x, "e2m1", inv=inv if scaled else None)
        e = s.astype(np.int64) - 127
        b = xs.reshape(7, -1, 32).astype(np.float64)
        r = np.maximum(np.abs(b).max(-1), 1e-30) / 6
        assert (r <= np.exp2(e)).all() and (r > np.exp2(e - 1)).all()
        a = np.abs(b) / np.exp2(e)[..., None]
        c = ((a > .25).astype(np.uint8) + (a > .75) + (a > 1.25) + (a > 1.75) + (a > 2.5) + (a > 3.5) + (a > 5.0))
        c = (c | np.where(b < 0, 8, 0)).astype(np.uint8).reshape(7, -1)
        assert np.array_equal(q, (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8))
    q, s = O.mx_quant_act(x, "e2m1")
    lo = np.stack([q[2, :16] & 15, q[2, :16] >> 4], 1).reshape(-1)
    assert list(lo[:8]) == [0, 8, 1, 8 | 2, 3, 4, 8 | 5, 6]


def test_quant_act_live_rows():
    x = O.bf16_to_f32(acts_bf16(6, 256, seed=17))
    q, s = O.mx_quant_act(x, "e4m3", live=4)
    q2, s2 = O.mx_quant_act(x[:4], "e4m3")
    assert np.array_equal(q[:4], q2) and (q[4:] == 0).all() and (s[4:] == 0).all()


# ------------------------------------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("fmt", ["e4m3", "e2m1"])
def test_mx_gemm_matches_numpy_float64(fmt):
    M, N, K = 11, 48, 512
    x = O.bf16_to_f32(acts_bf16(M, K, seed=18))
    aq, a_s = O.mx_quant_act(x, fmt)
    wq, ws = O.mx_pack(weights_f32(N, K, seed=19), "ocp")
    y, ya = O.mx_gemm(aq, a_s, wq, ws)
    if fmt == "e4m3":
        av = _e4m3_lut()[aq]
    else:
        av = _decode_e2m1_rows(aq)
    A = _scaled(av, a_s)
    W = _scaled(_decode_e2m1_rows(wq), ws)
    want = A @ W.T
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12 * np.abs(A).max() * np.abs(W).max())
    assert np.allclose(ya, np.abs(A) @ np.abs(W).T, rtol=1e-12)
    # the quantized product tracks the unquantized one (the C4 workload's relative-error budget is 1e-2 per output;
    # here the whole-matrix relative error of MX quantization itself)
    ref = x.astype(np.float64) @ weights_f32(N, K, seed=19).astype(np.float64).T
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 0.2
