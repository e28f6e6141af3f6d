"""Pins the CPU oracle (oracle/prism_oracle.c) to things other than its own formulas: torch's and numpy's float
conversions, exact rational arithmetic, brute-force integer sums, float64 error bounds, hand-built cases whose
result depends on the order of roundings, and the product package's torch restatement of the weight formats."""
import fractions
import math

import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, q6k_random_blocks, q8_weights, rng, weights_f32

F = fractions.Fraction


# ------------------------------------------------------------------------------------------------ conversions
def _specials():
    v = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e-8, 6e-8, 5.96e-8, 2.98e-8, 3e-8, 6.1e-5, 6.09e-5,
         1e30, -1e30, float("inf"), -float("inf"), 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8]
    return np.array(v, np.float32)


def test_bf16_conversion_matches_torch():
    x = np.concatenate([_specials(), rng(1).standard_normal(20000).astype(np.float32) * 10,
                        rng(2).integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    x = x[~np.isnan(x)]
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got_np = O.bf16_bits(x)
    assert np.array_equal(got_np, want)
    got_c = np.array([O.f32_to_bf16_c(v) for v in x[:3000]], np.uint16)
    assert np.array_equal(got_c, want[:3000])


def test_half_conversion_matches_numpy():
    x = np.concatenate([_specials(), rng(3).standard_normal(5000).astype(np.float32) * 1e-3,
                        rng(4).standard_normal(5000).astype(np.float32) * 3e4,
                        rng(5).standard_normal(3000).astype(np.float32) * 1e-6])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_half_c(v) for v in x], np.uint16)
    assert np.array_equal(got, want)
    every = np.arange(0, 2 ** 16, dtype=np.uint32).astype(np.uint16)
    back = np.array([O.half_to_f32_c(h) for h in every], np.float32)
    ref = every.view(np.float16).astype(np.float32)
    same = (back.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(back) & np.isnan(ref))
    assert same.all()


def _is_correctly_rounded_f32(r, exact):
    r = np.float32(r)
    if not math.isfinite(float(r)):
        return False
    lo, hi = np.nextafter(r, np.float32(-np.inf)), np.nextafter(r, np.float32(np.inf))
    e = abs(F(float(r)) - exact)
    for nb in (lo, hi):
        en = abs(F(float(nb)) - exact)
        if en < e:
            return False
        if en == e and (int(np.float32(nb).view(np.uint32)) & 1) == 0:
            return False                                  # a tie must go to the even neighbour
    return True


def test_fmaf_is_correctly_rounded():
    g = rng(6)
    for _ in range(400):
        a, b, c = (np.float32(v) for v in g.standard_normal(3) * np.array([1e3, 1e-3, 1.0]))
        r = O.fmaf(a, b, c)
        assert _is_correctly_rounded_f32(r, F(float(a)) * F(float(b)) + F(float(c)))
    # a case where fma and mul-then-add differ
    a = b = np.float32(1 + 2 ** -12)
    c = np.float32(-(1 + 2 ** -11))
    assert O.fmaf(a, b, c) == 2.0 ** -24 and np.float32(np.float32(a * b) + c) == 0.0


# ------------------------------------------------------------------------------------------------ Q8_0
def test_q8_0_quantizer_round_trip_and_torch():
    from prism_amd import gguf_formats as GF
    w = weights_f32(64, 512, seed=7)
    w[3, :32] = 0.0                                          # an all-zero block: d = 0, q = 0
    qs, d = O.q8_0_quantize(w)
    df = d.view(np.float16).astype(np.float32)
    deq = (qs.reshape(64, 16, 32).astype(np.float32) * df[..., None]).reshape(64, 512)
    assert np.all(np.abs(deq - w) <= df.repeat(32, 1) * 0.5 * (1 + 2e-3) + 1e-12)
    blk = np.abs(w.reshape(64, 16, 32))
    amax_pos = blk.argmax(-1)
    qa = np.take_along_axis(np.abs(qs.reshape(64, 16, 32)), amax_pos[..., None], -1)[..., 0]
    assert np.all(qa[df > 0] == 127) and np.all(qs[3, :32] == 0) and d[3, 0] == 0
    t = GF.quantize_q8_0(torch.from_numpy(w))
    assert np.array_equal(t.qs.numpy(), qs) and np.array_equal(t.d.view(torch.int16).numpy().view(np.uint16), d)
    raw = GF.q8_0_to_gguf_bytes(t)
    assert raw.shape == (64, 16, 34)
    back = GF.q8_0_from_gguf_bytes(raw, 64, 512)
    assert torch.equal(back.qs, t.qs) and torch.equal(back.d.view(torch.int16), t.d.view(torch.int16))


def test_quant_rows_special_cases():
    x = acts_bf16(6, 256, seed=8)
    x[1] = 0                                                 # zero row
    x[2, 17] = O.bf16_bits(np.array([-300.0], np.float32))[0]
    q, s = O.quant_rows_i8(x)
    xf = O.bf16_to_f32(x)
    assert s[1] == np.float32(np.float32(1e-10) / np.float32(127.0)) and np.all(q[1] == 0)
    assert q[2, 17] == -127
    for m in (0, 2, 3):
        assert np.abs(q[m]).max() == 127
    scale = np.maximum(np.abs(xf).max(1), np.float32(1e-10)).astype(np.float32) / np.float32(127.0)
    assert np.array_equal(s, scale.astype(np.float32))
    want = np.rint(xf / scale[:, None]).astype(np.int8)
    assert np.array_equal(q, want)
    inv = (rng(9).random(256).astype(np.float32) + 0.5)
    q2, s2 = O.quant_rows_i8(x, inv_s=inv)
    y = (xf * inv[None]).astype(np.float32)
    sc2 = np.maximum(np.abs(y).max(1), np.float32(1e-10)).astype(np.float32) / np.float32(127.0)
    assert np.array_equal(s2, sc2) and np.array_equal(q2, np.rint(y / sc2[:, None]).astype(np.int8))
    q3, s3 = O.quant_rows_i8(x, live=4)
    assert np.all(q3[4:] == 0) and np.all(s3[4:] == 0) and np.array_equal(q3[:4], q[:4])


def test_quant_rows_groups():
    x = acts_bf16(5, 512, seed=10)
    for gk in (32, 128, 512):
        q, s = O.quant_rows_groups(x, gk)
        xf = O.bf16_to_f32(x).reshape(5, 512 // gk, gk)
        sc = np.maximum(np.abs(xf).max(-1), np.float32(1e-10)) / np.float32(127.0)
        assert np.array_equal(s, sc.astype(np.float32))
        assert np.array_equal(q, np.rint(xf / sc[..., None]).astype(np.int8).reshape(5, 512))
    q1, s1 = O.quant_rows_groups(x, 512)
    q2, s2 = O.quant_rows_i8(x)
    assert np.array_equal(q1, q2) and np.array_equal(s1[:, 0], s2)


# ------------------------------------------------------------------------------------------------ W8A8
def test_w8a8_block_sums_brute_force():
    a = rng(11).integers(-127, 128, (7, 128), dtype=np.int8)
    w = rng(12).integers(-127, 128, (9, 128), dtype=np.int8)
    P = O.w8a8_block_sums(a, w, 32)
    want = np.einsum("mgk,ngk->mng", a.reshape(7, 4, 32).astype(np.int64), w.reshape(9, 4, 32).astype(np.int64))
    assert np.array_equal(P, want)


def _w8a8_f64(a, sa, w, sw, gk):
    M, K = a.shape
    N, G = w.shape[0], K // gk
    P = np.einsum("mgk,ngk->mng", a.reshape(M, G, gk).astype(np.float64), w.reshape(N, G, gk).astype(np.float64))
    sa2 = sa.astype(np.float64).reshape(M, 1, -1)
    t = P * sa2 * sw.astype(np.float64)[None]
    return t.sum(-1), np.abs(t).sum(-1), G


def test_w8a8_gemm_error_bound_and_epilogues():
    qs, d = q8_weights(48, 1024, seed=13)
    a, s = O.quant_rows_i8(acts_bf16(9, 1024, seed=14))
    exact, mag, G = _w8a8_f64(a, s[:, None], qs, d.view(np.float16).astype(np.float32), 32)
    base = rng(15).standard_normal((9, 48)).astype(np.float32)
    y = O.w8a8_gemm(a, s, qs, d, 32, epi=1, out=np.zeros((9, 48), np.float32))
    u = 2.0 ** -24
    assert np.all(np.abs(y - exact) <= (G + 3) * u * mag + 1e-30)
    r1 = O.w8a8_gemm(a, s, qs, d, 32, epi=1, out=base.copy())
    assert np.array_equal(r1, (base + y).astype(np.float32))           # epi 1 = RN(out + y)
    r0 = O.w8a8_gemm(a, s, qs, d, 32, epi=0)
    assert np.array_equal(r0, O.bf16_bits(y))                          # epi 0 = bf16(y)
    # fp32 weight scales give the same bits as the fp16 ones (the widening is exact)
    r0b = O.w8a8_gemm(a, s, qs, d.view(np.float16).astype(np.float32), 32, epi=0)
    assert np.array_equal(r0, r0b)
    # per-token scale broadcast == per-group scale array holding the same value
    r0c = O.w8a8_gemm(a, np.repeat(s[:, None], 32, 1), qs, d, 32, epi=0)
    assert np.array_equal(r0, r0c)
    # live rows
    r0d = O.w8a8_gemm(a, s, qs, d, 32, epi=0, live=5)
    assert np.array_equal(r0d[:5], r0[:5]) and np.all(r0d[5:] == 0)


def test_w8a8_reassoc_order_replayed_and_bounded():
    """The reassociated order (not the reference's): one element replayed with the pinned fmaf and numpy's fp32
    multiply; every output within the rounding bound of the float64 value; the bf16 results equal the reference
    order's on all but a few outputs in 10^4 and are within 1 bf16 ulp plus the two orders' fp32 bounds of them."""
    M, N, K = 40, 96, 2048
    qs, d = q8_weights(N, K, seed=16)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=17))
    sw = d.view(np.float16).astype(np.float32)
    exact, mag, G = _w8a8_f64(a, s[:, None], qs, sw, 32)
    y = O.w8a8_gemm_reassoc(a, s, qs, d, 32, epi=1, out=np.zeros((M, N), np.float32))
    u = 2.0 ** -24
    assert np.all(np.abs(y - exact) <= (G + 3) * u * mag + 1e-30)
    P = O.w8a8_block_sums(a, qs, 32)
    m, n = 7, 33
    r = np.float32(0)
    for g in range(G):
        r = np.float32(O.fmaf(np.float32(P[m, n, g]), sw[n, g], r))
    assert y[m, n] == np.float32(r * s[m])
    base = rng(18).standard_normal((M, N)).astype(np.float32)
    assert np.array_equal(O.w8a8_gemm_reassoc(a, s, qs, d, 32, epi=1, out=base.copy()), (base + y).astype(np.float32))
    r0 = O.w8a8_gemm_reassoc(a, s, qs, d, 32, epi=0)
    assert np.array_equal(r0, O.bf16_bits(y))
    ref = O.w8a8_gemm(a, s, qs, d, 32, epi=0)
    assert (r0 == ref).mean() > 0.999
    yr, yq = O.bf16_to_f32(ref).astype(np.float64), O.bf16_to_f32(r0).astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(yr), 1e-38))) - 7)
    assert np.all(np.abs(yr - yq) <= ulp + 2 * (G + 3) * u * mag)
    live = O.w8a8_gemm_reassoc(a, s, qs, d, 32, epi=0, live=5)
    assert np.array_equal(live[:5], r0[:5]) and np.all(live[5:] == 0)


def test_w8a8_group_order_is_sequential():
    """Three blocks with terms 2^24, 1, -2^24: in block order the 1 is lost to round-to-even (result 0); any other
    order or an exact sum gives 1."""
    a = np.zeros((1, 96), np.int8)
    w = np.zeros((16, 96), np.int8)
    a[0, 0:32], w[0, 0:32] = 16, 32           # P0 = 16384
    a[0, 32], w[0, 32] = 1, 1                 # P1 = 1
    a[0, 64:96], w[0, 64:96] = 16, -32        # P2 = -16384
    sw = np.ones((16, 3), np.float32)
    sw[0, 0] = sw[0, 2] = 1024.0              # t0 = 2^24, t2 = -2^24
    y = O.w8a8_gemm(a, np.ones(1, np.float32), w, sw.astype(np.float16).view(np.uint16), 32, epi=1,
                    out=np.zeros((1, 16), np.float32))
    assert y[0, 0] == 0.0


def test_w8a8_scale_order_is_activation_then_weight():
    """RN(RN(P * sa) * sw), not RN(P * RN(sa * sw)): find values where the two differ and check the oracle."""
    g = rng(16)
    for _ in range(2000):
        P = int(g.integers(-500000, 500000))
        sa = np.float32(g.random() * 1e-2 + 1e-4)
        sw = np.float16(g.random() * 1e-3 + 1e-5)
        ref = np.float32(np.float32(np.float32(P) * sa) * np.float32(sw))
        alt = np.float32(np.float32(P) * np.float32(sa * np.float32(sw)))
        if ref != alt:
            break
    else:
        pytest.skip("no discriminating case found")
    # build a, w with that block sum: a = [P // 127 ... ] spread over 32 lanes
    a = np.zeros((1, 32), np.int8)
    w = np.zeros((16, 32), np.int8)
    rem = P
    for i in range(32):
        step = int(np.clip(rem, -127 * 127, 127 * 127))
        if step == 0:
            break
        aa = 127 if step > 0 else -127
        ww = abs(step) // 127
        a[0, i], w[0, i] = aa, ww
        rem -= aa * ww
        if rem != 0 and abs(rem) < 127:
            a[0, i + 1], w[0, i + 1] = rem, 1
            rem = 0
            break
    assert O.w8a8_block_sums(a, w, 32)[0, 0, 0] == P
    sws = np.full((16, 1), sw, np.float16).view(np.uint16)
    y = O.w8a8_gemm(a, np.array([sa], np.float32), w, sws, 32, epi=1, out=np.zeros((1, 16), np.float32))
    assert y[0, 0] == ref


def test_w8a8_per_channel_reduces_to_closed_form():
    a = rng(17).integers(-127, 128, (4, 256), dtype=np.int8)
    w = rng(18).integers(-127, 128, (16, 256), dtype=np.int8)
    sa = (rng(19).random(4) * 1e-2).astype(np.float32)
    sw = (rng(20).random((16, 1)) * 1e-3).astype(np.float32)
    y = O.w8a8_gemm(a, sa, w, sw, 256, epi=1, out=np.zeros((4, 16), np.float32))
    P = a.astype(np.int64) @ w.astype(np.int64).T
    want = ((P.astype(np.float32) * sa[:, None]).astype(np.float32) * sw[:, 0][None]).astype(np.float32)
    assert np.array_equal(y, want)


# ------------------------------------------------------------------------------------------------ Q4_K / W4A8
def _np_dequant_q4k(blocks):
    """Independent decoder of GGUF block_q4_K (ggml layout: d, dmin fp16; 12 bytes of 6-bit scales/mins packed as
    get_scale_min_k4; 4 x 32 bytes of quants, low nibbles sub-block 2c, high 2c + 1)."""
    N, NB, _ = blocks.shape
    out = np.zeros((N, NB * 256), np.float32)
    for n in range(N):
        for b in range(NB):
            o = blocks[n, b]
            d = o[0:2].view(np.float16).astype(np.float32)[0]
            dm = o[2:4].view(np.float16).astype(np.float32)[0]
            s = o[4:16].astype(np.int32)
            for j in range(8):
                if j < 4:
                    sc, m = s[j] & 63, s[j + 4] & 63
                else:
                    sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)
                    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
                byte = o[16 + 32 * (j // 2): 16 + 32 * (j // 2) + 32].astype(np.int32)
                q = (byte >> 4) if j % 2 else (byte & 0xF)
                out[n, b * 256 + 32 * j: b * 256 + 32 * j + 32] = (np.float32(d * np.float32(sc)) * q.astype(np.float32)
                                                                    - np.float32(dm * np.float32(m)))
    return out


def test_fold_parts_is_the_unsplit_epilogue():
    """The deferred residual add: one slot holding numpy's brute-force int64 sums gives the oracle GEMM's gk = K,
    epi 1 residual bit for bit; random splits of those sums into 2-5 slots give the same bits; rows >= live keep
    their values; fp16 weight scales give the same bits as the same values in fp32."""
    g = rng(41)
    M, N, K = 9, 80, 512
    a = g.integers(-127, 128, (M, K)).astype(np.int8)
    w = g.integers(-127, 128, (N, K)).astype(np.int8)
    sa = (g.random(M) * 0.02).astype(np.float32)
    sw16 = (g.random(N) * 0.01).astype(np.float16)
    sw = sw16.astype(np.float32)
    h = (g.standard_normal((M, N)) * 3).astype(np.float32)
    ref = O.w8a8_gemm(a, sa, w, sw.reshape(N, 1), K, epi=1, out=h.copy())
    P = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(O.fold_parts(h.copy(), P[None].astype(np.int32), sa, sw).view(np.int32), ref.view(np.int32))
    for S in (2, 3, 5):
        cut = g.integers(-2 ** 20, 2 ** 20, (S - 1, M, N))
        parts = np.concatenate([cut, (P - cut.sum(0))[None]]).astype(np.int32)
        assert np.array_equal(parts.astype(np.int64).sum(0), P)
        got = O.fold_parts(h.copy(), parts, sa, sw16.view(np.uint16))
        assert np.array_equal(got.view(np.int32), ref.view(np.int32))
    part = O.fold_parts(h.copy(), P[None].astype(np.int32), sa, sw, live=4)
    assert np.array_equal(part[:4].view(np.int32), ref[:4].view(np.int32)) and np.array_equal(part[4:], h[4:])


def test_q4k_quantizer_layout_and_torch():
    from prism_amd import gguf_formats as GF
    w = weights_f32(6, 512, seed=21)
    blocks = O.q4k_quantize(w)
    deq = O.q4k_dequant(blocks)
    assert np.array_equal(deq, _np_dequant_q4k(blocks))
    # round trip: within half a quantization step plus the 6-bit scale error, on average close
    assert np.abs(deq - w).max() < 0.02 and np.abs(deq - w).mean() < 0.003
    t = GF.quantize_q4k(torch.from_numpy(w))
    assert np.array_equal(t.raw.numpy(), blocks)
    assert np.array_equal(t.dequant().numpy(), deq)


def test_q4k_repack_reproduces_dequant():
    w = weights_f32(5, 512, seed=22)
    blocks = O.q4k_quantize(w)
    W = O.q4k_repack(blocks)
    N, K = 5, 512
    q = W["q"].reshape(N, K // 32, 16).astype(np.int32)
    vals = np.concatenate([q & 0xF, q >> 4], -1).reshape(N, K // 256, 8, 32).astype(np.float32)
    d = W["d"].T[:, :, None]
    dm = W["dm"].T[:, :, None]
    sc = W["sc"].transpose(1, 0, 2).astype(np.float32)
    mn = W["mn"].transpose(1, 0, 2).astype(np.float32)
    rec = ((d * sc).astype(np.float32)[..., None] * vals - (dm * mn).astype(np.float32)[..., None]).reshape(N, K)
    assert np.array_equal(rec, O.q4k_dequant(blocks))


def test_quant_rows_g_against_numpy():
    x = O.bf16_to_f32(acts_bf16(7, 1024, seed=23))
    x[2] = 0
    for group in (256, 1024):
        xq, a, xs = O.quant_rows_g(x, group)
        g = x.reshape(7, 1024 // group, group)
        sc = np.maximum(np.abs(g).max(-1), np.float32(1e-10)) / np.float32(127.0)
        assert np.array_equal(a, sc.T.astype(np.float32))
        want = np.rint(g / sc[..., None]).astype(np.int8).reshape(7, 1024)
        assert np.array_equal(xq, want)
        S = want.reshape(7, 32, 32).astype(np.int32).sum(-1)
        assert np.array_equal(O.group_sums(xs), S)
        assert xs.min() >= -64 and (xs[:, :, :8] >= 0).all()
    q1, s1 = O.quant_rows_i8(O.bf16_bits(x))
    xq, a, _ = O.quant_rows_g(x, 1024)
    assert np.array_equal(q1, xq) and np.array_equal(s1, a[0])


def test_w4a8_integer_sums_and_error_bound():
    N, K, M = 16, 512, 5
    blocks = O.q4k_quantize(weights_f32(N, K, seed=24))
    W = O.q4k_repack(blocks)
    x = O.bf16_to_f32(acts_bf16(M, K, seed=25))
    xq, a, xs = O.quant_rows_g(x, 256)
    out, acc, mins = O.w4a8_gemm(xq, a, xs, W, epi=1, out=np.zeros((M, N), np.float32), sums=True)
    q = W["q"].reshape(N, K // 32, 16).astype(np.int64)
    vals = np.concatenate([q & 0xF, q >> 4], -1).reshape(N, K // 256, 8, 32)
    P = np.einsum("mbgk,nbgk->mnbg", xq.reshape(M, K // 256, 8, 32).astype(np.int64), vals)
    sc = W["sc"].transpose(1, 0, 2).astype(np.int64)     # [N, NB, 8]
    mn = W["mn"].transpose(1, 0, 2).astype(np.int64)
    assert np.array_equal(acc, (P * sc[None]).sum(-1))
    S = O.group_sums(xs).reshape(M, K // 256, 8).astype(np.int64)
    assert np.array_equal(mins, np.einsum("mbg,nbg->mnb", S, mn))
    # float64 value of the same arithmetic; fp32 result within the rounding bound
    t = W["d"].T[None].astype(np.float64) * acc - W["dm"].T[None].astype(np.float64) * mins
    exact = (a.T[:, None, :].astype(np.float64) * t).sum(-1)
    mag = (np.abs(a.T[:, None, :].astype(np.float64)) * (np.abs(W["d"].T[None] * acc) + np.abs(W["dm"].T[None] * mins))).sum(-1)
    assert np.all(np.abs(out - exact) <= 8 * (K // 256 + 2) * 2.0 ** -24 * mag)
    # one element replayed with exact-rational fma / mul roundings (pins fma vs mul-then-add)
    m, n = 3, 11
    y = np.float32(0)
    for b in range(K // 256):
        t1 = np.float32(np.float32(W["d"][b, n]) * np.float32(acc[m, n, b]))
        t2 = np.float32(O.fmaf(-W["dm"][b, n], np.float32(mins[m, n, b]), t1))
        y = np.float32(O.fmaf(a[b, m], t2, y))
    assert out[m, n] == y
    o0 = O.w4a8_gemm(xq, a, xs, W, epi=0)
    assert np.array_equal(o0, O.bf16_bits(out))
    o_tok = O.w4a8_gemm(xq, np.repeat(a[:1], K // 256, 0), xs, W, epi=0)
    o_b = O.w4a8_gemm(xq, a[0].copy(), xs, W, epi=0)
    assert np.array_equal(o_tok, o_b)                   # a [M] broadcast == a [K/256, M] of equal rows


# --------------------------------------------------------------------------------------------------------- Q6_K
def _np_q6k_values(blocks):
    """The reference's reading of block_q6_K (kernels/w4a8.py:82-90): per half, the four 32-value parts built from
    ql low / ql high nibbles and the 2-bit fields of qh, minus 32."""
    ql = blocks[..., 0:128].astype(np.int32)
    qh = blocks[..., 128:192].astype(np.int32)
    parts = []
    for h in range(2):
        lo, hi, top = ql[..., 64 * h:64 * h + 32], ql[..., 64 * h + 32:64 * h + 64], qh[..., 32 * h:32 * h + 32]
        parts += [(lo & 0xF) | ((top & 3) << 4), (hi & 0xF) | (((top >> 2) & 3) << 4),
                  (lo >> 4) | (((top >> 4) & 3) << 4), (hi >> 4) | (((top >> 6) & 3) << 4)]
    return np.concatenate(parts, -1) - 32                # [N, NB, 256]


def test_q6k_layout_dequant_and_repack():
    N, NB = 7, 3
    blocks = q6k_random_blocks(N, NB, 51)
    v = _np_q6k_values(blocks)
    W = O.q6k_repack(blocks)
    assert np.array_equal(W["q"], v.reshape(N, NB * 256).astype(np.int8))
    sc = blocks[..., 192:208].view(np.int8)
    assert np.array_equal(W["sc"], sc.transpose(1, 0, 2))
    d = blocks[..., 208:210].copy().view(np.float16)[..., 0].astype(np.float32)
    assert np.array_equal(W["d"], d.T)
    want = (d[..., None] * sc.astype(np.float32)).astype(np.float32).repeat(16, -1) * v.astype(np.float32)
    assert np.array_equal(O.q6k_dequant(blocks), want.reshape(N, NB * 256))


def test_q6k_quantizer_round_trip_and_torch():
    from prism_amd import gguf_formats as GF
    w = weights_f32(6, 512, seed=52)
    blocks = O.q6k_quantize(w)
    v = _np_q6k_values(blocks)
    assert v.min() >= -32 and v.max() <= 31
    deq = O.q6k_dequant(blocks)
    d = blocks[..., 208:210].copy().view(np.float16)[..., 0].astype(np.float32)
    eff = (d[..., None] * blocks[..., 192:208].view(np.int8)).reshape(6, 32)          # each sub-block's step
    err = np.abs(deq - w).reshape(6, 32, 16)
    wa = np.abs(w).reshape(6, 32, 16)
    clamped = wa > 31.5 * eff[..., None]
    assert ((err <= 0.5 * eff[..., None] * (1 + 1e-6)) | clamped).all()
    assert (err[clamped] <= (wa - 31 * eff[..., None])[clamped] * (1 + 1e-6)).all()
    assert err.mean() < 0.3 * eff.mean()
    t = GF.quantize_q6k(torch.from_numpy(w))
    assert np.array_equal(t.raw.numpy(), blocks)
    assert np.array_equal(t.dequant().numpy(), deq)


def test_w4a8_q6k_integer_sums_and_error_bound():
    N, K, M = 16, 768, 5
    blocks = q6k_random_blocks(N, K // 256, 53)
    W = O.q6k_repack(blocks)
    x = O.bf16_to_f32(acts_bf16(M, K, seed=54))
    xq, a, _ = O.quant_rows_g(x, 256)
    out, acc = O.w4a8_gemm_q6k(xq, a, W, epi=1, out=np.zeros((M, N), np.float32), sums=True)
    P = np.einsum("mbhk,nbhk->mnbh", xq.reshape(M, K // 256, 16, 16).astype(np.int64),
                  W["q"].reshape(N, K // 256, 16, 16).astype(np.int64))
    sc = W["sc"].transpose(1, 0, 2).astype(np.int64)          # [N, NB, 16]
    assert np.array_equal(acc, (P * sc[None]).sum(-1))
    t = W["d"].T[None].astype(np.float64) * acc
    exact = (a.T[:, None, :].astype(np.float64) * t).sum(-1)
    mag = (np.abs(a.T[:, None, :].astype(np.float64)) * np.abs(t)).sum(-1)
    assert np.all(np.abs(out - exact) <= 4 * (K // 256 + 2) * 2.0 ** -24 * mag)
    m, n = 2, 9                                               # one element replayed: mul then fma per super-block
    y = np.float32(0)
    for b in range(K // 256):
        y = np.float32(O.fmaf(a[b, m], np.float32(np.float32(W["d"][b, n]) * np.float32(acc[m, n, b])), y))
    assert out[m, n] == y
    assert np.array_equal(O.w4a8_gemm_q6k(xq, a, W, epi=0), O.bf16_bits(out))
    o_tok = O.w4a8_gemm_q6k(xq, np.repeat(a[:1], K // 256, 0), W, epi=0)
    assert np.array_equal(o_tok, O.w4a8_gemm_q6k(xq, a[0].copy(), W, epi=0))
