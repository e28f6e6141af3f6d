"""GPU parity of the W4A8 activation producer (rows_g) and the Q4_K W4A8 GEMM against the CPU oracle.

Bit-exact throughout: the producer's int8 values, scales and split per-32 sums (as the reference's
tests/test_w4a8.py checks rows_g against quantize_ref); the packed weight layout against a numpy restatement; the
integer super-block sums through a case whose fp32 arithmetic is exact; the bf16 outputs and fp32 residual adds of
both kernels (decode, tile) against gemm_ref's arithmetic (the reference checks every kernel against gemm_ref with
torch.equal), for config 3's shape class and ragged / live-row cases."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, half_integer_rows, rng, weights_f32

pytestmark = pytest.mark.gpu


def _t(x, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t if dtype is None else t.view(dtype)


def _live(n, dev):
    return torch.tensor([n], dtype=torch.int32, device=dev)


def _np_pack(blocks):
    """GGUF block_q4_K bytes [N, NB, 144] -> (qv [N/16, NB, 2, 64, 16], meta [N/16, NB, 16, 16])."""
    N, NB, _ = blocks.shape
    qs = blocks[:, :, 16:].reshape(N, NB, 4, 32).astype(np.uint32)
    vals = np.stack([qs & 15, qs >> 4], 3).reshape(N, NB, 8, 32)              # [row, b, sub-block, 32]
    r = vals.reshape(N // 16, 16, NB, 2, 2, 4, 2, 8)                           # [nt, row, b, h, pp, q, half8, t]
    lo, hi = r[..., 0, :], r[..., 1, :]                                         # [nt, row, b, h, pp, q, t]
    byte = (lo | (hi << 4)).astype(np.uint8)
    qv = byte.transpose(0, 2, 3, 5, 1, 4, 6).reshape(N // 16, NB, 2, 64, 16)  # lane = q * 16 + row, byte = pp 8 + t
    meta = blocks[:, :, :16].reshape(N // 16, 16, NB, 16).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(qv), np.ascontiguousarray(meta)


def _w4(dev, blocks):
    from prism_amd import gguf_formats as GF
    from prism_amd import w4a8 as KW4
    N, NB, _ = blocks.shape
    return KW4.repack(GF.KQuant(_t(blocks, dev), GF.GGML_Q4_K, NB * 256))


def test_pack_layout(dev):
    blocks = O.q4k_quantize(weights_f32(48, 768, seed=41))
    w = _w4(dev, blocks)
    torch.cuda.synchronize()
    qv, meta = _np_pack(blocks)
    assert np.array_equal(w.qv.cpu().numpy(), qv) and np.array_equal(w.meta.cpu().numpy(), meta)


@pytest.mark.parametrize("M,K,group,live", [(33, 2560, 256, 33), (16, 5120, 256, 11), (16, 5120, 5120, 16),
                                            (3, 4096, 4096, 3), (1, 256, 256, 1)])
def test_rows_g_bit_exact(dev, M, K, group, live):
    from prism_amd import quant as KQ
    x = acts_bf16(M, K, seed=K + M)
    x[0, 5] = O.bf16_bits(np.array([-40.0], np.float32))[0]
    q = torch.full((M, K), 9, dtype=torch.int8, device=dev)
    s = torch.zeros(K // group, M, dtype=torch.float32, device=dev)
    xs = torch.zeros(K // 256, M, 16, dtype=torch.int8, device=dev)
    KQ.rows_g(_t(x, dev, torch.bfloat16), q, s, xs, _live(live, dev), M, group=group)
    rq, ra, rxs = O.quant_rows_g(O.bf16_to_f32(x), group, live=live)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy()[:live], rq[:live])
    assert np.array_equal(s.cpu().numpy()[:, :live], ra[:, :live])
    assert np.array_equal(xs.cpu().numpy()[:, :live], rxs[:, :live])


@pytest.mark.parametrize("group", [256, 1024])
def test_rows_g_half_integers(dev, group):
    """The W4A8 quantizer on quotients at and beside half-integers (see _inputs.half_integer_rows)."""
    from prism_amd import quant as KQ
    x = half_integer_rows(1024)
    M, K = x.shape
    q = torch.zeros((M, K), dtype=torch.int8, device=dev)
    s = torch.zeros(K // group, M, dtype=torch.float32, device=dev)
    xs = torch.zeros(K // 256, M, 16, dtype=torch.int8, device=dev)
    KQ.rows_g(_t(x, dev, torch.bfloat16), q, s, xs, _live(M, dev), M, group=group)
    rq, ra, rxs = O.quant_rows_g(O.bf16_to_f32(x), group, live=M)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), ra)
    assert np.array_equal(xs.cpu().numpy(), rxs)


def _case(N, K, M, seed, group=256):
    blocks = O.q4k_quantize(weights_f32(N, K, seed=seed))
    x = O.bf16_to_f32(acts_bf16(M, K, seed=seed + 1))
    xq, a, xs = O.quant_rows_g(x, group)
    return blocks, xq, a, xs


def _gemm(dev, w, xq, a, xs, epi, kernel, live=None, out0=None):
    from prism_amd import w4a8 as KW4
    M = xq.shape[0]
    live = M if live is None else live
    if epi == 0:
        out = torch.full((M, w.n), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    else:
        out = _t(out0, dev).clone()
    ad = _t(a, dev)
    KW4.gemm(_t(xq, dev), ad, _t(xs, dev), w, out, _live(live, dev), epi=epi, kernel=kernel)
    torch.cuda.synchronize()
    return out


def _bal_fits(M, K):
    """The balanced kernel's LDS rule: activation image M (K + 32), sums K M / 16, scales K M / 64, terms 2.3 KB per
    row (12 units x 3 rounds x 16 outputs x 4 bytes)."""
    return M * (K + 32) + K // 16 * M + K // 64 * M + 3 * 12 * M * 64 + 64 <= 160 * 1024


CASES = [  # (M, N, K, live, group)
    (1, 16, 256, 1, 256), (4, 64, 1024, 3, 256), (16, 128, 5120, 16, 256), (16, 256, 5120, 16, 5120),
    (7, 48, 2560, 5, 256), (64, 128, 1024, 64, 256), (100, 272, 768, 77, 256), (130, 128, 2048, 130, 2048),
    # the decode kernel's two wave counts (4 waves: N > 2048 and K < 6144), a long K with several ring trips per
    # wave, and K beyond the decode kernel's LDS for 16 rows (the tile kernel runs)
    (16, 2576, 1024, 13, 256), (2, 2064, 512, 2, 256), (4, 32, 12288, 4, 256), (16, 16, 41216, 16, 256),
    # from 5 rows with N % 32 == 0 the decode kernel takes two tiles per workgroup (4 waves each here)
    (12, 2560, 1024, 9, 256),
]


@pytest.mark.parametrize("M,N,K,live,group", CASES)
def test_gemm_bit_exact(dev, M, N, K, live, group):
    blocks, xq, a, xs = _case(N, K, M, seed=N + K + M, group=group)
    W = O.q4k_repack(blocks)
    ao = a if group == 256 else a[0].copy()
    want0 = O.w4a8_gemm(xq, ao, xs, W, epi=0, live=live)
    base = rng(M + N).standard_normal((M, N)).astype(np.float32)
    want1 = O.w4a8_gemm(xq, ao, xs, W, epi=1, out=base.copy(), live=live)
    w = _w4(dev, blocks)
    for kernel in ["tile"] + (["decode", "stream"] if M <= 16 and _bal_fits(M, K) else ["decode"] if M <= 16 else []):
        got0 = _gemm(dev, w, xq, a, xs, 0, kernel, live=live).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got0[:live], want0[:live]), kernel
        assert (got0[live:] == 7).all(), kernel
        got1 = _gemm(dev, w, xq, a, xs, 1, kernel, live=live, out0=base).cpu().numpy()
        assert np.array_equal(got1, want1), kernel


def test_config3_decode_slice_bit_exact(dev):
    """Config 3's decode shape class: M = 16, K = 5120, a slice of N = 13824 (1024 rows), one scale per token."""
    blocks, xq, a, xs = _case(1024, 5120, 16, seed=3, group=5120)
    W = O.q4k_repack(blocks)
    want = O.w4a8_gemm(xq, a[0].copy(), xs, W, epi=0)
    w = _w4(dev, blocks)
    for kernel in ("decode", "stream", "tile"):
        got = _gemm(dev, w, xq, a, xs, 0, kernel).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got, want), kernel


def test_integer_sums_exact(dev):
    """Blocks with d = dmin = 1 and unit activation scales make every fp32 step exact, so the output is
    sum_b (acc_b - mins_b): the int32 super-block sums themselves."""
    N, K, M = 32, 1024, 16
    g = rng(5)
    blocks = g.integers(0, 256, (N, K // 256, 144), dtype=np.uint8)
    blocks[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blocks[:, :, 2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    x = g.integers(-127, 128, (M, K), dtype=np.int8)
    S = x.reshape(M, K // 32, 32).astype(np.int32).sum(-1).reshape(M, K // 256, 8)
    xs = np.concatenate([S & 63, S >> 6], -1).astype(np.int8).transpose(1, 0, 2).copy()
    a = np.ones(M, np.float32)
    W = O.q4k_repack(blocks)
    _, acc, mins = O.w4a8_gemm(x, a, xs, W, epi=1, out=np.zeros((M, N), np.float32), sums=True)
    want = (acc.astype(np.int64) - mins).sum(-1)
    w = _w4(dev, blocks)
    for kernel in ("decode", "stream", "tile"):
        got = _gemm(dev, w, x, a, xs, 1, kernel, out0=np.zeros((M, N), np.float32)).cpu().numpy()
        assert np.array_equal(got.astype(np.int64), want), kernel


def test_stream_kernel_limits(dev):
    """kernel="stream" on Q4_K weights is the balanced-grid kernel: more than 16 rows, or an activation image beyond
    LDS, is an error rather than a silent fallback."""
    blocks, xq, a, xs = _case(32, 512, 17, seed=77)
    with pytest.raises(Exception):
        _gemm(dev, _w4(dev, blocks), xq, a, xs, 0, "stream")
    blocks, xq, a, xs = _case(16, 41216, 16, seed=78)
    with pytest.raises(Exception):
        _gemm(dev, _w4(dev, blocks), xq, a, xs, 0, "stream")
