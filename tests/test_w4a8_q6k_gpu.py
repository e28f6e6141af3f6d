"""GPU parity of the W4A8 GEMM on Q6_K weights (kernels/w4a8.py:19-20, gemm_ref :193-197) against the CPU oracle,
bit for bit: the load-time pack's layout, bf16 stores and fp32 residual adds from the decode and tile kernels, one
activation scale per 256 inputs or per token, live rows, blocks of every bit pattern (negative and -128 scales), the
integer super-block sums, a fused projection mixing Q4_K and Q6_K segments, and the load step from a GGUF tensor's
bytes (prism_amd.weights) for Q8_0, Q4_K and Q6_K."""
import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, q6k_random_blocks, rng, weights_f32

pytestmark = pytest.mark.gpu


def _t(x, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t if dtype is None else t.view(dtype)


def _live(n, dev):
    return torch.tensor([n], dtype=torch.int32, device=dev)


def _np_pack(blocks):
    """block_q6_K bytes [N, NB, 210] -> (qv int8 [N/16, NB, 4, 64, 16], meta uint8 [N/16, NB, 288])."""
    from prism_amd import gguf_formats as GF
    N, NB, _ = blocks.shape
    v = GF.q6k_values(torch.from_numpy(blocks)).numpy().astype(np.int8)          # [N, NB, 256] in k order
    r = v.reshape(N // 16, 16, NB, 4, 2, 4, 8)                                  # [nt, row, b, j, u, q, t]
    qv = r.transpose(0, 2, 3, 5, 1, 4, 6).reshape(N // 16, NB, 4, 64, 16)       # lane = q * 16 + row, byte = 8 u + t
    sc = blocks[..., 192:208].reshape(N // 16, 16, NB, 16).transpose(0, 2, 1, 3).reshape(N // 16, NB, 256)
    d = blocks[..., 208:210].reshape(N // 16, 16, NB, 2).transpose(0, 2, 1, 3).reshape(N // 16, NB, 32)
    return np.ascontiguousarray(qv), np.ascontiguousarray(np.concatenate([sc, d], -1))


def _w6(dev, blocks):
    from prism_amd import gguf_formats as GF
    from prism_amd import w4a8 as KW4
    return KW4.repack(GF.KQuant(_t(blocks, dev), GF.GGML_Q6_K, blocks.shape[1] * 256))


def test_pack_layout(dev):
    blocks = q6k_random_blocks(48, 3, seed=61)
    w = _w6(dev, blocks)
    torch.cuda.synchronize()
    qv, meta = _np_pack(blocks)
    assert np.array_equal(w.qv.cpu().numpy(), qv) and np.array_equal(w.meta.cpu().numpy(), meta)


def _gemm(dev, w, xq, a, epi, kernel, live=None, out0=None):
    from prism_amd import w4a8 as KW4
    M, K = xq.shape
    live = M if live is None else live
    if epi == 0:
        out = torch.full((M, w.n), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    else:
        out = _t(out0, dev).clone()
    xs = torch.zeros(K // 256, M, 16, dtype=torch.int8, device=dev)
    KW4.gemm(_t(xq, dev), _t(a, dev), xs, w, out, _live(live, dev), epi=epi, kernel=kernel)
    torch.cuda.synchronize()
    return out


CASES = [  # (M, N, K, live, group, random blocks)
    (1, 16, 256, 1, 256, True), (4, 64, 1024, 3, 256, False), (16, 128, 5120, 16, 256, True),
    (16, 256, 5120, 16, 5120, False), (7, 48, 2560, 5, 256, True), (64, 128, 1024, 64, 256, False),
    (100, 272, 768, 77, 256, True), (130, 128, 2048, 130, 2048, False),
    (8, 96, 2560, 6, 256, True),       # 5-8 rows, N % 32 == 0: the decode kernel's two tiles per workgroup
]


@pytest.mark.parametrize("M,N,K,live,group,rand", CASES)
def test_gemm_bit_exact(dev, M, N, K, live, group, rand):
    seed = N + K + M
    blocks = q6k_random_blocks(N, K // 256, seed) if rand else O.q6k_quantize(weights_f32(N, K, seed=seed))
    xq, a, _ = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=seed + 1)), group)
    W = O.q6k_repack(blocks)
    ao = a if group == 256 else a[0].copy()
    want0 = O.w4a8_gemm_q6k(xq, ao, W, epi=0, live=live)
    base = rng(M + N).standard_normal((M, N)).astype(np.float32)
    want1 = O.w4a8_gemm_q6k(xq, ao, W, epi=1, out=base.copy(), live=live)
    w = _w6(dev, blocks)
    for kernel in ["tile"] + (["decode", "stream"] if M <= 16 else []):
        got0 = _gemm(dev, w, xq, a, 0, kernel, live=live).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got0[:live], want0[:live]), kernel
        assert (got0[live:] == 7).all(), kernel
        got1 = _gemm(dev, w, xq, a, 1, kernel, live=live, out0=base).cpu().numpy()
        assert np.array_equal(got1, want1), kernel


def test_integer_sums_exact(dev):
    """d = 1 and unit activation scales with activations in -3..3 keep every fp32 step exact (|sums| < 2^24), so
    the output is the sum over super-blocks of the int32 acc itself."""
    N, K, M = 32, 1024, 16
    g = rng(62)
    blocks = q6k_random_blocks(N, K // 256, 63)
    blocks[..., 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    x = g.integers(-3, 4, (M, K), dtype=np.int8)
    a = np.ones(M, np.float32)
    W = O.q6k_repack(blocks)
    _, acc = O.w4a8_gemm_q6k(x, a, W, epi=1, out=np.zeros((M, N), np.float32), sums=True)
    want = acc.astype(np.int64).sum(-1)
    assert np.abs(want).max() < 2 ** 24
    w = _w6(dev, blocks)
    for kernel in ("decode", "stream", "tile"):
        got = _gemm(dev, w, x, a, 1, kernel, out0=np.zeros((M, N), np.float32)).cpu().numpy()
        assert np.array_equal(got.astype(np.int64), want), kernel


def test_mixed_segments(dev):
    """A fused projection of a Q4_K, a Q6_K and a Q4_K matrix (kernels/w4a8.py:107-140): one GEMM per segment into
    its columns, each bit-equal to its oracle."""
    from prism_amd import gguf_formats as GF
    from prism_amd import w4a8 as KW4
    M, K = 16, 1024
    parts = [("q4k", 64), ("q6k", 32), ("q4k", 48)]
    raws = [O.q4k_quantize(weights_f32(n, K, seed=70 + i)) if kind == "q4k" else
            O.q6k_quantize(weights_f32(n, K, seed=70 + i)) for i, (kind, n) in enumerate(parts)]
    kqs = [GF.KQuant(_t(r, dev), kind, K) for r, (kind, _) in zip(raws, parts)]
    segs = KW4.segments(kqs, dev)
    assert [w.kind for w, _ in segs] == ["q4k", "q6k", "q4k"]
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=75)), 256)
    out = torch.zeros(M, KW4.seg_width(segs), dtype=torch.bfloat16, device=dev)
    KW4.gemm_segs(_t(xq, dev), _t(a, dev), _t(xs, dev), segs, out, _live(M, dev))
    torch.cuda.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    off = 0
    for r, (kind, n) in zip(raws, parts):
        want = (O.w4a8_gemm(xq, a, xs, O.q4k_repack(r)) if kind == "q4k" else
                O.w4a8_gemm_q6k(xq, a, O.q6k_repack(r)))
        assert np.array_equal(got[:, off:off + n], want), kind
        off += n


@pytest.mark.parametrize("ggml_type", [8, 12, 14])
def test_from_gguf_bytes(dev, ggml_type):
    """prism_amd.weights.from_gguf: a tensor's GGUF bytes (ggml dims [inputs, outputs]) to the device operand, then
    the GEMM bit-equal to the oracle on the same bytes."""
    from prism_amd import w4a8 as KW4
    from prism_amd import w8a8 as KW
    from prism_amd import weights as PW
    N, K, M = 64, 1024, 5
    w = weights_f32(N, K, seed=80 + ggml_type)
    x = O.bf16_to_f32(acts_bf16(M, K, seed=90))
    out = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
    if ggml_type == 8:
        qs, d = O.q8_0_quantize(w)                          # block_q8_0: fp16 d, then 32 int8
        raw = np.concatenate([d.reshape(N, K // 32, 1).view(np.uint8), qs.view(np.uint8).reshape(N, K // 32, 32)], -1)
        op = PW.from_gguf(raw.reshape(-1), ggml_type, (K, N), dev)
        q, s = O.quant_rows_i8(O.bf16_bits(x))
        want = O.w8a8_gemm(q, s, qs, d, 32, epi=0)
        KW.gemm(_t(q, dev), _t(s, dev), op[0], op[1], out, _live(M, dev), 32)
    else:
        raw = O.q4k_quantize(w) if ggml_type == 12 else O.q6k_quantize(w)
        op = PW.from_gguf(raw.reshape(-1), ggml_type, (K, N), dev)
        xq, a, xs = O.quant_rows_g(x, 256)
        want = (O.w4a8_gemm(xq, a, xs, O.q4k_repack(raw)) if ggml_type == 12 else
                O.w4a8_gemm_q6k(xq, a, O.q6k_repack(raw)))
        KW4.gemm(_t(xq, dev), _t(a, dev), _t(xs, dev), op, out, _live(M, dev))
    torch.cuda.synchronize()
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), want)
