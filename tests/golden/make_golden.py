"""Writes the committed golden fixtures of this build: seeded inputs (numpy PCG64) and the oracle's outputs, small
enough to commit.  The reference holds no numeric fixtures for this path, so these pin the oracle against itself
over time (a regression check) and give the GPU tests fixed vectors.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402


def q8_case(M, N, K, seed):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = O.bf16_bits(g.standard_normal((M, K), dtype=np.float32))
    qs, d = O.q8_0_quantize(w)
    q, s = O.quant_rows_i8(x)
    out = O.w8a8_gemm(q, s, qs, d, 32, epi=0)
    P = O.w8a8_block_sums(q, qs, 32)
    return dict(x=x, qs=qs, d=d, q=q, s=s, out=out, P=P)


def q4k_case(M, N, K, seed, group):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = O.bf16_bits(g.standard_normal((M, K), dtype=np.float32))
    blocks = O.q4k_quantize(w)
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(x), group)
    W = O.q4k_repack(blocks)
    out, acc, mins = O.w4a8_gemm(xq, a if group == 256 else a[0].copy(), xs, W, epi=0, sums=True)
    return dict(x=x, blocks=blocks, xq=xq, a=a, xs=xs, out=out, acc=acc, mins=mins)


def main():
    np.savez_compressed(os.path.join(HERE, "q8_0_w8a8_m4_n32_k256.npz"), **q8_case(4, 32, 256, seed=1000))
    np.savez_compressed(os.path.join(HERE, "q4k_w4a8_m3_n16_k512_g256.npz"), **q4k_case(3, 16, 512, 1001, 256))
    np.savez_compressed(os.path.join(HERE, "q4k_w4a8_m2_n16_k512_tok.npz"), **q4k_case(2, 16, 512, 1002, 512))


if __name__ == "__main__":
    main()
