"""Seeded CPU inputs shared by the tests (numpy PCG64), following the value distributions of the benchmark
configs: weights fp32 N(0, 0.02^2) quantized to Q8_0 / Q4_K, activations N(0, 1) rounded to bf16."""
import numpy as np

import oracle as O

# MXFP4 GEMM tolerance for the fp32 result, relative to sum |terms| (the float64 value's absolute terms).  The scaled
# MFMA adds its 128 products and the accumulator with a limited alignment window, not as a chain of rounded fp32
# adds: on operands whose block scales span 2^20 (products over about 2^48) one v_mfma_scale_f32_16x16x128_f8f6f4
# was measured up to 205 u sum|terms| off (u = 2^-24), a 2048-input chain 284 u; Gaussian operands of one scale 13 u.
# The bound is 1024 u, four times the worst measured.
MX_ACC_REL = 2.0 ** -14


def rng(seed):
    return np.random.default_rng(seed)


def weights_f32(N, K, seed, std=0.02):
    return (rng(seed).standard_normal((N, K), dtype=np.float32) * np.float32(std)).astype(np.float32)


def acts_bf16(M, K, seed, std=1.0):
    """bf16 bit patterns uint16 [M, K]."""
    x = rng(seed).standard_normal((M, K), dtype=np.float32) * np.float32(std)
    return O.bf16_bits(x)


def q8_weights(N, K, seed):
    return O.q8_0_quantize(weights_f32(N, K, seed))


def int8_acts(M, K, seed):
    return O.quant_rows_i8(acts_bf16(M, K, seed))


def q6k_random_blocks(N, NB, seed):
    """Arbitrary block_q6_K bytes (every bit pattern of ql, qh and the int8 scales, -128 included) with finite
    positive fp16 d: the GEMM takes the file's bytes as they are."""
    g = rng(seed)
    b = g.integers(0, 256, (N, NB, 210), dtype=np.uint8)
    b[..., 192] = 0x80                                    # one scale of -128 per super-block
    d = (g.random((N, NB)) * 1e-3 + 1e-5).astype(np.float16)
    b[..., 208:210] = d.view(np.uint8).reshape(N, NB, 2)
    return b


def half_integer_rows(K):
    """bf16 rows whose quotients y / scale sit on and beside half-integers, where the quantizers' rounding is decided:
    row 0 has amax 127 (scale 1: every k + 1/2 an exact tie, rounded to even), row 1 amax 127 / 32 (scale 2^-5, exact
    ties again), row 2 amax 381 (scale 3: (k + 1/2) 3 rounded to bf16 lands just beside the half-integers), row 3 the
    same with a sign flip per element.  K a multiple of 256."""
    k = np.arange(K) % 254 - 127                               # -127 .. 126
    rows = np.empty((4, K), np.float32)
    rows[0] = k + 0.5
    rows[1] = (k + 0.5) / 32
    rows[2] = (k + 0.5) * 3
    rows[3] = -rows[2] * np.where(np.arange(K) % 2, 1, -1)
    rows[0, 0], rows[1, 0], rows[2, 0], rows[3, 0] = 127.0, 127.0 / 32, 381.0, -381.0   # the row maxima
    return O.bf16_bits(rows)
