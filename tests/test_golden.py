"""The committed golden fixtures (tests/golden/make_golden.py): the oracle must reproduce them bit for bit (CPU);
the GPU kernels must reproduce them too (marked gpu)."""
import glob
import os

import numpy as np
import pytest

import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(HERE, name), allow_pickle=False))


def test_fixtures_present():
    assert len(glob.glob(os.path.join(HERE, "*.npz"))) >= 3


def test_oracle_reproduces_q8_fixture():
    f = _load("q8_0_w8a8_m4_n32_k256.npz")
    q, s = O.quant_rows_i8(f["x"])
    assert np.array_equal(q, f["q"]) and np.array_equal(s, f["s"])
    assert np.array_equal(O.w8a8_block_sums(q, f["qs"], 32), f["P"])
    assert np.array_equal(O.w8a8_gemm(q, s, f["qs"], f["d"], 32, epi=0), f["out"])


@pytest.mark.parametrize("name,group", [("q4k_w4a8_m3_n16_k512_g256.npz", 256), ("q4k_w4a8_m2_n16_k512_tok.npz", 512)])
def test_oracle_reproduces_q4k_fixture(name, group):
    f = _load(name)
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(f["x"]), group)
    assert np.array_equal(xq, f["xq"]) and np.array_equal(a, f["a"]) and np.array_equal(xs, f["xs"])
    out, acc, mins = O.w4a8_gemm(xq, a if group == 256 else a[0].copy(), xs, O.q4k_repack(f["blocks"]), epi=0, sums=True)
    assert np.array_equal(out, f["out"]) and np.array_equal(acc, f["acc"]) and np.array_equal(mins, f["mins"])


@pytest.mark.gpu
def test_gpu_reproduces_fixtures(dev):
    import torch
    from prism_amd import gguf_formats as GF
    from prism_amd import quant as KQ
    from prism_amd import w4a8 as KW4
    from prism_amd import w8a8 as KW
    f = _load("q8_0_w8a8_m4_n32_k256.npz")
    M, K = f["x"].shape
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    q = torch.empty(M, K, dtype=torch.int8, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    KQ.rows_q8(torch.from_numpy(f["x"]).to(dev).view(torch.bfloat16), None, q, s, n, M)
    pw = KW.pack_q8(torch.from_numpy(f["qs"]).to(dev), torch.from_numpy(f["d"]).to(dev).view(torch.float16))
    for kernel in ("decode", "tile"):
        out = torch.empty(M, f["qs"].shape[0], dtype=torch.bfloat16, device=dev)
        KW.gemm(q, s, pw, None, out, n, 32, kernel=kernel)
        assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), f["out"]), kernel
    for name in ("q4k_w4a8_m3_n16_k512_g256.npz", "q4k_w4a8_m2_n16_k512_tok.npz"):
        f = _load(name)
        M, K = f["xq"].shape
        n = torch.tensor([M], dtype=torch.int32, device=dev)
        w4 = KW4.repack(GF.KQuant(torch.from_numpy(f["blocks"]).to(dev), GF.GGML_Q4_K, K))
        for kernel in ("decode", "tile"):
            out = torch.empty(M, w4.n, dtype=torch.bfloat16, device=dev)
            KW4.gemm(torch.from_numpy(f["xq"]).to(dev), torch.from_numpy(f["a"]).to(dev), torch.from_numpy(f["xs"]).to(dev),
                     w4, out, n, kernel=kernel)
            assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), f["out"]), (name, kernel)
