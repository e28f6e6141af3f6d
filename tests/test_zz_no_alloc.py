"""prism_w8a8_q8_0_packed_gemm_noalloc, the entry point that allocates nothing: through the C ABI it gives the bits of
prism_w8a8_q8_0_packed_gemm with a caller's workspace, on two calls in a row (the second smaller), for the balanced
decode kernel that uses the library's scratch array and for the kernel the library picks by itself."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, q8_weights

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _run(dev, fn, M, N, K, seed, kernel, epi):
    from prism_amd import _lib as L
    from prism_amd import w8a8 as KW
    qs, d = q8_weights(N, K, seed=seed)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=seed + 1))
    pw = KW.pack_q8(_t(qs, dev), _t(d, dev).view(torch.float16))
    ad, sd = _t(a, dev), _t(s, dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    if epi == 0:
        out = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    else:
        out = _t(np.random.default_rng(seed).standard_normal((M, N)).astype(np.float32), dev)
    args = [L.ptr(ad), L.ptr(sd), 1, L.ptr(pw.qt), L.ptr(pw.dt), L.ptr(out), N, L.ptr(n), M, N, K, epi, kernel]
    if fn == "prism_w8a8_q8_0_packed_gemm":
        ws = KW.workspace(dev)
        args += [L.ptr(ws), ws.numel()]
    torch.cuda.synchronize()
    print(f"{fn} M={M} N={N} K={K} kernel={kernel} epi={epi}", flush=True)
    L.call(fn, *args, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu().numpy() if epi == 0 else out.cpu().numpy()


@pytest.mark.parametrize("kernel", [4, -1])
def test_noalloc_two_calls_match(dev, kernel):
    for (M, N, K, epi) in ((16, 5120, 5120, 0), (7, 1024, 2048, 1)):     # the second call smaller
        want = _run(dev, "prism_w8a8_q8_0_packed_gemm", M, N, K, 31 + M, kernel, epi)
        got = _run(dev, "prism_w8a8_q8_0_packed_gemm_noalloc", M, N, K, 31 + M, kernel, epi)
        assert np.array_equal(got, want), (M, N, K, kernel)
