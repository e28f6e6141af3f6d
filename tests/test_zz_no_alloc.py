"""prism_w8a8_q8_0_packed_gemm_noalloc, the entry point that allocates nothing: through the C ABI it gives the bits of
prism_w8a8_q8_0_packed_gemm with a caller's workspace, on two calls in a row (the second smaller), for the balanced
decode kernel that uses the library's scratch array and for the kernel the library picks by itself; a call with
fewer live rows than M leaves the array as a later full call needs it (checked against the oracle); the entry point
captured in a graph replays to the eager bits; and in a fresh process whose first call on the device is made under
graph capture, the replays give the workspace form's bits."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, q8_weights

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _case(dev, M, N, K, seed, epi, live=None):
    """Device operands of one call and the oracle's result for its live rows."""
    from prism_amd import w8a8 as KW
    qs, d = q8_weights(N, K, seed=seed)
    a, s = O.quant_rows_i8(acts_bf16(M, K, seed=seed + 1))
    pw = KW.pack_q8(_t(qs, dev), _t(d, dev).view(torch.float16))
    n = torch.tensor([M if live is None else live], dtype=torch.int32, device=dev)
    if epi == 0:
        out0 = np.full((M, N), 7, dtype=np.int16)
    else:
        out0 = np.random.default_rng(seed).standard_normal((M, N)).astype(np.float32)
    return dict(a=_t(a, dev), s=_t(s, dev), pw=pw, n=n, out=_t(out0, dev), out0=out0, M=M, N=N, K=K, epi=epi,
                want=lambda: O.w8a8_gemm(a, s, qs, d, 32, epi=epi, out=None if epi == 0 else out0.copy()))


def _call(dev, fn, c, kernel, stream=None):
    from prism_amd import _lib as L
    from prism_amd import w8a8 as KW
    M, N, K = c["M"], c["N"], c["K"]
    args = [L.ptr(c["a"]), L.ptr(c["s"]), 1, L.ptr(c["pw"].qt), L.ptr(c["pw"].dt), L.ptr(c["out"]), N,
            L.ptr(c["n"]), M, N, K, c["epi"], kernel]
    if fn == "prism_w8a8_q8_0_packed_gemm":
        ws = KW.workspace(dev)
        args += [L.ptr(ws), ws.numel()]
    st = stream if stream is not None else torch.cuda.current_stream()
    L.call(fn, *args, ctypes.c_void_p(st.cuda_stream))


def _bits(c):
    return c["out"].cpu().numpy()


def _run(dev, fn, M, N, K, seed, kernel, epi):
    c = _case(dev, M, N, K, seed, epi)
    torch.cuda.synchronize()
    print(f"{fn} M={M} N={N} K={K} kernel={kernel} epi={epi}", flush=True)
    _call(dev, fn, c, kernel)
    torch.cuda.synchronize()
    return _bits(c)


@pytest.mark.parametrize("kernel", [4, -1])
def test_noalloc_two_calls_match(dev, kernel):
    for (M, N, K, epi) in ((16, 5120, 5120, 0), (7, 1024, 2048, 1)):     # the second call smaller
        want = _run(dev, "prism_w8a8_q8_0_packed_gemm", M, N, K, 31 + M, kernel, epi)
        got = _run(dev, "prism_w8a8_q8_0_packed_gemm_noalloc", M, N, K, 31 + M, kernel, epi)
        assert np.array_equal(got, want), (M, N, K, kernel)


def test_noalloc_partial_rows_then_full(dev):
    """A call with 5 live rows of 16 (the balanced kernel hands sums for all 16 rows), then a full call on other
    operands: both equal the oracle, so the first left the scratch array as the second needs it."""
    M, N, K = 16, 5120, 5120
    c1 = _case(dev, M, N, K, 41, 0, live=5)
    print("noalloc partial rows: live=5 of 16", flush=True)
    _call(dev, "prism_w8a8_q8_0_packed_gemm_noalloc", c1, 4)
    torch.cuda.synchronize()
    got = _bits(c1)
    want = c1["want"]()
    assert np.array_equal(got[:5].view(np.uint16), want[:5])
    assert np.array_equal(got[5:], c1["out0"][5:])                        # rows >= live untouched
    c2 = _case(dev, M, N, K, 43, 1)
    print("noalloc full call after it", flush=True)
    _call(dev, "prism_w8a8_q8_0_packed_gemm_noalloc", c2, 4)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(c2), c2["want"]())


def _capture_and_replay(dev, c, kernel, replays=2):
    """Captures one noalloc call on a side stream, replays it `replays` times (eager work and synchronizations between
    the replays), returns each replay's output bits."""
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        _call(dev, "prism_w8a8_q8_0_packed_gemm_noalloc", c, kernel, stream=s)
    res = []
    for r in range(replays):
        print(f"noalloc graph replay {r}", flush=True)
        c["out"].copy_(_t(c["out0"], dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        res.append(_bits(c))
        torch.zeros(1 << 20, device=dev).sum().item()                       # eager work between the replays
    del g
    return res


@pytest.mark.parametrize("epi", [0, 1])
def test_noalloc_graph_replay(dev, epi):
    c = _case(dev, 13, 5120, 5120, 51 + epi, epi)
    _call(dev, "prism_w8a8_q8_0_packed_gemm_noalloc", c, 4)                   # eager
    torch.cuda.synchronize()
    eager = _bits(c)
    want = c["want"]()
    assert np.array_equal(eager.view(np.uint16) if epi == 0 else eager, want)
    for got in _capture_and_replay(dev, c, 4, replays=3):
        assert np.array_equal(got, eager)


def _first_call_captured():
    """Child process: the device's first noalloc call is made under graph capture; the replays must give the
    workspace form's bits."""
    dev = torch.device("cuda:0")
    c = _case(dev, 16, 5120, 5120, 61, 0)
    reps = _capture_and_replay(dev, c, 4, replays=2)
    c["out"].copy_(_t(c["out0"], dev))
    _call(dev, "prism_w8a8_q8_0_packed_gemm", c, 4)
    torch.cuda.synchronize()
    ref = _bits(c)
    for got in reps:
        assert np.array_equal(got, ref)
    assert np.array_equal(ref.view(np.uint16), c["want"]())
    print("first-call-under-capture: ok", flush=True)


def test_noalloc_first_call_under_capture(dev):
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([here, root, os.path.join(root, "startlux-prism_amd")] +
                                        ([env["PYTHONPATH"]] if env.get("PYTHONPATH") else []))
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--first-call-captured"], env=env,
                       capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-4000:], flush=True)
    assert r.returncode == 0 and "first-call-under-capture: ok" in r.stdout


if __name__ == "__main__" and "--first-call-captured" in sys.argv:
    _first_call_captured()
