"""The C ABI's argument checks, run on the CPU: every entry point validates its pointers, sizes, alignment and kernel
choice before it touches the GPU, and answers with the documented code (PRISM_ERR_ARG / _SHAPE / _ALIGN), or
PRISM_OK with nothing launched for zero rows.  The pointers here are placeholders that are never dereferenced."""
import os

import pytest

OK, SHAPE, ALIGN, ARG = 0, 1, 2, 3
P = 0x100000          # a 16-byte-aligned placeholder address
U = 0x100001          # a misaligned one


@pytest.fixture(scope="module")
def lib():
    from prism_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libprism_amd.so not built (run __graft_entry__.build())")
    return L.lib()


def test_q8_0_packed_gemm_checks(lib):
    f = lib.prism_w8a8_q8_0_packed_gemm

    def call(a=P, qt=P, out=P, M=16, N=64, K=256, epi=0, kernel=-1, ws=None, wsb=0):
        return f(a, P, 1, qt, P, out, N, P, M, N, K, epi, kernel, ws, wsb, None)
    assert call(a=None) == ARG
    assert call(epi=2) == ARG
    assert call(K=192) == SHAPE                  # K % 128
    assert call(N=40) == SHAPE                   # N % 16
    assert call(a=U) == ALIGN
    assert call(qt=U) == ALIGN
    assert call(kernel=5) == ARG
    assert call(kernel=4) == ARG                 # the balanced decode kernel needs a workspace
    assert call(kernel=4, ws=P, wsb=16) == ARG   # ... of prism_w8a8_q8_0_packed_workspace_bytes
    assert call(kernel=4, M=17, ws=P, wsb=1 << 20) == SHAPE      # it holds up to 16 rows
    assert lib.prism_w8a8_q8_0_packed_workspace_bytes(64, 256) == 4 * 16 * 16 * 8
    assert call(kernel=1, M=65) == ARG           # the decode kernels hold up to 64 rows
    assert call(M=0) == OK
    assert call(M=0, kernel=3) == OK             # the reassociated prefill kernel is a valid choice


def test_pack_checks_match_the_gemms(lib):
    """The Q8_0 pack takes the packed GEMM's K rule (K % 128), so every packed operand is usable; the per-channel
    pack keeps K % 64, its GEMM's rule."""
    assert lib.prism_q8_0_pack(P, P, P, P, 64, 192, None) == SHAPE
    assert lib.prism_q8_0_pack(P, P, P, P, 40, 256, None) == SHAPE
    assert lib.prism_q8_0_pack(U, P, P, P, 64, 256, None) == ALIGN
    assert lib.prism_i8_pack(P, P, 64, 96, None) == SHAPE
    assert lib.prism_i8_pack(U, P, 64, 192, None) == ALIGN


def test_w4a8_q4k_gemm_checks(lib):
    f = lib.prism_w4a8_q4k_gemm

    def call(xq=P, qv=P, M=16, N=64, K=512, epi=0, kernel=-1, ws=None, ws_bytes=0):
        return f(xq, P, 0, P, qv, P, P, N, P, M, N, K, epi, kernel, ws, ws_bytes, None)
    assert call(xq=None) == ARG
    assert call(K=384) == SHAPE                  # K % 256
    assert call(qv=U) == ALIGN
    assert call(epi=3) == ARG
    assert call(kernel=3) == ARG
    assert call(kernel=2) == ARG                 # the balanced kernel needs its workspace
    assert call(kernel=2, ws=P, ws_bytes=64) == ARG                  # too small: 4 workgroups x 2 KB
    assert call(kernel=2, M=17, ws=P, ws_bytes=1 << 20) == SHAPE     # at most 16 rows
    assert call(kernel=2, K=1 << 16, ws=P, ws_bytes=1 << 20) == SHAPE  # the activation image exceeds LDS
    assert call(kernel=1, M=17) == ARG
    assert call(M=0) == OK


def test_mxfp4_gemm_checks(lib):
    f = lib.prism_mxfp4_gemm

    def call(aq=P, fmt=0, M=16, N=64, K=256, epi=0, out=P, kernel=-1):
        return f(aq, P, fmt, P, P, out, N, P, M, N, K, epi, kernel, None)
    assert call(aq=None) == ARG
    assert call(fmt=2) == ARG                    # neither e4m3 (0), e4m3 panels (1) nor e2m1 (4)
    assert call(fmt=1, kernel=1) == SHAPE        # panel activations: the tile kernel only
    assert call(fmt=1, M=0) == OK
    assert call(K=192) == SHAPE                  # K % 128
    assert call(aq=U) == ALIGN
    assert call(epi=1, out=P + 8) == ALIGN       # the fp32 residual needs 16-byte rows
    assert call(M=0) == OK


def test_mxfp4_split_checks(lib):
    f = lib.prism_mxfp4_gemm_ws

    def call(fmt=0, M=16, N=64, K=2048, kernel=2, work=P, work_bytes=1 << 20):
        return f(P, P, fmt, P, P, P, N, P, M, N, K, 0, kernel, work, work_bytes, None)
    assert call(work=None, work_bytes=0) == ARG     # the split decode needs its workspace
    assert call(work_bytes=1024) == SHAPE           # 2 segments x 4 tiles x 1 KB
    assert call(M=17) == SHAPE                      # one 16-row block
    assert call(fmt=4) == SHAPE                     # e4m3 row-major activations only
    assert call(fmt=1) == SHAPE                     # panels: the tile kernel only
    assert call(work=U) == ALIGN                    # 16-byte aligned segment sums
    assert call(M=0) == OK
    b = lib.prism_mxfp4_split_workspace_bytes
    assert b(5120, 5120) == 5 * 320 * 1024 and b(64, 1024) == 16 and b(60, 128) == 0 and b(64, 192) == 0


def test_mxfp4_quant_act_checks(lib):
    f = lib.prism_mxfp4_quant_act
    assert f(P, 0, 256, None, P, P, None, 16, 256, 2, None) == ARG            # fmt
    assert f(P, 0, 160, None, P, P, None, 16, 160, 1, None) == SHAPE          # panels: K % 128
    assert f(P, 0, 256, None, P, P, None, 0, 256, 1, None) == OK


def test_quant_and_split_checks(lib):
    q = lib.prism_quant_rows_i8
    assert q(None, 64, None, P, P, P, 4, 64, None) == ARG
    assert q(P, 64, None, P, P, P, 4, 60, None) == SHAPE     # K % 8
    assert q(U, 64, None, P, P, P, 4, 64, None) == ALIGN
    assert q(P, 64, None, P, P, P, 0, 64, None) == OK
    s = lib.prism_w8a8_pc_packed_gemm_split
    assert s(P, P, P, 64 * 64, 64, P, 64, 64, 1024, 0, None) == ARG           # split < 1
    assert s(P, P, P, 10, 64, P, 64, 64, 1024, 2, None) == SHAPE              # the slots would overlap
    assert s(P, P, P, 64 * 64, 64, P, 64, 64, 64, 2, None) == SHAPE           # fewer 64-input chunks than parts
    assert s(P, P, U, 64 * 64, 64, P, 64, 64, 1024, 2, None) == ALIGN
    assert s(P, P, P, 64 * 64, 64, P, 0, 64, 1024, 2, None) == OK
