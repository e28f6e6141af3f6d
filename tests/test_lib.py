"""The C-ABI library builds for gfx950, loads without a GPU, and exports every entry point include/prism_amd.h
declares (no compute calls here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "prism_amd.h")


def _declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^PRISM_API\s[\w\s\*]*?\b(prism_\w+)\s*\(", src, re.M)))


def test_header_declares_entry_points():
    names = _declared()
    for n in ("prism_quant_rows_i8", "prism_w8a8_gemm", "prism_w4a8_q4k_gemm", "prism_error_string"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from prism_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libprism_amd.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(L.LIB_PATH)
    for n in _declared():
        assert hasattr(lib, n), n
    L.lib()
    assert set(L.exported_symbols()) == set(_declared())
    assert L.lib().prism_version() >= 100
    assert L.lib().prism_error_string(1) == b"unsupported shape"


def test_library_has_no_cpu_fallback_symbols():
    """The product library holds only gfx950 device code plus the launch shims: no oracle symbols."""
    from prism_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libprism_amd.so not built")
    lib = ctypes.CDLL(L.LIB_PATH)
    assert not hasattr(lib, "orc_w8a8_gemm")


def test_kquant_reference_field_order():
    """KQuant(raw, type, k) in the reference's positional order with ggml ids (gguf_weights.py:100-112); the old
    (raw, k, type) order or an unknown type raises instead of silently taking k = 12."""
    import torch
    from prism_amd import gguf_formats as GF
    raw = torch.zeros(16, 2, 144, dtype=torch.uint8)
    kq = GF.KQuant(raw, 12, 512)
    assert kq.kind == "q4k" and kq.shape == (16, 512)
    assert GF.KQuant(torch.zeros(16, 2, 210, dtype=torch.uint8), GF.GGML_Q6_K, 512).kind == "q6k"
    assert GF.KQuant(raw, "q4k", 512).kind == "q4k"
    with pytest.raises(ValueError):
        GF.KQuant(raw, 512, 12)
    with pytest.raises(ValueError):
        GF.KQuant(raw, 8, 512)
