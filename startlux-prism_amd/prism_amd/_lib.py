"""Loader for libprism_amd.so, the gfx950 kernels' C ABI (include/prism_amd.h).

The library is built in-tree by startlux-prism_amd/build.py.  There is no fallback: if the library is missing or
the device is not a gfx950, every op raises.  Tensors are handed over as raw device pointers plus sizes, and the
kernels launch on torch's current HIP stream of the tensors' device.
"""
import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libprism_amd.so")

_i64, _p, _int = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int

_SIGS = {
    "prism_version": (_int, []),
    "prism_error_string": (ctypes.c_char_p, [_int]),
    "prism_quant_rows_i8": (_int, [_p, _i64, _p, _p, _p, _p, _i64, _i64, _p]),
    "prism_quant_rows_groups": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "prism_quant_rows_g": (_int, [_p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "prism_w8a8_gemm": (_int, [_p, _p, _i64, _i64, _p, _p, _int, _p, _i64, _p, _i64, _i64, _i64, _i64, _int, _int,
                               _p]),
    "prism_q8_0_pack": (_int, [_p, _p, _p, _p, _i64, _i64, _p]),
    "prism_w8a8_q8_0_packed_gemm": (_int, [_p, _p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _int, _int, _p,
                                           _i64, _p]),
    "prism_w8a8_q8_0_packed_workspace_bytes": (_i64, [_i64, _i64]),
    "prism_w8a8_q8_0_packed_gemm_noalloc": (_int, [_p, _p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _int, _int,
                                                   _p]),
    "prism_q4k_pack": (_int, [_p, _p, _p, _i64, _i64, _p]),
    "prism_w4a8_q4k_gemm": (_int, [_p, _p, _i64, _p, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _int, _int, _p, _i64,
                                   _p]),
    "prism_q6k_pack": (_int, [_p, _p, _p, _i64, _i64, _p]),
    "prism_w4a8_q6k_gemm": (_int, [_p, _p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _int, _int, _p]),
    "prism_i8_pack": (_int, [_p, _p, _i64, _i64, _p]),
    "prism_w8a8_pc_packed_gemm": (_int, [_p, _p, _i64, _p, _p, _int, _p, _i64, _p, _i64, _i64, _i64, _int, _int, _p]),
    "prism_w8a8_pc_packed_gemm_split": (_int, [_p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _int, _p]),
    "prism_w8a8_pc_packed_gemm_ws": (_int, [_p, _p, _i64, _p, _p, _int, _p, _i64, _p, _i64, _i64, _i64, _int, _int,
                                            _p, _i64, _p]),
    "prism_w8a8_pc_split_workspace_bytes": (_i64, [_i64, _i64]),
    "prism_norm_quant": (_int, [_p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, ctypes.c_float, _int, _p]),
    "prism_norm_quant_fold": (_int, [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, ctypes.c_float, _int, _p, _i64, _i64,
                                     _int, _p, _i64, _p, _int, _p]),
    "prism_fold_parts": (_int, [_p, _i64, _p, _i64, _i64, _int, _p, _i64, _p, _int, _p, _i64, _i64, _p]),
    "prism_swiglu_quant": (_int, [_p, _int, _i64, _p, _p, _p, _p, _p, _i64, _i64, _int, _p]),
    "prism_gated_norm_quant": (_int, [_p, _i64, _p, _int, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                                      ctypes.c_float, _int, _p]),
    "prism_mxfp4_pack": (_int, [_p, _i64, _p, _p, _i64, _i64, _int, _p]),
    "prism_mxfp4_repack": (_int, [_p, _p, _p, _p, _i64, _i64, _p]),
    "prism_mxfp4_quant_act": (_int, [_p, _int, _i64, _p, _p, _p, _p, _i64, _i64, _int, _p]),
    "prism_probe_mfma": (_int, [_int, _i64, _i64, _p, _p]),
    "prism_probe_mfma_ops": (_i64, [_int]),
    "prism_probe_read": (_int, [_p, _i64, _i64, _p, _p]),
    "prism_mxfp4_gemm": (_int, [_p, _p, _int, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _int, _int, _p]),
    "prism_mxfp4_gemm_ws": (_int, [_p, _p, _int, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _int, _int, _p, _i64, _p]),
    "prism_mxfp4_split_workspace_bytes": (_i64, [_i64, _i64]),
}

_lib = None


class PrismError(RuntimeError):
    pass


def lib():
    """The loaded library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PrismError(f"{LIB_PATH} is missing: build it with python startlux-prism_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def exported_symbols():
    return list(_SIGS)


_checked = set()


def _check_device(dev):
    if dev.type != "cuda":
        raise PrismError(f"prism_amd ops run on the GPU; got a tensor on {dev}")
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _checked:
        arch = torch.cuda.get_device_properties(idx).gcnArchName.split(":")[0]
        if arch != "gfx950":
            raise PrismError(f"prism_amd is built for gfx950 (MI355X); device {idx} is {arch}")
        _checked.add(idx)
    return idx


def stream_of(t):
    """torch's current stream handle on t's device."""
    idx = _check_device(t.device)
    return ctypes.c_void_p(torch.cuda.current_stream(idx).cuda_stream)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().prism_error_string(rc).decode()
        raise PrismError(f"{name}: {msg} (code {rc})")
