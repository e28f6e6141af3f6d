"""GGUF tensors to the device layouts the GEMMs stream, once at load: the step of gguf_weights.py:221-236 (_q8, _kq:
a tensor's blocks as read from the file, ggml dims [inputs, outputs]) followed by the repacks of kernels/w8a8.py:274-286
(weight_from_q8) and kernels/w4a8.py:70-94 (repack).  Parsing the GGUF file itself (header, metadata, offsets) is the
caller's: this module starts from one tensor's bytes.
"""
import math

import numpy as np
import torch

from . import gguf_formats as GF
from . import w4a8 as KW4
from . import w8a8 as KW

GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = GF.GGML_Q8_0, GF.GGML_Q4_K, GF.GGML_Q6_K
BLOCKS = {GGML_Q8_0: (32, GF.Q8_0_BYTES), GGML_Q4_K: (256, GF.Q4_K_BYTES), GGML_Q6_K: (256, GF.Q6_K_BYTES)}


def from_gguf(raw, ggml_type, dims, device, gk=32):
    """raw: the tensor's bytes as stored (uint8 numpy array or torch tensor, any shape); ggml_type; dims: ggml dims
    (inputs first).  Returns the GEMM's weight operand on `device`: for Q8_0, weight_from_q8(q8, gk) (gk = 32: the
    packed Q8_0 layout; gk = K: per channel); for Q4_K / Q6_K, the W4A8 W4."""
    if ggml_type not in BLOCKS:
        raise ValueError(f"ggml type {ggml_type}: the hot path takes Q8_0, Q4_K and Q6_K tensors")
    k, n = int(dims[0]), int(math.prod(int(d) for d in dims[1:]))
    per, nb = BLOCKS[ggml_type]
    if k % per:
        raise ValueError(f"{k} inputs are not whole {per}-value blocks")
    t = torch.from_numpy(np.ascontiguousarray(raw).view(np.uint8)) if isinstance(raw, np.ndarray) else raw
    if t.dtype != torch.uint8 or t.numel() != n * (k // per) * nb:
        raise ValueError(f"expected {n * (k // per) * nb} bytes of blocks, got {t.numel()} ({t.dtype})")
    t = t.reshape(n, k // per, nb).to(device)
    if ggml_type == GGML_Q8_0:
        return KW.weight_from_q8(GF.q8_0_from_gguf_bytes(t, n, k), gk)
    return KW4.repack(GF.KQuant(t, ggml_type, k))
