"""Per-shape kernel choice from tables measured on this GPU's model: the MI355X counterpart of the reference's tuned
dispatch (kernels/w8a8.py:144-168 _table / _choice, kernels/w4a8.py:296-326 _table / pick_cuda).

Tables (JSON next to this module, written by prism_amd.tune on the GPU they describe):
  gemm_table_<tag>.json   W8A8, per channel (gk = K): "NxK" -> {M: [kernel]}, looked up at the measured M nearest
                          to the request in log scale (kernels/w8a8.py:163-168).
  q8_table_<tag>.json     W8A8 on Q8_0 weights (gk = 32, the packed layout): keyed and looked up as the gemm table.
                          The reference serves gk = 32 with one Triton rule and no table.
  w4a8_table_<tag>.json   W4A8: "kind,N,K" (kind q4k or q6k) -> {M: [kernel]}, looked up at the smallest measured M
                          >= the request, else the largest (kernels/w4a8.py:309-316).
<tag> is "mi355x" on gfx950.  A kernel is a name of the op's KERNELS ("tile", "decode", "mid", "stream", and "split" for the per-channel
split decode).  STARTLUX_PRISM_GEMM_TABLE,
STARTLUX_PRISM_Q8_TABLE and STARTLUX_PRISM_W4A8_TABLE name other files, or "off"; without a table (or for a shape it does not
hold) the library's own rule picks (kernel "auto").  Every kernel computes the same bits, so a table changes speed
only.
"""
import functools
import json
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))
ENV = {"gemm_table": "STARTLUX_PRISM_GEMM_TABLE", "q8_table": "STARTLUX_PRISM_Q8_TABLE", "w4a8_table": "STARTLUX_PRISM_W4A8_TABLE"}


@functools.lru_cache(None)
def gpu_tag():
    """The table tag of GPU 0: "mi355x" for gfx950 (MI355X / MI350X), else its architecture name."""
    import torch
    if not torch.cuda.is_available():
        return None
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    return "mi355x" if arch == "gfx950" else arch


def table_path(prefix):
    env = os.environ.get(ENV[prefix])
    if env:
        return env
    tag = gpu_tag()
    return None if tag is None else os.path.join(HERE, f"{prefix}_{tag}.json")


@functools.lru_cache(None)
def load(prefix):
    """{key: [(M, kernel)] sorted by M} of a table, {} when off or absent."""
    path = table_path(prefix)
    if path is None or path == "off" or not os.path.exists(path):
        return {}
    raw = json.load(open(path))["table"]
    return {k: sorted((int(m), c[0]) for m, c in v.items()) for k, v in raw.items()}


def _nearest(entries, M):
    return min(entries, key=lambda e: abs(math.log(e[0]) - math.log(max(M, 1))))[1]


def _at_least(entries, M):
    return next((c for m, c in entries if m >= M), entries[-1][1])


def w8a8_kernel(N, K, M, gk):
    """The table's kernel for a W8A8 product (gk = K: per channel; gk = 32: Q8_0), or "auto"."""
    prefix = "gemm_table" if gk == K else ("q8_table" if gk == 32 else None)
    entries = load(prefix).get(f"{N}x{K}") if prefix else None
    return _nearest(entries, M) if entries else "auto"


def w4a8_kernel(kind, N, K, M):
    """The table's kernel for a W4A8 product on kind ("q4k" / "q6k") weights, or "auto"."""
    entries = load("w4a8_table").get(f"{kind},{N},{K}")
    return _at_least(entries, M) if entries else "auto"
