"""torch_ops.load() registers the reference's op schemas (csrc/w8a8_gemm.cu:794-797, csrc/w4a8_gemm.cu:963-966)
under torch.ops.startlux_prism, argument for argument (no GPU needed: registration only)."""
import torch

from prism_amd import torch_ops


def _args(schema):
    return [(a.name, str(a.type), a.default_value, a.alias_info is not None and a.alias_info.is_write)
            for a in schema.arguments]


def test_schemas_match_the_reference():
    ops = torch_ops.load()
    assert torch_ops.load() is ops                       # registering twice is a no-op
    w8 = _args(ops.w8a8_gemm.default._schema)
    assert [n for n, *_ in w8] == ["a", "sa", "w", "sw", "out", "n_rows", "epi", "cfg", "split", "stages", "mode",
                                   "workspace", "counters", "slot_stride", "pdl"]
    assert [n for n, _, _, wr in w8 if wr] == ["out", "workspace", "counters"]
    assert {n: d for n, _, d, _ in w8 if d is not None} == {"mode": 2, "slot_stride": 0, "pdl": 0}
    assert [n for n, t, _, _ in w8 if t == "Optional[Tensor]"] == ["workspace", "counters"]
    sk = _args(ops.w8a8_gemm_sk.default._schema)
    assert [n for n, *_ in sk] == ["a", "sa", "w", "sw", "out", "n_rows", "ws", "counters", "epi", "cfg", "stages",
                                   "grid", "sk_waves", "pdl"]
    w4 = _args(ops.w4a8_gemm.default._schema)
    assert [n for n, *_ in w4] == ["a", "a_s", "xs", "wq", "wsc", "wmn", "wd", "wdm", "out", "n_rows", "kind", "epi",
                                   "cfg", "stages", "pdl"]
    assert [n for n, t, _, _ in w4 if t == "Optional[Tensor]"] == ["wmn", "wdm"]
    assert [n for n, _, _, wr in w4 if wr] == ["out"]
    for op in (ops.w8a8_gemm, ops.w8a8_gemm_sk, ops.w4a8_gemm):
        assert len(op.default._schema.returns) == 0
