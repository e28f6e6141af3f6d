"""PackedPC row slices (host logic, no GPU): w[r0:r1] is a view of whole 16-row chunks with its scales, the form the
engine's fused-projection slice lw["qkv_q"][qn:] takes after the load-time pack_i8."""
import pytest
import torch

from prism_amd import w8a8 as KW


def _packed(n=64, k=128):
    qt = torch.arange(n // 16 * (k // 64) * 64 * 16, dtype=torch.int32).to(torch.int8).view(n // 16, k // 64, 64, 16)
    ws = torch.arange(n, dtype=torch.float32).view(n, 1)
    return KW.PackedPC(qt, ws, n, k)


def test_row_slice_is_a_view_of_whole_chunks():
    w = _packed()
    s = w[32:]
    assert isinstance(s, KW.PackedPC) and s.shape == (32, 128) and s.n == 32 and s.k == 128
    assert s.qt.data_ptr() == w.qt[2].data_ptr() and s.qt.is_contiguous()
    assert torch.equal(s.ws.view(-1), torch.arange(32, 64, dtype=torch.float32))
    assert w[16:48].qt.shape[0] == 2


def test_integer_index_keeps_tuple_fields():
    w = _packed()
    assert w[0] is w.qt and w[2] == 64


@pytest.mark.parametrize("key", [slice(8, None), slice(0, 40), slice(0, 64, 2), slice(32, 32)])
def test_partial_chunks_refused(key):
    with pytest.raises(ValueError):
        _packed()[key]
