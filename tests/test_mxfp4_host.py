"""Host logic of the MXFP4 module (no GPU): `mxfp4.panels_to_rows` undoes the e4m3 panel layout the header and
mx_act_panel_offset document (byte 1024 h + 16 (16 p + r) + i of chunk st of block b holds row 16 b + r, input
128 st + 64 h + 16 p + i), for row counts that are and are not multiples of 16; gemm refuses row-major weights;
the engine's CUTLASS hooks are inert."""
import numpy as np
import pytest
import torch

from prism_amd import mxfp4 as MX


def _panels_by_formula(rows):
    """The panel buffer of a row-major [n, k] byte matrix, element by element from the documented formula."""
    n, k = rows.shape
    nb = (n + 15) // 16
    pan = np.zeros((nb, k // 128, 2048), np.uint8)
    for r in range(n):
        for kk in range(k):
            b, rr, st, h, p, i = r // 16, r % 16, kk // 128, (kk // 64) % 2, (kk // 16) % 4, kk % 16
            pan[b, st, 1024 * h + 16 * (16 * p + rr) + i] = rows[r, kk]
    return pan


@pytest.mark.parametrize("n,k", [(1, 128), (16, 256), (21, 384)])
def test_panels_to_rows_inverts_the_layout(n, k):
    rows = np.random.default_rng(n + k).integers(0, 256, size=(n, k), dtype=np.uint8)
    pan = torch.from_numpy(_panels_by_formula(rows))
    assert tuple(pan.shape) == MX._panel_shape(n, k)
    assert np.array_equal(MX.panels_to_rows(pan, n).numpy(), rows)


def test_act_panels_shape_and_k_rule():
    assert tuple(MX.act_panels(33, 256, "cpu").shape) == (3, 2, 2048)
    with pytest.raises(ValueError):
        MX.act_panels(16, 192, "cpu")


def test_mxfp4_gemm_refuses_row_major_weights():
    """A row-major MX4 (the reference pack's or a side file's bytes) is refused with the conversion to use, never
    read as the device layout."""
    n, k = 32, 256
    w = MX.MX4(torch.zeros(n, k // 2, dtype=torch.uint8), torch.zeros(n, k // 32, dtype=torch.uint8), n, k)
    a = torch.zeros(4, k, dtype=torch.uint8)
    s = torch.zeros(4, k // 32, dtype=torch.uint8)
    out = torch.zeros(4, n, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="from_rows"):
        MX.gemm(a, s, w, out, 4)


def test_cutlass_hooks_are_inert():
    """The engine's load_mlp asks cutlass_enabled() and may call cutlass_prepare (engine/mxfp4.py:77-81)."""
    assert MX.cutlass_enabled() is False
    w = MX.MX4(torch.zeros(1), torch.zeros(1), 16, 128)
    assert MX.cutlass_prepare(w) is w
