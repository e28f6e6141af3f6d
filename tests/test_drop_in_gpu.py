"""The engine's own call shapes through the drop-in, as the reference's engine makes them.

* W4A8: engine/model.py:287 builds `KW4.segments(m, dev)` from the reference's gguf_weights.KQuant objects, whose
  fields are (raw, type, k) with type the ggml id (12 = Q4_K, 14 = Q6_K; gguf_weights.py:100-112).  A local dataclass
  of that shape (not the reference module) goes through segments -> gemm_segs on a projection mixing Q4_K and Q6_K,
  with the last-layer row slice seg_rows (engine/model.py:958).
* W8A8 per channel: engine/model.py:848-852 passes smooth_quant's plain int8 [N, K] weights and fp32 [N] row scales
  (engine/model.py:72-82), row-sliced for the last layer's queries, with gk = K."""
import dataclasses

import numpy as np
import pytest
import torch

import oracle as O
from _inputs import acts_bf16, rng, weights_f32

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


@dataclasses.dataclass
class EngineKQuant:
    """The shape of the reference engine's gguf_weights.KQuant: raw uint8 [n, k/256, block bytes], ggml type id, k."""
    raw: torch.Tensor
    type: int
    k: int

    def to(self, device):
        return EngineKQuant(self.raw.to(device), self.type, self.k)


def test_engine_kquant_segments(dev):
    from prism_amd import w4a8 as KW4
    M, K = 9, 1536
    parts = [(12, 64), (14, 48), (12, 32), (12, 16)]        # q | k (Q6_K) | v | z, as a Q4_K_M file mixes them
    raws = [O.q4k_quantize(weights_f32(n, K, seed=500 + i)) if t == 12 else
            O.q6k_quantize(weights_f32(n, K, seed=500 + i)) for i, (t, n) in enumerate(parts)]
    kqs = [EngineKQuant(torch.from_numpy(r), t, K) for r, (t, _) in zip(raws, parts)]     # on the host, as loaded
    segs = KW4.segments(kqs, dev)
    assert [(w.kind, w.n, off) for w, off in segs] == [("q4k", 64, 0), ("q6k", 48, 64), ("q4k", 48, 112)]
    width = KW4.seg_width(segs)
    xq, a, xs = O.quant_rows_g(O.bf16_to_f32(acts_bf16(M, K, seed=510)), 256)
    wants = [O.w4a8_gemm(xq, a, xs, O.q4k_repack(r)) if t == 12 else O.w4a8_gemm_q6k(xq, a, O.q6k_repack(r))
             for r, (t, _) in zip(raws, parts)]
    want = np.concatenate(wants, 1)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    out = torch.zeros(M, width, dtype=torch.bfloat16, device=dev)
    KW4.gemm_segs(_t(xq, dev), _t(a, dev), _t(xs, dev), segs, out, n)
    torch.cuda.synchronize()
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), want)
    # the last layer's slice of the fused projection (engine/model.py:958): columns 64.. only
    part = torch.zeros(M, width - 64, dtype=torch.bfloat16, device=dev)
    KW4.gemm_segs(_t(xq, dev), _t(a, dev), _t(xs, dev), KW4.seg_rows(segs, 64, width), part, n)
    torch.cuda.synchronize()
    assert np.array_equal(part.view(torch.int16).cpu().numpy().view(np.uint16), want[:, 64:])


@pytest.mark.parametrize("form", ["plain", "packed_at_load"])
def test_engine_per_channel_plain_weights(dev, form):
    """KW.gemm(xq, as_, lw["qkv_q"][qn:], lw["qkv_s"][qn:], proj[:, qn:], tok, hidden) with smooth_quant's int8 [N, K]
    and fp32 [N] as they are (plain), or after the one load-time line `wq = KW.pack_i8(wq, ws)` (packed_at_load: the
    engine's calls and row slices unchanged, the packed per-channel kernels)."""
    from prism_amd import w8a8 as KW
    M, K, N, qn = 21, 2048, 384, 128
    g = rng(520)
    wf = torch.from_numpy(weights_f32(N, K, seed=521))
    ws = wf.abs().amax(1).clamp_min(1e-8) / 127.0                 # smooth_quant's row scales, fp32 [N]
    wq = torch.round(wf / ws[:, None]).clamp(-127, 127).to(torch.int8).contiguous()
    a, sa = O.quant_rows_i8(acts_bf16(M, K, seed=522))
    want = O.w8a8_gemm(a, sa, wq.numpy(), ws.numpy().reshape(N, 1), K, epi=0)
    wd, wsd = wq.to(dev), ws.to(dev)
    if form == "packed_at_load":
        wd = KW.pack_i8(wd, wsd)
        assert wd.shape == (N, K) and wd[qn:].shape == (N - qn, K)
    ad, sad = _t(a, dev), _t(sa, dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    proj = torch.full((M, N), 7, dtype=torch.int16, device=dev).view(torch.bfloat16)
    KW.gemm(ad, sad, wd, wsd, proj, n, K)
    KW.gemm(ad, sad, wd[qn:], wsd[qn:], proj[:, qn:], n, K)     # the row slice, into a column slice of proj
    base = g.standard_normal((M, N)).astype(np.float32)
    h = _t(base, dev)
    KW.gemm(ad, sad, wd, wsd, h, n, K, epi=1)                      # the residual add (o / down projections)
    torch.cuda.synchronize()
    assert np.array_equal(proj.view(torch.int16).cpu().numpy().view(np.uint16), want)
    want1 = O.w8a8_gemm(a, sa, wq.numpy(), ws.numpy().reshape(N, 1), K, epi=1, out=base.copy())
    assert np.array_equal(h.cpu().numpy(), want1)
