"""GGUF weight formats on the hot path: Q8_0 (32 values: fp16 scale + 32 int8), Q4_K (256 values: fp16 d, dmin,
12 bytes of 6-bit sub-block scales and mins, 128 bytes of 4-bit quants) and Q6_K (256 values: 128 bytes of low 4
bits, 64 of high 2 bits, 16 int8 scales of 16 values, fp16 d), as torch tensors on any device.

Restated from StartLux-Prism gguf.py:413-416 (block sizes), gguf_weights.py:30-46 (Q8), :56-70 (get_scale_min_k4,
Q4_K dequantization), :85-97 (Q6_K dequantization), :100-133 (KQuant, as_q8) and :221-227 (_q8: 34-byte blocks
split into the qs / d planes).  The quantizers produce synthetic weights for tests and benchmarks; the reference
itself only reads these formats from files (its Q8_0 quantizer as_q8 is followed here; the Q4_K and Q6_K quantizers
are this build's own).
"""
import dataclasses

import torch

QK = 32            # Q8_0 block
QK_K = 256         # k-quant super-block
Q8_0_BYTES = 34
Q4_K_BYTES = 144
Q6_K_BYTES = 210
GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 8, 12, 14        # ggml type ids (gguf.py:13-15)
_KIND = {GGML_Q4_K: "q4k", GGML_Q6_K: "q6k", "q4k": "q4k", "q6k": "q6k"}


def kquant_kind(t):
    """A k-quant type, as the reference's ggml id (12, 14) or this build's name ("q4k", "q6k") -> the name."""
    try:
        return _KIND[int(t) if not isinstance(t, str) else t]
    except (KeyError, TypeError, ValueError):
        raise ValueError(f"k-quant type {t!r}: Q4_K (12) and Q6_K (14) are supported") from None


@dataclasses.dataclass
class Q8:
    """A Q8_0 matrix [n, k]: qs int8 [n, k], d fp16 [n, k / 32] (gguf_weights.py:30-46)."""
    qs: torch.Tensor
    d: torch.Tensor

    @property
    def shape(self):
        return tuple(self.qs.shape)

    def to(self, device):
        return Q8(self.qs.to(device), self.d.to(device))

    def dequant(self, dtype=torch.float32, rows=None):
        qs, d = (self.qs, self.d) if rows is None else (self.qs[rows], self.d[rows])
        w = qs.view(*qs.shape[:-1], -1, QK).to(torch.float32) * d.to(torch.float32).unsqueeze(-1)
        return w.reshape(qs.shape).to(dtype)

    def nbytes_gguf(self):
        return self.qs.numel() // QK * Q8_0_BYTES


def quantize_q8_0(w):
    """fp32 [n, k] -> Q8 by llama.cpp's Q8_0 rule as the reference writes it (gguf_weights.py:129-131):
    dh = fp16(amax / 127), q = clamp(round(w * (1 / float(dh))), -127, 127) (round half to even)."""
    n, k = w.shape
    b = w.to(torch.float32).reshape(n, k // QK, QK)
    dh = (b.abs().amax(-1) / 127).half()
    inv = torch.where(dh > 0, 1.0 / dh.float(), torch.zeros_like(dh, dtype=torch.float32))
    qs = torch.round(b * inv[..., None]).clamp(-127, 127).to(torch.int8).reshape(n, k)
    return Q8(qs.contiguous(), dh.contiguous())


def q8_0_from_gguf_bytes(raw, n, k):
    """uint8 [n, k/32, 34] GGUF blocks -> Q8 planes (gguf_weights.py:221-227)."""
    raw = raw.reshape(n, k // QK, Q8_0_BYTES)
    d = raw[..., :2].contiguous().view(torch.float16).reshape(n, k // QK)
    qs = raw[..., 2:].contiguous().view(torch.int8).reshape(n, k)
    return Q8(qs.contiguous(), d.contiguous())


def q8_0_to_gguf_bytes(q8):
    """Q8 -> uint8 [n, k/32, 34] GGUF blocks (the inverse of q8_0_from_gguf_bytes)."""
    n, k = q8.shape
    d = q8.d.contiguous().view(torch.uint8).reshape(n, k // QK, 2)
    qs = q8.qs.contiguous().view(torch.uint8).reshape(n, k // QK, QK)
    return torch.cat([d, qs], -1).contiguous()


def scale_min_k4(s):
    """The 8 six-bit scales and mins of Q4_K super-blocks (ggml get_scale_min_k4, gguf_weights.py:56-60):
    s int32 [..., 12] -> (sc, mn) int32 [..., 8]."""
    sc = torch.cat([s[..., 0:4] & 63, (s[..., 8:12] & 0xF) | ((s[..., 0:4] >> 6) << 4)], -1)
    mn = torch.cat([s[..., 4:8] & 63, (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)], -1)
    return sc, mn


@dataclasses.dataclass
class KQuant:
    """A k-quant matrix [n, k] as its raw super-blocks: raw uint8 [n, k / 256, 144] for Q4_K, [n, k / 256, 210]
    for Q6_K.  Fields and their positional order are the reference's (gguf_weights.py:100-112): type is the ggml id
    (GGML_Q4_K = 12, GGML_Q6_K = 14); the names "q4k" / "q6k" are accepted too."""
    raw: torch.Tensor
    type: int
    k: int

    def __post_init__(self):
        kquant_kind(self.type)
        if isinstance(self.k, str) or int(self.k) % QK_K:
            raise ValueError(f"KQuant(raw, type, k): k = {self.k!r} must be a multiple of {QK_K}")

    @property
    def kind(self):
        return kquant_kind(self.type)

    @property
    def shape(self):
        return (self.raw.shape[0], self.k)

    def to(self, device):
        return KQuant(self.raw.to(device), self.type, self.k)

    def dequant(self, dtype=torch.float32):
        """Q4_K: y = (d sc) q - (dmin m) in fp32, ggml's order of products (gguf_weights.py:63-70).  Q6_K:
        y = (d sc) (q - 32) (:85-97)."""
        if self.kind == "q6k":
            b = self.raw.reshape(-1, Q6_K_BYTES)
            sc = b[:, 192:208].contiguous().view(torch.int8).float()
            d = b[:, 208:210].contiguous().view(torch.float16).float()
            return ((d * sc).repeat_interleave(16, 1) * q6k_values(b).float()).reshape(self.raw.shape[0], self.k).to(dtype)
        b = self.raw.reshape(-1, Q4_K_BYTES)
        d = b[:, 0:2].contiguous().view(torch.float16).float()
        dmin = b[:, 2:4].contiguous().view(torch.float16).float()
        sc, mn = scale_min_k4(b[:, 4:16].to(torch.int32))
        q = b[:, 16:144].to(torch.int32).view(-1, 4, 32)
        q = torch.stack([q & 0xF, q >> 4], 2).view(-1, 8, 32).float()
        y = (d * sc.float())[:, :, None] * q - (dmin * mn.float())[:, :, None]
        return y.reshape(self.raw.shape[0], self.k).to(dtype)

    def nbytes_gguf(self):
        return self.raw.numel()


def quantize_q4k(w):
    """fp32 [n, k] -> KQuant: this build's Q4_K quantizer.  Per sub-block j of 32: lo = min(0, min x),
    scale_j = (max x - lo) / 15, min_j = -lo; d = fp16(max scale / 63), dmin = fp16(max min / 63);
    sc_j = clamp(rint(scale_j / d), 0, 63), m_j = clamp(rint(min_j / dmin), 0, 63);
    q = clamp(rint((x + dmin m_j) / (d sc_j)), 0, 15)."""
    n, k = w.shape
    x = w.to(torch.float32).reshape(n, k // QK_K, 8, 32)
    lo = torch.clamp(x.amin(-1), max=0.0)
    hi = x.amax(-1)
    scale = (hi - lo) / 15.0
    mn = -lo
    dh = (scale.amax(-1) / 63.0).half()
    dmh = (mn.amax(-1) / 63.0).half()
    d, dmin = dh.float()[..., None], dmh.float()[..., None]
    zero = torch.zeros_like(scale)
    sc = torch.where(d > 0, torch.round(scale / torch.where(d > 0, d, 1.0)), zero).clamp(0, 63)
    m = torch.where(dmin > 0, torch.round(mn / torch.where(dmin > 0, dmin, 1.0)), zero).clamp(0, 63)
    step = (d * sc)[..., None]
    off = (dmin * m)[..., None]
    q = torch.where(step > 0, torch.round((x + off) / torch.where(step > 0, step, 1.0)), torch.zeros_like(x))
    q = q.clamp(0, 15).to(torch.int32)                                    # [n, nb, 8, 32]
    sc, m = sc.to(torch.int32), m.to(torch.int32)                          # [n, nb, 8]
    s12 = torch.cat([(sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6),
                     (m[..., 0:4] & 63) | ((m[..., 4:8] >> 4) << 6),
                     (sc[..., 4:8] & 0xF) | ((m[..., 4:8] & 0xF) << 4)], -1)
    qv = q.reshape(n, k // QK_K, 4, 2, 32)
    qs = qv[:, :, :, 0, :] | (qv[:, :, :, 1, :] << 4)                        # per 32 bytes: sub-blocks 2c, 2c + 1
    raw = torch.cat([dh.view(torch.uint8).reshape(n, k // QK_K, 2).to(torch.int32),
                     dmh.view(torch.uint8).reshape(n, k // QK_K, 2).to(torch.int32),
                     s12, qs.reshape(n, k // QK_K, 128)], -1).to(torch.uint8)
    return KQuant(raw.contiguous(), GGML_Q4_K, k)


def q6k_values(b):
    """uint8 [..., 210] block_q6_K bytes -> int32 [..., 256] values q - 32 in k order: per half of 128, the four
    32-value parts from the low / high nibbles of ql and the 2-bit fields of qh (gguf_weights.py:85-97)."""
    ql, qh = b[..., 0:128].to(torch.int32), b[..., 128:192].to(torch.int32)
    parts = []
    for h in range(2):
        lo, hi, top = ql[..., 64 * h:64 * h + 32], ql[..., 64 * h + 32:64 * h + 64], qh[..., 32 * h:32 * h + 32]
        parts += [(lo & 0xF) | ((top & 3) << 4), (hi & 0xF) | (((top >> 2) & 3) << 4),
                  (lo >> 4) | (((top >> 4) & 3) << 4), (hi >> 4) | (((top >> 6) & 3) << 4)]
    return torch.cat(parts, -1) - 32


def quantize_q6k(w):
    """fp32 [n, k] -> KQuant (type GGML_Q6_K): this build's Q6_K quantizer.  Per sub-block j of 16: scale_j =
    max|x| / 31; d = fp16(max scale / 127); sc_j = clamp(rint(scale_j / d), -128, 127);
    q = clamp(rint(x / (d sc_j)), -32, 31); stored as q + 32 in ggml's block_q6_K layout."""
    n, k = w.shape
    nb = k // QK_K
    x = w.to(torch.float32).reshape(n, nb, 16, 16)
    scale = x.abs().amax(-1) / 31.0
    dh = (scale.amax(-1) / 127.0).half()
    d = dh.float()[..., None]
    sc = torch.where(d > 0, torch.round(scale / torch.where(d > 0, d, 1.0)), torch.zeros_like(scale)).clamp(-128, 127)
    step = (d * sc)[..., None]
    q = torch.where(step != 0, torch.round(x / torch.where(step != 0, step, 1.0)), torch.zeros_like(x))
    Q = (q.clamp(-32, 31) + 32).to(torch.int32).reshape(n, nb, 2, 4, 32)       # [n, nb, half, part, l]
    ql = torch.cat([(Q[:, :, :, 0] & 15) | ((Q[:, :, :, 2] & 15) << 4),
                    (Q[:, :, :, 1] & 15) | ((Q[:, :, :, 3] & 15) << 4)], -1)     # [n, nb, half, 64]
    qh = (Q[:, :, :, 0] >> 4) | ((Q[:, :, :, 1] >> 4) << 2) | ((Q[:, :, :, 2] >> 4) << 4) | ((Q[:, :, :, 3] >> 4) << 6)
    raw = torch.cat([ql.reshape(n, nb, 128), qh.reshape(n, nb, 64), sc.to(torch.int32) & 0xFF,
                     dh.view(torch.uint8).reshape(n, nb, 2).to(torch.int32)], -1).to(torch.uint8)
    return KQuant(raw.contiguous(), GGML_Q6_K, k)
