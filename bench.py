"""Benchmark of the quantized linear-layer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu]

Workload (benchmark config 1): Q8_0 W8A8 prefill GEMM, fused gate|up, M = 8192 tokens, K = 5120, N = 27648.  One step
is the hot path over one batch: per-token int8 quantization of the bf16 activations (its own kernel), then the
W8A8 GEMM on the Q8_0 weights (int8 values + fp16 block scales, gk = 32) into bf16.  Inputs are synthetic with the
config's distributions (weights N(0, 0.02^2) quantized to Q8_0 on the GPU, activations N(0, 1) in bf16) and are
resident in HBM before the timed region.  `value` is TOPS of the whole step (2 M N K / step time); `roofline`
describes the GEMM kernel alone, timed with HIP events on the stream it is launched on, against the MI355X dense
int8 MFMA peak (5.0 POPS).

Also measured (key "configs", not the headline; GEMM kernels alone, graph-replayed): config 0 (Q8_0, M = 16,
K = N = 4096) and config 2 (Q8_0 decode, M in 1, 4, 16, 64; (K, N) = (5120, 5120), (17408, 5120)) as GB/s of packed
Q8_0 weight bytes; config 3 (Q4_K W4A8, M = 16 and 2048; and the same shape on Q6_K weights) and config 4 (MXFP4,
M = 16 and 4096), each against its roof (HBM for the decode sizes, the int8 or fp8 MFMA peak for the prefill
sizes); the engine's per-channel (gk = K) projections at config 1's shape and config 2's decode sizes; the fused
producers; and "c1_reassoc", the opt-in reassociated Q8_0 prefill kernel on config 1's operands (timed with HIP
events, not the headline: its rounding order is not the reference's; it reports the share of its bf16 outputs equal
to the exact kernel's).  Memory-bound shapes rotate weight
copies through more than 3 x the 256 MB MALL so that every launch streams its weights from HBM.

cpu_baseline: the CPU oracle (oracle/, the exact restatement of the reference's arithmetic, OpenMP) on a bounded
row sample of the same workload, on this host's cores; beside it, "reference_cpu_path": the reference's own CPU
emulation of this GEMM (tests/int8_sim.py:75-81, fp32 fake quantization and matmul in torch, 16 threads).

peaks_measured: the library's probes on this GPU (dense int8 / fp8 / fp4 / bf16 MFMA chains, and HBM reads of 1 GiB
and of the decode weight sizes, graph-replayed as the decode lines are); roofline.peak stays MI355X's published
figure, roofline.peak_measured is the probe's.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "startlux-prism_amd"))

PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
PEAK_FP8_TFLOPS = 5000.0     # MI355X dense fp8 (and fp8 x fp4) MFMA
MALL_BYTES = 256 << 20

M1, K1, N1 = 8192, 5120, 27648


def q8_bytes(N, K):
    return N * K // 32 * 34


def make_q8_weights(N, K, seed, dev):
    """Q8_0 weights of N(0, 0.02^2) values, in the GEMM's operand form (kernels/w8a8.py weight_from_q8, gk = 32):
    the MFMA-native packed layout."""
    import torch
    from prism_amd import gguf_formats as GF
    from prism_amd import w8a8 as KW
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = torch.randn(N, K, generator=g, device=dev, dtype=torch.float32) * 0.02
    q8 = GF.quantize_q8_0(w)
    del w
    packed, _ = KW.weight_from_q8(q8, 32)
    return q8, packed


def make_acts(M, K, seed, dev):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn(M, K, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)


def bench_prefill(steps, warmup, dev):
    import torch
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    q8, pw = make_q8_weights(N1, K1, 1, dev)
    x = make_acts(M1, K1, 2, dev)
    q = torch.empty(M1, K1, dtype=torch.int8, device=dev)
    s = torch.empty(M1, dtype=torch.float32, device=dev)
    out = torch.empty(M1, N1, dtype=torch.bfloat16, device=dev)
    n = torch.tensor([M1], dtype=torch.int32, device=dev)

    def step():
        KQ.rows_q8(x, None, q, s, n, M1)
        KW.gemm(q, s, pw, None, out, n, 32, epi=0)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for e0, e1, e2 in ev:
        e0.record()
        KQ.rows_q8(x, None, q, s, n, M1)
        e1.record()
        KW.gemm(q, s, pw, None, out, n, 32, epi=0)
        e2.record()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(stop)
    gemm_ms = sum(e1.elapsed_time(e2) for _, e1, e2 in ev) / steps
    quant_ms = sum(e0.elapsed_time(e1) for e0, e1, _ in ev) / steps
    ops = 2.0 * M1 * N1 * K1
    res = dict(ms_per_step=total_ms / steps, wall_s=wall, gemm_ms=gemm_ms, quant_ms=quant_ms, ops=ops,
               value=ops / (total_ms / steps * 1e-3) / 1e12)
    # the opt-in reassociated kernel on the same operands (not the headline: its rounding order is not the
    # reference's); with the share of its bf16 outputs equal to the exact kernel's
    ora = torch.empty_like(out)
    KW.gemm(q, s, pw, None, ora, n, 32, epi=0, kernel="reassoc")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        KW.gemm(q, s, pw, None, ora, n, 32, epi=0, kernel="reassoc")
    e1.record()
    torch.cuda.synchronize()
    ra_ms = e0.elapsed_time(e1) / steps
    same = (ora.view(torch.int16) == out.view(torch.int16)).double().mean().item()
    res["reassoc"] = dict(kernel="reassoc", gemm_ms=round(ra_ms, 4), tops=round(ops / (ra_ms * 1e-3) / 1e12, 2),
                          frac=round(ops / (ra_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
                          bf16_equal_to_exact=round(same, 6))
    del ora
    sample = dict(q=q, s=s, qs=q8.qs, d=q8.d, x=x[:M1])
    return res, sample


def _graph_us(launch, copies, iters):
    """Mean microseconds per launch of launch(i) (i picks the weight copy), captured back to back in a HIP graph and
    replayed: the form the engine's captured decode steps run in."""
    import torch
    for i in range(min(copies, 3)):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            for i in range(iters):
                launch(i % copies)
    g.replay()                       # warm-up replay: clocks settle before the timed one
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    g.replay()
    b.record()
    torch.cuda.synchronize()
    del g
    return a.elapsed_time(b) / iters * 1e3


def _copies(wbytes, M):
    """Weight copies rotated per launch: more than 3 x the MALL for the memory-bound shapes, so that every launch
    streams its weights from HBM."""
    return max(3, -(-3 * MALL_BYTES // wbytes)) if M <= 64 else 1


def _row(M, K, N, us, wbytes, bound, peak=None):
    gbs = wbytes / (us * 1e-6) / 1e9
    tops = 2 * M * N * K / (us * 1e-6) / 1e12
    r = dict(M=M, K=K, N=N, us=round(us, 2), GBps=round(gbs, 1), TOPS=round(tops, 2), bound=bound, bytes=wbytes)
    r["frac"] = round(gbs / PEAK_HBM_GBS, 3) if bound == "hbm" else round(tops / peak, 4)
    return r


def bench_q8_decode(dev, shapes, Ms, iters=40):
    """Q8_0 W8A8 GEMMs at decode sizes (configs 0 and 2): GB/s of packed Q8_0 weight bytes."""
    import torch
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    rows = []
    for (K, N) in shapes:
        wbytes = q8_bytes(N, K)
        copies = _copies(wbytes, 1)
        _, base = make_q8_weights(N, K, 3, dev)
        ws = [KW.PackedQ8(base.qt.clone(), base.dt.clone(), N, K) for _ in range(copies)]
        for M in Ms:
            x = make_acts(M, K, 4, dev)
            q = torch.empty(M, K, dtype=torch.int8, device=dev)
            s = torch.empty(M, dtype=torch.float32, device=dev)
            n = torch.tensor([M], dtype=torch.int32, device=dev)
            KQ.rows_q8(x, None, q, s, n, M)
            out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
            us = _graph_us(lambda i: KW.gemm(q, s, ws[i], None, out, n, 32), copies, iters)
            rows.append(_row(M, K, N, us, wbytes, "hbm"))
        del ws, base
        torch.cuda.empty_cache()
    return rows


def bench_w4a8(dev, iters=20, kind="q4k"):
    """Config 3: Q4_K W4A8, K = 5120, N = 13824, M = 16 (memory-bound: GB/s of the device weight bytes, for Q4_K the
    file's 144 per 256 weights) and M = 2048 (int8 MFMA-bound), one activation scale per token plus per-32 sums
    (rows_g, not timed here).  kind "q6k": the same shape on Q6_K weights (device layout int8 values plus scales,
    4384 bytes per 16 rows x 256 inputs)."""
    import torch
    from prism_amd import gguf_formats as GF
    from prism_amd import quant as KQ
    from prism_amd import w4a8 as KW4
    K, N = 5120, 13824
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    w0 = torch.randn(N, K, generator=g, device=dev) * 0.02
    kq = GF.quantize_q6k(w0) if kind == "q6k" else GF.quantize_q4k(w0)
    del w0
    w1 = KW4.repack(kq)
    wbytes = w1.qv.numel() + w1.meta.numel()
    del w1
    rows = []
    for M in (16, 2048):
        copies = _copies(wbytes, M)
        ws = [KW4.repack(kq) for _ in range(copies)]
        x = make_acts(M, K, 6, dev)
        q = torch.empty(M, K, dtype=torch.int8, device=dev)
        s = torch.empty(1, M, dtype=torch.float32, device=dev)
        xs = torch.empty(K // 256, M, 16, dtype=torch.int8, device=dev)
        n = torch.tensor([M], dtype=torch.int32, device=dev)
        KQ.rows_g(x, q, s, xs, n, M, group=K)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        us = _graph_us(lambda i: KW4.gemm(q, s, xs, ws[i], out, n), copies, iters if M <= 64 else 20)
        rows.append(_row(M, K, N, us, wbytes, "hbm" if M <= 64 else "mfma", PEAK_INT8_TOPS))
        del ws
        torch.cuda.empty_cache()
    return rows


def bench_mxfp4(dev, iters=40):
    """Config 4: MXFP4, K = N = 5120, e2m1 weights (OCP scales) x e4m3 activations (per-32 e8m0), M = 16 (GB/s of
    weight bytes, 0.5 + 1/32 per weight) and M = 4096 (against the fp8 dense MFMA peak, 5.0 PFLOP/s)."""
    import torch
    from prism_amd import mxfp4 as MX
    K = N = 5120
    wbytes = N * K // 2 + N * K // 32
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    base = MX.pack(torch.randn(N, K, generator=g, device=dev) * 0.02, "ocp")
    rows = []
    for M in (16, 4096):
        copies = _copies(wbytes, M)
        ws = [MX.MX4(base.q.clone(), base.s.clone(), N, K) for _ in range(copies)]
        x = make_acts(M, K, 8, dev)
        q = torch.empty(M, K, dtype=torch.uint8, device=dev)
        s = torch.empty(M, K // 32, dtype=torch.uint8, device=dev)
        MX.quantize_act_fp8(x, q, s)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        us = _graph_us(lambda i: MX.gemm(q, s, ws[i], out, M), copies, iters if M <= 64 else 40)
        if M > 64:      # prefill: the activations in the panel layout the tile kernel reads (same bits)
            qp = MX.act_panels(M, K, dev)
            MX.quantize_act_fp8(x, qp, s)
            us_rows = us
            us = _graph_us(lambda i: MX.gemm(qp, s, ws[i], out, M), copies, 40)
        rows.append(_row(M, K, N, us, wbytes, "hbm" if M <= 64 else "mfma", PEAK_FP8_TFLOPS))
        if M > 64:
            rows[-1].update(act_layout="panels", us_row_major_acts=round(us_rows, 2))
        del ws
        torch.cuda.empty_cache()
    return rows


def bench_per_channel(dev, iters=40, decode_only=False):
    """The engine's per-channel (gk = K) W8A8 projections (its production path): packed int8 weights
    (weight_from_q8(q8, K)), one activation scale per token; prefill at config 1's shape (against the int8 MFMA peak)
    and the decode sizes of config 2 (GB/s of the int8 weight bytes)."""
    import torch
    from prism_amd import gguf_formats as GF
    from prism_amd import w8a8 as KW
    rows = []
    shapes = ((M1, K1, N1), (1, 5120, 5120), (16, 5120, 5120), (64, 5120, 5120), (1, 17408, 5120),
              (16, 17408, 5120), (64, 17408, 5120))
    for (M, K, N) in shapes[1:] if decode_only else shapes:
        g = torch.Generator(device=dev)
        g.manual_seed(9)
        q8 = GF.quantize_q8_0(torch.randn(N, K, generator=g, device=dev) * 0.02)
        base, _ = KW.weight_from_q8(q8, K)
        del q8
        wbytes = N * K
        copies = _copies(wbytes, M)
        ws = [base] + [KW.PackedPC(base.qt.clone(), base.ws, N, K) for _ in range(copies - 1)]
        x = make_acts(M, K, 10, dev)
        from prism_amd import quant as KQ
        q = torch.empty(M, K, dtype=torch.int8, device=dev)
        s = torch.empty(M, dtype=torch.float32, device=dev)
        n = torch.tensor([M], dtype=torch.int32, device=dev)
        KQ.rows_q8(x, None, q, s, n, M)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        us = _graph_us(lambda i: KW.gemm(q, s, ws[i], None, out, n, K), copies, iters if M <= 64 else 10)
        rows.append(_row(M, K, N, us, wbytes, "hbm" if M <= 64 else "mfma", PEAK_INT8_TOPS))
        del ws, base, out, x, q
        torch.cuda.empty_cache()
    return rows


def bench_per_channel_plain(dev, iters=40):
    """The per-channel GEMM on plain int8 planes (w int8 [N, K], fp32 w_s [N]): the operand an engine holds when it
    requantizes its weights itself instead of calling weight_from_q8 (which packs them).  Same kernels through the
    row-major entry point prism_w8a8_gemm, at the shapes of bench_per_channel."""
    import torch
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    rows = []
    for (M, K, N) in ((M1, K1, N1), (1, 5120, 5120), (16, 5120, 5120), (64, 5120, 5120), (1, 17408, 5120),
                      (16, 17408, 5120), (64, 17408, 5120)):
        g = torch.Generator(device=dev)
        g.manual_seed(9)
        wbytes = N * K
        copies = _copies(wbytes, M)
        ws = [torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev) for _ in range(copies)]
        sw = torch.rand(N, generator=g, device=dev)
        x = make_acts(M, K, 10, dev)
        q = torch.empty(M, K, dtype=torch.int8, device=dev)
        s = torch.empty(M, dtype=torch.float32, device=dev)
        n = torch.tensor([M], dtype=torch.int32, device=dev)
        KQ.rows_q8(x, None, q, s, n, M)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        us = _graph_us(lambda i: KW.gemm(q, s, ws[i], sw, out, n, K), copies, iters if M <= 64 else 10)
        rows.append(_row(M, K, N, us, wbytes, "hbm" if M <= 64 else "mfma", PEAK_INT8_TOPS))
        del ws, out, x, q
        torch.cuda.empty_cache()
    return rows


def bench_deferred(dev, iters=40):
    """The engine's down projection at 64 decode rows (K 17408 -> HID 5120, per channel, residual add) followed by the
    norm_q8 that reads the residual: unsplit (epilogue 1, then norm_q8) against deferred (K in defer_split parts
    into int32 slots, then norm_q8 finishing the add); both leave the same bits in the residual and the int8 rows."""
    import torch
    from prism_amd import quant as KQ
    from prism_amd import w8a8 as KW
    M, K, N = 64, 17408, 5120
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev)
    copies = _copies(N * K, 1)
    ws = [KW.pack_i8(w, torch.rand(N, generator=g, device=dev)) for _ in range(copies)]
    del w
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8, device=dev)
    sa = torch.rand(M, generator=g, device=dev)
    n = torch.tensor([M], dtype=torch.int32, device=dev)
    h = torch.randn(M, N, generator=g, device=dev)
    nw = torch.rand(N, generator=g, device=dev) + 0.5
    q = torch.empty(M, N, dtype=torch.int8, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    slots = torch.empty(4, M, N, dtype=torch.int32, device=dev)

    def unsplit(i):
        KW.gemm(a, sa, ws[i], None, h, n, K, epi=1)
        KQ.norm_q8(h, nw, q, s, n, M, 1e-6)

    def deferred(i):
        KQ.norm_q8(h, nw, q, s, n, M, 1e-6, pending=KW.gemm(a, sa, ws[i], None, h, n, K, epi=1, slots=slots))

    u = _graph_us(unsplit, copies, iters)
    d = _graph_us(deferred, copies, iters)
    del ws
    torch.cuda.empty_cache()
    return [dict(M=M, K=K, N=N, split=KW.defer_split(M, N, K, 4), us_unsplit=round(u, 2), us_deferred=round(d, 2))]


def bench_producers(dev, iters=20):
    """The fused producers at config 1's shapes (HBM-bound: GB/s of bytes read plus written): norm_q8 on the fp32
    residual (T = 8192, HID = 5120) and swiglu_q8 on the bf16 gate|up output (T = 8192, FF = 13824), plus the
    per-token quantizer rows_q8 of the headline step, and gated_norm_q8 on the linear-attention output (48 value heads
    of 128, gate bf16 from the projection); and their decode size (T = 16)."""
    import torch
    from prism_amd import quant as KQ
    rows = []
    for T in (M1, 16):
        n = torch.tensor([T], dtype=torch.int32, device=dev)
        h = torch.randn(T, K1, device=dev)
        w = torch.rand(K1, device=dev) + 0.5
        q = torch.empty(T, K1, dtype=torch.int8, device=dev)
        s = torch.empty(T, dtype=torch.float32, device=dev)
        us = _graph_us(lambda i: KQ.norm_q8(h, w, q, s, n, T, 1e-6), 1, iters)
        b = T * K1 * 4 + K1 * 4 + T * K1 + 4 * T
        rows.append(dict(op="norm_q8", T=T, K=K1, us=round(us, 2), GBps=round(b / us / 1e3, 1),
                         frac=round(b / us / 1e3 / PEAK_HBM_GBS, 3)))
        FF = N1 // 2
        gu = torch.randn(T, 2 * FF, device=dev).to(torch.bfloat16)
        inv = torch.rand(FF, device=dev) + 0.5
        q2 = torch.empty(T, FF, dtype=torch.int8, device=dev)
        us = _graph_us(lambda i: KQ.swiglu_q8(gu, inv, q2, s, n, T), 1, iters)
        b = T * 2 * FF * 2 + FF * 4 + T * FF + 4 * T
        rows.append(dict(op="swiglu_q8", T=T, K=FF, us=round(us, 2), GBps=round(b / us / 1e3, 1),
                         frac=round(b / us / 1e3 / PEAK_HBM_GBS, 3)))
        x = torch.randn(T, K1, device=dev).to(torch.bfloat16)
        us = _graph_us(lambda i: KQ.rows_q8(x, None, q, s, n, T), 1, iters)
        b = T * K1 * 2 + T * K1 + 4 * T
        rows.append(dict(op="rows_q8", T=T, K=K1, us=round(us, 2), GBps=round(b / us / 1e3, 1),
                         frac=round(b / us / 1e3 / PEAK_HBM_GBS, 3)))
        HV, D = 48, 128
        o = torch.randn(T, HV * D, device=dev)
        proj = torch.randn(T, 2 * HV * D, device=dev).to(torch.bfloat16)
        wd = torch.rand(D, device=dev) + 0.5
        inv3 = torch.rand(HV * D, device=dev) + 0.5
        q3 = torch.empty(T, HV * D, dtype=torch.int8, device=dev)
        cfg = type("Cfg", (), {"v_heads": HV, "gdn_dim": D, "eps": 1e-6})()
        us = _graph_us(lambda i: KQ.gated_norm_q8(o, proj, HV * D, wd, inv3, q3, s, n, T, cfg), 1, iters)
        b = T * HV * D * (4 + 2 + 1) + HV * D * 4 + 4 * T
        rows.append(dict(op="gated_norm_q8", T=T, K=HV * D, us=round(us, 2), GBps=round(b / us / 1e3, 1),
                         frac=round(b / us / 1e3 / PEAK_HBM_GBS, 3)))
        del h, gu, x, q, q2, o, proj, q3
        torch.cuda.empty_cache()
    return rows


CONFIG_LINES = {
    "producers": bench_producers,
    "per_channel": bench_per_channel,
    "per_channel_plain": bench_per_channel_plain,
    "per_channel_deferred": bench_deferred,
    "c0": lambda dev: bench_q8_decode(dev, [(4096, 4096)], (16,)),
    "c2": lambda dev: bench_q8_decode(dev, [(5120, 5120), (17408, 5120)], (1, 4, 16, 64)),
    "c3": bench_w4a8,
    "c3_q6k": lambda dev: bench_w4a8(dev, kind="q6k"),
    "c4": bench_mxfp4,
}
# Lines that --only accepts besides the keys above: the per-channel decode sizes without the prefill.
EXTRA_LINES = {"per_channel_decode": lambda dev: bench_per_channel(dev, decode_only=True)}


def bench_configs(dev, only=None):
    table = dict(CONFIG_LINES, **EXTRA_LINES) if only else CONFIG_LINES
    names = only or list(CONFIG_LINES)
    return {k: table[k](dev) for k in names}


def cpu_baseline(sample, rows):
    """The oracle's exact W8A8 GEMM on the first `rows` rows of the same quantized activations and weights."""
    import numpy as np
    import oracle as O
    a = sample["q"][:rows].cpu().numpy()
    s = sample["s"][:rows].cpu().numpy()
    w = sample["qs"].cpu().numpy()
    d = sample["d"].view(__import__("torch").int16).cpu().numpy().view(np.uint16)
    threads = min(os.cpu_count() or 1, 16)
    O.lib()
    t0 = time.perf_counter()
    O.w8a8_gemm(a, s, w, d, 32, epi=0, nthreads=threads)
    dt = time.perf_counter() - t0
    ops = 2.0 * rows * N1 * K1
    return dict(value=round(ops / dt / 1e12, 4), unit="TOPS", cores=threads, kind="port",
                sample=f"{rows} of {M1} rows of config 1 (K={K1}, N={N1}), exact int32-per-block oracle, "
                       f"{dt:.1f} s")


def cpu_reference_path(sample, rows_max=M1, budget_s=5.0):
    """The reference's own CPU path for this GEMM (tests/int8_sim.py:75-81, torch.set_num_threads(16) at :41): fp32
    fake quantization of the activations per token (scale amax / 127, round, rescale) and an fp32 matmul against the
    dequantized weights (Q8_0 values times their fp16 block scales), timed on a row sample of config 1's operands.
    The weights' dequantization is set-up, not timed (the reference caches it, :63-72)."""
    import torch
    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    qs, d = sample["qs"].cpu(), sample["d"].cpu()
    w = (qs.view(N1, K1 // 32, 32).float() * d.float().view(N1, K1 // 32, 1)).view(N1, K1)
    x = sample["x"].cpu().float()
    rows = 64
    while True:
        xs = x[:rows]
        t0 = time.perf_counter()
        sc = xs.abs().amax(1, keepdim=True).clamp_min(1e-10) / 127
        xq = torch.round(xs / sc) * sc
        _ = xq @ w.T
        dt = time.perf_counter() - t0
        if dt > budget_s / 4 or rows >= rows_max:
            break
        rows = min(rows_max, rows * 4)
    ops = 2.0 * rows * N1 * K1
    return dict(value=round(ops / dt / 1e12, 4), unit="TOPS", threads=threads, os_cpu_count=os.cpu_count(),
                torch_threads=torch.get_num_threads(),
                sample=f"{rows} of {M1} rows of config 1, fp32 fake-quant matmul (tests/int8_sim.py:75-81), "
                       f"{dt:.2f} s")


def read_probe(dev, sizes):
    """The attainable HBM read time of each byte size in `sizes`: the library's read probe (prism_probe_read, 16-byte
    loads over the whole buffer) graph-replayed back to back with copies rotated past the MALL, exactly as the decode
    lines are timed.  Returns {nbytes: (us, GB/s)}."""
    import ctypes
    import torch
    from prism_amd import _lib as L
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)   # noqa: E731
    sink = torch.zeros(1 << 16, dtype=torch.float32, device=dev)
    out = {}
    sizes = sorted(set(int(n) for n in sizes))
    if not sizes:
        return out
    buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    for nbytes in sizes:
        copies = _copies(nbytes, 1)
        views = [buf[i * nbytes:(i + 1) * nbytes] for i in range(min(copies, (1 << 30) // nbytes))]
        us = _graph_us(lambda i: L.call("prism_probe_read", L.ptr(views[i]), nbytes, 256, L.ptr(sink), st()),
                       len(views), 40)
        out[nbytes] = (us, nbytes / us / 1e3)
    del buf
    torch.cuda.empty_cache()
    return out


def annotate_hbm_rows(configs, probes):
    """Every HBM-bound line also against the read probe of its own byte size (the rate a pure read of those bytes
    attains here), besides `frac` against the published 8 TB/s."""
    for rows in configs.values():
        for row in rows if isinstance(rows, list) else []:
            if row.get("bound") == "hbm" and row.get("bytes") in probes:
                us, gbs = probes[row["bytes"]]
                row["read_probe_us"] = round(us, 2)
                row["read_probe_GBps"] = round(gbs, 1)
                row["frac_of_measured"] = round(row["GBps"] / gbs, 3)


def hbm_sizes(configs):
    return [r["bytes"] for rows in configs.values() if isinstance(rows, list) for r in rows
            if r.get("bound") == "hbm" and "bytes" in r]


def measure_peaks(dev):
    """The roofline denominators measured on this GPU with the library's probes: dense MFMA rates (int8, fp8, fp4,
    bf16; independent MFMA chains in registers) and the HBM read rate (a 1 GiB stream, and the decode GEMMs' sizes
    streamed back to back from a HIP graph with copies rotated past the MALL, as the decode lines are timed)."""
    import ctypes
    import torch
    from prism_amd import _lib as L
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)   # noqa: E731
    sink = torch.zeros(1 << 16, dtype=torch.float32, device=dev)
    out = {}
    wgs, iters = 256 * 8, 256
    for kind, name in ((0, "int8_tops"), (1, "fp8_tflops"), (2, "fp4_tflops"), (3, "bf16_tflops"),
                       (4, "int8_random_operands_tops"), (5, "fp4xfp8_random_operands_tflops")):
        best = 1e30
        for _ in range(4):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            L.call("prism_probe_mfma", kind, wgs, iters, L.ptr(sink), st())
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1))
        ops = wgs * 4 * iters * 4 * L.lib().prism_probe_mfma_ops(kind)
        out[name] = round(ops / (best * 1e-3) / 1e12, 1)
    buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    best = 1e30
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        L.call("prism_probe_read", L.ptr(buf), buf.numel(), 2048, L.ptr(sink), st())
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1))
    out["hbm_gbs_1gib"] = round(buf.numel() / (best * 1e-3) / 1e9, 1)
    for nbytes in (q8_bytes(5120, 5120), q8_bytes(5120, 17408)):
        copies = _copies(nbytes, 1)
        views = [buf[i * nbytes:(i + 1) * nbytes] for i in range(min(copies, (1 << 30) // nbytes))]
        us = _graph_us(lambda i: L.call("prism_probe_read", L.ptr(views[i]), nbytes, 256, L.ptr(sink), st()),
                       len(views), 40)
        out[f"read_{nbytes}_bytes_us"] = round(us, 2)
        out[f"read_{nbytes}_bytes_gbs"] = round(nbytes / us / 1e3, 1)
    del buf
    torch.cuda.empty_cache()
    return out


def traffic_from_profiles():
    """HBM bytes per launch of the GEMM from the committed rocprofv3 --pmc summary, if present."""
    p = os.path.join(ROOT, "profiles", "w8a8_tile_prefill_traffic.json")
    if os.path.exists(p):
        try:
            return json.load(open(p)).get("traffic_bytes")
        except (OSError, ValueError):
            return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-sweep", action="store_true", help="skip the per-config measurements")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=M1)
    ap.add_argument("--only", default=None,
                    help="comma-separated config lines (c0, c2, c3, c3_q6k, c4, per_channel, per_channel_decode, "
                         "per_channel_plain, per_channel_deferred, producers): run just those and print them as one JSON line, "
                         "without the headline (for profiling one kernel family)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device copy (3 times): the calibration kernel for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE, whose true traffic is known")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the hot path shards by output "
              "columns with no exchange; see the sharding notes).  Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if a.only:
        unknown = [k for k in a.only.split(",") if k not in CONFIG_LINES and k not in EXTRA_LINES]
        if unknown:
            raise SystemExit(f"bench.py: unknown --only line(s) {unknown}; known: "
                             f"{sorted(list(CONFIG_LINES) + list(EXTRA_LINES))}")
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.copy_probe:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4}))
        return
    if a.only:
        configs = bench_configs(dev, a.only.split(","))
        annotate_hbm_rows(configs, read_probe(dev, hbm_sizes(configs)))
        print(json.dumps({"configs": configs}), flush=True)
        return
    res, sample = bench_prefill(a.steps, a.warmup, dev)
    configs = None if a.no_sweep else bench_configs(dev)
    peaks = measure_peaks(dev)
    if configs:
        probes = read_probe(dev, hbm_sizes(configs))
        annotate_hbm_rows(configs, probes)
        peaks["read_probe_us_by_bytes"] = {str(k): round(v[0], 2) for k, v in probes.items()}
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(sample, a.cpu_rows)
        cpu["reference_cpu_path"] = cpu_reference_path(sample)
        cpu["os_cpu_count"] = os.cpu_count()
    achieved = res["ops"] / (res["gemm_ms"] * 1e-3) / 1e12
    # int8 MFMA-bound lines also against the int8 rate measured with GEMM-like (changing, pseudo-random) operands:
    # the power limit holds the clock lower for those than for the constant-operand probe
    for key in ("per_channel", "per_channel_plain", "c3", "c3_q6k"):
        for row in (configs or {}).get(key, []):
            if row.get("bound") == "mfma" and "TOPS" in row:
                row["frac_of_measured_random_operands"] = round(row["TOPS"] / peaks["int8_random_operands_tops"], 4)
    for row in (configs or {}).get("c4", []):                     # MXFP4: fp4 operands on the f8f6f4 MFMA
        if row.get("bound") == "mfma" and "TOPS" in row:
            row["frac_of_measured_random_operands"] = round(row["TOPS"] / peaks["fp4xfp8_random_operands_tflops"], 4)
    line = {
        "metric": "W8A8/W4A8 GEMM TOPS and GB/s vs MI355X roofline, prefill M=8192 and decode M=1..64",
        "value": round(res["value"], 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "Q8_0 W8A8 prefill gate|up (config 1): rows_q8 + GEMM, gk=32, bf16 out",
                   "M": M1, "K": K1, "N": N1, "gemm_ms": round(res["gemm_ms"], 4),
                   "quant_ms": round(res["quant_ms"], 4)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": traffic_from_profiles(),
                     "peak_measured": peaks["int8_tops"],
                     "frac_of_measured": round(achieved / peaks["int8_tops"], 4),
                     "peak_measured_random_operands": peaks["int8_random_operands_tops"],
                     "frac_of_measured_random_operands": round(achieved / peaks["int8_random_operands_tops"], 4)},
        "peaks_measured": peaks,
        "cpu_baseline": cpu,
        "configs": dict(configs or {}, c1_reassoc=res["reassoc"]),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
