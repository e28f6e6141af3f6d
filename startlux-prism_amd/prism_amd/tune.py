"""Measures the dispatch tables (prism_amd.dispatch) on the GPU it runs on: the counterpart of the reference's
bench/cuda_gemm_micro.py --table and bench/w4a8_table.py.

    cd startlux-prism_amd && python -m prism_amd.tune [--tables gemm,q8,w4a8] [--out DIR] [--quick]

For each projection shape of the 27B model (the shapes of the reference's tables, kernels/gemm_table_h200.json and
w4a8_table_h200.json, with N a multiple of 16) and each of the reference's token buckets, every kernel valid at that
token count is timed with its weights streamed from HBM (copies rotated through more than 3 x the 256 MB MALL, the
launches replayed from a HIP graph) and the fastest is recorded.  Token counts where one kernel is valid (W4A8's
tile kernel beyond 16 rows) are recorded without timing.  Every kernel computes the same bits, so
the table changes speed only.
"""
import argparse
import json
import os
import sys
import time

import torch

from . import _lib as L
from . import dispatch
from . import gguf_formats as GF
from . import w4a8 as KW4
from . import w8a8 as KW

MS = [1, 2, 4, 8, 16, 32, 64, 128, 192, 256, 320, 384, 512, 640, 768, 1024, 1280, 1536, 2048, 2560, 3072, 4096,
      5120, 6144, 8192]
W8_SHAPES = [(512, 5120), (1024, 5120), (2048, 5120), (3072, 5120), (3584, 5120), (6144, 5120), (7168, 5120),
             (8240, 5120), (8704, 5120), (12288, 5120), (14336, 5120), (16480, 5120), (17408, 5120), (34816, 5120),
             (5120, 6144), (5120, 17408)]
W4_SHAPES = [("q4k", 1024, 5120), ("q4k", 6240, 5120), ("q4k", 12288, 5120), ("q4k", 13312, 5120),
             ("q4k", 14336, 5120), ("q4k", 16480, 5120), ("q4k", 34816, 5120), ("q4k", 5120, 6144),
             ("q4k", 5120, 17408), ("q6k", 1024, 5120), ("q6k", 10240, 5120), ("q6k", 5120, 17408)]
MALL = 256 << 20


def _copies(nbytes):
    return max(2, -(-3 * MALL // nbytes))


def _time(launch, copies, iters=20, reps=3):
    """Median microseconds per launch of launch(i) over `reps` replays of a graph of `iters` launches."""
    for i in range(min(copies, 2)):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            for i in range(iters):
                launch(i % copies)
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) * 1e3 / iters)
    del g
    return sorted(ts)[len(ts) // 2]


def _pick(cands, launch_for, copies, M):
    if len(cands) == 1:
        return cands[0], {}
    us = {}
    for c in cands:
        try:
            us[c] = _time(launch_for(c), copies if M <= 256 else 1, iters=20 if M <= 256 else 5)
        except L.PrismError:         # not valid at this shape (e.g. an activation image beyond LDS)
            continue
    return min(us, key=us.get), us


def tune_w8(kind, shapes, Ms, dev, log):
    """kind "q8": Q8_0 packed (gk = 32); "gemm": per channel (gk = K)."""
    table = {}
    for (N, K) in shapes:
        g = torch.Generator(device=dev)
        g.manual_seed(N + K)
        qs = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev)
        if kind == "q8":
            d = (torch.rand(N, K // 32, generator=g, device=dev) * 1e-3).half()
            base = KW.pack_q8(qs, d)
            nbytes = N * K // 32 * 34
            ws = [base] + [KW.PackedQ8(base.qt.clone(), base.dt.clone(), N, K) for _ in range(_copies(nbytes) - 1)]
            gk = 32
        else:
            base = KW.pack_i8(qs, torch.rand(N, 1, generator=g, device=dev))
            nbytes = N * K
            ws = [base] + [KW.PackedPC(base.qt.clone(), base.ws.clone(), N, K) for _ in range(_copies(nbytes) - 1)]
            gk = K
        del qs
        row = {}
        for M in Ms:
            a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8, device=dev)
            s = torch.rand(M, generator=g, device=dev)
            out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
            n = torch.tensor([M], dtype=torch.int32, device=dev)
            if kind == "q8":
                # "decode" hands 17..64 rows to the "mid" kernel, so it is a candidate up to 16 rows only
                cands = ["decode", "stream", "mid", "tile"] if M <= 16 else ["mid", "tile"]
            else:
                cands = ["decode", "split", "tile"] if M <= 512 else ["decode", "tile"]
            best, us = _pick(cands, lambda c: (lambda i: KW.gemm(a, s, ws[i], None, out, n, gk, kernel=c)),
                             len(ws), M)
            row[str(M)] = [best]
            if us:
                log(f"{kind} {N}x{K} M={M}: " + " ".join(f"{c} {t:.1f}" for c, t in us.items()) + f" -> {best}")
            del a, out
        table[f"{N}x{K}"] = row
        del ws, base
        torch.cuda.empty_cache()
    return table


def tune_w4(shapes, Ms, dev, log):
    table = {}
    for (kind, N, K) in shapes:
        g = torch.Generator(device=dev)
        g.manual_seed(N + K)
        w0 = torch.randn(N, K, generator=g, device=dev) * 0.02
        kq = GF.quantize_q6k(w0) if kind == "q6k" else GF.quantize_q4k(w0)
        del w0
        base = KW4.repack(kq)
        nbytes = base.qv.numel() + base.meta.numel()
        ws = [base] + [KW4.W4(kind, base.qv.clone(), base.meta.clone(), N, K) for _ in range(_copies(nbytes) - 1)]
        row = {}
        for M in Ms:
            xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8, device=dev)
            a = torch.rand(1, M, generator=g, device=dev)
            xs = torch.randint(-64, 64, (K // 256, M, 16), generator=g, dtype=torch.int8, device=dev)
            out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
            n = torch.tensor([M], dtype=torch.int32, device=dev)
            cands = ["decode", "stream", "tile"] if M <= 16 else ["tile"]
            best, us = _pick(cands, lambda c: (lambda i: KW4.gemm(xq, a, xs, ws[i], out, n, kernel=c)), len(ws), M)
            row[str(M)] = [best]
            if us:
                log(f"{kind} {N}x{K} M={M}: " + " ".join(f"{c} {t:.1f}" for c, t in us.items()) + f" -> {best}")
            del xq, xs, out
        table[f"{kind},{N},{K}"] = row
        del ws, base
        torch.cuda.empty_cache()
    return table


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--tables", default="gemm,q8,w4a8")
    ap.add_argument("--out", default=dispatch.HERE)
    ap.add_argument("--quick", action="store_true", help="two shapes per table, token counts up to 64")
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    tag = dispatch.gpu_tag()
    name = torch.cuda.get_device_properties(0).name
    Ms = [m for m in MS if m <= 64] if args.quick else MS
    w8s = W8_SHAPES[:2] if args.quick else W8_SHAPES
    w4s = W4_SHAPES[:2] if args.quick else W4_SHAPES

    def log(msg):
        print(msg, flush=True)

    stamp = time.strftime("%Y-%m-%d")
    for t in args.tables.split(","):
        t0 = time.time()
        if t in ("gemm", "q8"):
            table = tune_w8(t, w8s, Ms, dev, log)
            prefix = "gemm_table" if t == "gemm" else "q8_table"
        elif t == "w4a8":
            table = tune_w4(w4s, Ms, dev, log)
            prefix = "w4a8_table"
        else:
            raise SystemExit(f"unknown table {t}")
        doc = {"gpu": name, "source": f"prism_amd.tune ({t}: weights streamed from HBM, graph-replayed launches, "
                                      f"median of 3), {stamp}", "table": table}
        path = os.path.join(args.out, f"{prefix}_{tag}.json")
        with open(path, "w") as f:
            json.dump(doc, f, indent=1, sort_keys=True)
        log(f"wrote {path} ({len(table)} shapes, {time.time() - t0:.0f} s)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
