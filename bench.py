#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

Metric: int4 GEMV HBM GB/s (config 2: W 14336 x 4096 int4 g32,
fp16 scales, fp16 x -> fp16 y) plus int4 dequant-GEMM TFLOP/s at M = 2048
(config 4).  A "step" is one call of the path over one batch; `value` is the
GEMV's whole-job throughput in GB/s with every input resident in HBM.

Timing: the K timed launches are captured once into a HIP graph (through torch's
graph API on the plugin's stream) and replayed, bracketed by HIP events on that
stream.  Weight/scale copies rotate over >= 512 MB so the 256 MB MALL cannot hold
them.  The CPU baseline times the oracle (a C restatement of the reference WGSL,
OpenMP) on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

C2 = dict(n_out=14336, k=4096, gs=32)
C2_BYTES = 14336 * 4096 // 2 + 14336 * (4096 // 32) * 2 + 4096 * 2 + 14336 * 2  # 33,067,008
C4 = dict(n_out=14336, k=4096, m=2048, gs=32)
C4_FLOPS = 2 * 2048 * 14336 * 4096
C3 = dict(n_out=28672, k=8192)
C5 = dict(n_out=11008, k=4096, m=256, gs=128)
INT8_MFMA_PEAK_TOPS = 5000.0
COPY_BYTES = 512 * 2**20
SPIN_CYCLES = 200_000  # device spin ahead of the timed replay (~0.1 ms of shader clocks)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.md")
MFMA_FILE = os.path.join(ROOT, "profiles", "mfma_utilization.md")


def _profile_value(path: str, tag: str, key: str, cast):
    """A `<tag> <key>: <value>` line of a committed rocprofv3 summary; None when absent."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"{tag} {key}:"):
                    return cast(line.split(":", 1)[1].strip().split()[0])
    except OSError:
        pass
    return None


def measured_traffic(key: str):
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    (scaled by the copy-kernel calibration), recorded in profiles/hbm_traffic.md as
    a line `traffic <key>: <bytes>`; None when not recorded."""
    return _profile_value(TRAFFIC_FILE, "traffic", key, int)


def measured_mfma_busy(key: str):
    """Fraction of the kernel's cycles with the matrix pipes busy, from rocprofv3 --pmc
    SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x GRBM_GUI_ACTIVE / 8), recorded in
    profiles/mfma_utilization.md as `mfma_busy <key>: <fraction>`; None when absent."""
    return _profile_value(MFMA_FILE, "mfma_busy", key, float)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def timed_graph(torch, ctx, launch, steps: int, warmup: int, settle_s: float = 0.025):
    """Warm up eagerly (`warmup` launches), capture `steps` launches into one graph,
    replay it untimed until the GPU has run this workload for `settle_s` seconds (the
    first replays after a switch of workload run at lower clocks), then time exactly
    one replay (`steps` launches) with HIP events on the launch stream.

    The timed replay is queued behind a short device-side spin and one more untimed
    replay, so every packet of it is already in the queue when the GPU reaches the
    first event: the events bracket the K launches back to back, without the host's
    graph-launch latency (tens of microseconds, which would otherwise be spread over
    the K launches).  Returns seconds for the timed replay."""
    s = torch.cuda.Stream()
    ctx.set_stream(s.cuda_stream)
    ctx.set_synchronous(False)
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            launch(i)
    t0 = time.perf_counter()
    for _ in range(50):
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= settle_s:
            break
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        torch.cuda._sleep(SPIN_CYCLES)  # holds the queue while the host enqueues the rest
        g.replay()                      # untimed: keeps the clocks at the workload's level
        e0.record(s)
        g.replay()
        e1.record(s)
    e1.synchronize()
    torch.cuda.synchronize()
    ctx.set_stream(None)
    ctx.set_synchronous(True)
    return e0.elapsed_time(e1) / 1e3


def bench_floor(torch, ctx, steps, warmup):
    """Streaming floor at config 2's size, with a kernel that is not this plugin's: torch's
    device copy moving C2_BYTES per launch (half read, half written), rotated over copies
    beyond the 256 MB MALL and timed like every leg; and the same copy at 512 MiB per
    launch, where the launch ramp and tail no longer matter.  What the C2 GEMV's HBM rate
    is compared against (`--only floor`; not in the default run)."""
    out = {}
    for label, nb, copies in (("c2_bytes", C2_BYTES // 2, 17), ("512MiB", COPY_BYTES // 2, 2)):
        src = [torch.empty(nb, dtype=torch.uint8, device="cuda").random_(0, 255) for _ in range(copies)]
        dst = [torch.empty_like(t) for t in src]

        def launch(i):
            dst[i % copies].copy_(src[i % copies])

        n = max(3, min(steps, 100))
        per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
        out[label] = {"bytes_per_launch": 2 * nb, "us_per_launch": round(per * 1e6, 2),
                      "gbs": round(2 * nb / per / 1e9, 1), "frac": round(2 * nb / per / 1e9 / HBM_PEAK_GBS, 4)}
        del src, dst
    return out


def bench_vendor(torch, steps, warmup):
    """The vendor library on config 4's shape, for comparison only: torch's plain bf16 GEMM
    (hipBLASLt) X[2048 x 4096] . W[4096 x 14336] with no quantization, as torch.mm with W
    stored [K x N] and as F.linear with W stored [N x K] (the weight layout of config 4).
    Eager launches timed with HIP events on the current stream (each is ~0.2 ms, so the
    launch gaps are negligible).  `--only vendor`; not in the default run."""
    import torch.nn.functional as F
    m, n, k = C4["m"], C4["n_out"], C4["k"]
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    w_kn = torch.randn(k, n, device="cuda", dtype=torch.bfloat16)
    w_nk = torch.randn(n, k, device="cuda", dtype=torch.bfloat16)
    out = {}
    for label, fn in (("mm_w_kxn", lambda: torch.mm(x, w_kn)), ("linear_w_nxk", lambda: F.linear(x, w_nk))):
        for _ in range(max(3, warmup)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n_it = max(5, min(steps, 50))
        e0.record()
        for _ in range(n_it):
            fn()
        e1.record()
        e1.synchronize()
        per = e0.elapsed_time(e1) / 1e3 / n_it
        tf = 2.0 * m * n * k / per / 1e12
        out[label] = {"us_per_launch": round(per * 1e6, 1), "tflops": round(tf, 1),
                      "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    return out


def bench_c2(torch, W, ctx, steps, warmup):
    from util import int4_weights
    r = np.random.default_rng(2)
    _, Wp, s = int4_weights(r, C2["n_out"], C2["k"], C2["gs"])
    x = r.standard_normal(C2["k"]).astype(np.float16)
    copies = max(2, -(-512 * 2**20 // (Wp.nbytes + s.nbytes)))
    # one weight copy and its scales per "layer", allocated together as a model loader would
    wbs, sbs = [], []
    for _ in range(copies):
        wbs.append(ctx.upload(Wp))
        sbs.append(ctx.upload(s))
    xb = ctx.upload(x)
    yb = ctx.alloc(C2["n_out"] * 2)
    d = W.qdesc(C2["n_out"], C2["k"], 1, 4, C2["gs"], W.NIBBLE_OFFSET_BINARY, W.SCALE_F16,
                W.F16, W.F16)

    def launch(i):
        ctx.qmatmul(d, wbs[i % copies], sbs[i % copies], xb, None, yb)

    sec = timed_graph(torch, ctx, launch, steps, warmup)
    per = sec / steps
    return {"sec": sec, "per_launch_s": per, "gbs": C2_BYTES / per / 1e9, "copies": copies,
            "W": Wp, "s": s, "x": x}


def bench_c4(torch, W, ctx, steps, warmup):
    from util import bf16_bits, int4_weights
    r = np.random.default_rng(4)
    _, Wp, s = int4_weights(r, C4["n_out"], C4["k"], C4["gs"])
    X = bf16_bits(r.standard_normal((C4["m"], C4["k"])).astype(np.float32))
    wb, sb, xb = ctx.upload(Wp), ctx.upload(s), ctx.upload(X)
    yb = ctx.alloc(C4["m"] * C4["n_out"] * 2)
    d = W.qdesc(C4["n_out"], C4["k"], C4["m"], 4, C4["gs"], W.NIBBLE_OFFSET_BINARY, W.SCALE_F16,
                W.BF16, W.BF16)
    ctx.qmatmul(d, wb, sb, xb, None, yb)  # raises NOT_SUPPORTED if no kernel

    def launch(i):
        ctx.qmatmul(d, wb, sb, xb, None, yb)

    n = max(3, min(steps, 50))
    sec = timed_graph(torch, ctx, launch, n, max(1, warmup // 4))
    per = sec / n
    tf = C4_FLOPS / per / 1e12
    return {"per_launch_s": per, "tflops": tf, "frac": tf / MFMA_F16_PEAK_TFLOPS, "steps": n}


C1_BYTES = 4096 * 4096 * 4 + 4096 * 4 + 4096 * 4  # W + x read, y written: 67,141,632


def bench_c1(torch, W, ctx, steps, warmup):
    """Config 1 through the ABI's own slot: op_matmul_f32(W, x, y, M=4096, K=4096, N=1)."""
    r = np.random.default_rng(1)
    A = (r.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    x = r.standard_normal(4096).astype(np.float32)
    copies = max(2, -(-512 * 2**20 // A.nbytes))
    abs_ = [ctx.upload(A) for _ in range(copies)]
    xb, yb = ctx.upload(x), ctx.alloc(4096 * 4)

    def launch(i):
        ctx.matmul_f32(abs_[i % copies], xb, yb, 4096, 4096, 1)

    n = max(3, min(steps, 100))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    for b in abs_:
        b.free()
    gbs = C1_BYTES / per / 1e9
    return {"us_per_launch": round(per * 1e6, 2), "value": round(gbs, 2), "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("c1")}}


def c3_bytes(m):
    """Algorithmic HBM bytes of one config-3 call: int8 W + fp16 row scales + X + Y."""
    return C3["n_out"] * C3["k"] + C3["n_out"] * 2 + m * C3["k"] * 2 + m * C3["n_out"] * 2


def bench_c3(torch, W, ctx, m, steps, warmup):
    from util import int8_weights
    r = np.random.default_rng(30 + m)
    q, s = int8_weights(r, C3["n_out"], C3["k"])
    X = r.standard_normal((m, C3["k"])).astype(np.float16)
    copies = max(2, -(-512 * 2**20 // q.nbytes))
    wbs = [ctx.upload(q) for _ in range(copies)]
    sb, xb = ctx.upload(s), ctx.upload(X)
    yb = ctx.alloc(m * C3["n_out"] * 2)
    d = W.qdesc(C3["n_out"], C3["k"], m, 8, C3["k"], 0, W.SCALE_F16, W.F16, W.F16)

    def launch(i):
        ctx.qmatmul(d, wbs[i % copies], sb, xb, None, yb)

    n = max(3, min(steps, 100))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    for b in wbs:
        b.free()
    gbs = c3_bytes(m) / per / 1e9
    return {"m": m, "us_per_launch": round(per * 1e6, 2), "value": round(gbs, 2), "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic(f"c3m{m}")}}


def bench_c5(torch, W, ctx, steps, warmup):
    from util import int4_weights, quantize_rows_int8
    r = np.random.default_rng(5)
    _, Wp, s = int4_weights(r, C5["n_out"], C5["k"], C5["gs"], 1)
    a8, asc = quantize_rows_int8(r.standard_normal((C5["m"], C5["k"])).astype(np.float32))
    wb, sb, xb, asb = ctx.upload(Wp), ctx.upload(s), ctx.upload(a8), ctx.upload(asc)
    yb = ctx.alloc(C5["m"] * C5["n_out"] * 2)
    d = W.qdesc(C5["n_out"], C5["k"], C5["m"], 4, C5["gs"], 1, W.SCALE_F16, W.I8, W.F16)

    def launch(i):
        ctx.qmatmul(d, wb, sb, xb, asb, yb)

    n = max(3, min(steps, 100))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    ops = 2 * C5["m"] * C5["n_out"] * C5["k"]
    nbytes = Wp.nbytes + s.nbytes + a8.nbytes + asc.nbytes + C5["m"] * C5["n_out"] * 2
    tops = ops / per / 1e12
    return {"us_per_launch": round(per * 1e6, 2), "value": round(tops, 2), "unit": "TOP/s",
            "hbm_gbs": round(nbytes / per / 1e9, 2),
            "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_MFMA_PEAK_TOPS,
                         "unit": "TOP/s", "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4),
                         "traffic": measured_traffic("c5"), "mfma_busy": measured_mfma_busy("c5")}}


def bench_w8a8(torch, W, ctx, steps, warmup):
    """W8A8 at config 5's shape: int8 weights 11008 x 4096 with fp16 g128 scales x int8
    activations 256 x 4096 (per-token scales), fp16 out (matmul_int8 with group scales)."""
    from util import int8_weights, quantize_rows_int8
    r = np.random.default_rng(8)
    q, _ = int8_weights(r, C5["n_out"], C5["k"])
    s = r.uniform(0.001, 0.01, size=(C5["n_out"], C5["k"] // C5["gs"])).astype(np.float16)
    a8, asc = quantize_rows_int8(r.standard_normal((C5["m"], C5["k"])).astype(np.float32))
    wb, sb, xb, asb = ctx.upload(q), ctx.upload(s), ctx.upload(a8), ctx.upload(asc)
    yb = ctx.alloc(C5["m"] * C5["n_out"] * 2)
    d = W.qdesc(C5["n_out"], C5["k"], C5["m"], 8, C5["gs"], 0, W.SCALE_F16, W.I8, W.F16)

    def launch(i):
        ctx.qmatmul(d, wb, sb, xb, asb, yb)

    n = max(3, min(steps, 100))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    ops = 2 * C5["m"] * C5["n_out"] * C5["k"]
    tops = ops / per / 1e12
    nbytes = q.nbytes + s.nbytes + a8.nbytes + asc.nbytes + C5["m"] * C5["n_out"] * 2
    return {"us_per_launch": round(per * 1e6, 2), "value": round(tops, 2), "unit": "TOP/s",
            "hbm_gbs": round(nbytes / per / 1e9, 2),
            "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_MFMA_PEAK_TOPS,
                         "unit": "TOP/s", "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4),
                         "traffic": measured_traffic("w8a8")}}


QW_BYTES = 14336 * 4096 * 4 + 14336 * 4096 // 2 + 14336 * (4096 // 32) * 2  # read f32, write int4 + f16 scales


def bench_quantize(torch, W, ctx, steps, warmup):
    """Producer of configs 2/4: fp32 W [14336 x 4096] -> int4 g32 offset-binary + fp16
    scales (compute_group_scales + quantize_nax_int4_sym in one pass)."""
    r = np.random.default_rng(40)
    x = (r.standard_normal((14336, 4096)) * 0.02).astype(np.float32)
    copies = 3  # 3 x 235 MB of fp32 input: more than the 256 MB MALL holds
    xbs = [ctx.upload(x) for _ in range(copies)]
    qb, sb = ctx.alloc(14336 * 4096 // 2), ctx.alloc(14336 * 128 * 2)
    d = W.quant_desc(14336, 4096, 4, 32, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, W.F32)

    def launch(i):
        ctx.quantize(d, xbs[i % copies], qb, sb)

    n = max(3, min(steps, 30))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    for b in xbs:
        b.free()
    gbs = QW_BYTES / per / 1e9
    return {"us_per_launch": round(per * 1e6, 2), "value": round(gbs, 2), "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("quant")}}


DQ_BYTES = 14336 * 4096 // 2 + 14336 * (4096 // 32) * 2 + 14336 * 4096 * 4  # int4 + f16 scales in, f32 out
GB = {"batch": 64, "m": 4096, "n": 128}  # 64 heads x 4096 cached keys x head dim 128
GB_BYTES = GB["batch"] * (GB["m"] * GB["n"] + GB["n"] + GB["m"]) * 4  # A + x read, y written


def bench_dequantize(torch, W, ctx, steps, warmup):
    """dequantize_nax_int4_sym on config-4 weights: int4 g32 + fp16 scales -> fp32 W
    [14336 x 4096] (the reference's f32 output)."""
    from util import int4_weights
    r = np.random.default_rng(41)
    _, Wp, sc = int4_weights(r, 14336, 4096, 32)
    copies = 3
    qbs = [ctx.upload(Wp) for _ in range(copies)]
    sbs = [ctx.upload(sc) for _ in range(copies)]
    ob = ctx.alloc(14336 * 4096 * 4)
    d = W.quant_desc(14336, 4096, 4, 32, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, W.F32)

    def launch(i):
        ctx.dequantize(d, qbs[i % copies], sbs[i % copies], ob)

    n = max(3, min(steps, 30))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    for b in qbs + sbs + [ob]:
        b.free()
    gbs = DQ_BYTES / per / 1e9
    return {"us_per_launch": round(per * 1e6, 2), "value": round(gbs, 2), "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("dequant")}}


def bench_gemv_batched(torch, W, ctx, steps, warmup):
    """gemv_batched: 64 fp32 GEMVs of 4096 x 128 (one per head, a decode step's q.K^T over
    a 4096-token cache), one launch."""
    r = np.random.default_rng(42)
    B, M, N = GB["batch"], GB["m"], GB["n"]
    A = (r.standard_normal(B * M * N) * 0.02).astype(np.float32)
    x = r.standard_normal(B * N).astype(np.float32)
    copies = max(2, -(-512 * 2**20 // A.nbytes))
    abs_ = [ctx.upload(A) for _ in range(copies)]
    xb, yb = ctx.upload(x), ctx.alloc(B * M * 4)

    def launch(i):
        ctx.gemv_f32_batched(abs_[i % copies], xb, yb, M, N, B, M * N, N, M)

    n = max(3, min(steps, 100))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    for b in abs_ + [xb, yb]:
        b.free()
    gbs = GB_BYTES / per / 1e9
    return {"us_per_launch": round(per * 1e6, 2), "value": round(gbs, 2), "unit": "GB/s",
            "workload": f"{B} x ({M} x {N}) fp32, strides {M * N}/{N}/{M}",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("gemvb")}}


GT_BYTES = 4096 * 4096 * 4 + 4096 * 4 + 4096 * 4  # A + x read, y written


def bench_gemv_t(torch, W, ctx, steps, warmup):
    """gemv_transpose: y[4096] = A^T x over a 4096 x 4096 fp32 A (the config-1 matrix)."""
    r = np.random.default_rng(43)
    A = (r.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    x = r.standard_normal(4096).astype(np.float32)
    copies = max(2, -(-512 * 2**20 // A.nbytes))
    abs_ = [ctx.upload(A) for _ in range(copies)]
    xb, yb = ctx.upload(x), ctx.alloc(4096 * 4)

    def launch(i):
        ctx.gemv_f32(abs_[i % copies], xb, yb, 4096, 4096, trans=True)

    n = max(3, min(steps, 100))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    for b in abs_ + [xb, yb]:
        b.free()
    gbs = GT_BYTES / per / 1e9
    return {"us_per_launch": round(per * 1e6, 2), "value": round(gbs, 2), "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("gemvt")}}


MFMA_F32_PEAK_TFLOPS = 157.3


def bench_gemm_f32(torch, W, ctx, n, steps, warmup):
    """op_matmul_f32 as a general GEMM, C[n x n] = A[n x n] B[n x n] fp32 (the vtable's
    only matmul slot, src/webgpu_plugin.cpp:1721-1771; the reference README quotes 1024^2)."""
    r = np.random.default_rng(50 + n)
    A = r.standard_normal((n, n)).astype(np.float32)
    B = r.standard_normal((n, n)).astype(np.float32)
    ab, bb, cb = ctx.upload(A), ctx.upload(B), ctx.alloc(n * n * 4)

    def launch(i):
        ctx.matmul_f32(ab, bb, cb, n, n, n)

    k = max(3, min(steps, 50))
    per = timed_graph(torch, ctx, launch, k, max(1, warmup // 4)) / k
    for b in (ab, bb, cb):
        b.free()
    tf = 2.0 * n * n * n / per / 1e12
    return {"n": n, "us_per_launch": round(per * 1e6, 2), "value": round(tf, 2), "unit": "TFLOP/s",
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": MFMA_F32_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / MFMA_F32_PEAK_TFLOPS, 4),
                         "traffic": measured_traffic(f"gemm{n}")}}


GH_BYTES = 14336 * 4096 * 2 + 4096 * 2 + 14336 * 4  # A (f16) + x read, y (f32) written


def bench_gemv_f16(torch, W, ctx, steps, warmup):
    """fp16 GEMV with fp32 accumulation: y[14336] = A[14336 x 4096] x (config 2's shape, fp16
    weights)."""
    r = np.random.default_rng(44)
    A = (r.standard_normal((14336, 4096)) * 0.02).astype(np.float16)
    x = r.standard_normal(4096).astype(np.float16)
    copies = max(2, -(-512 * 2**20 // A.nbytes))
    abs_ = [ctx.upload(A) for _ in range(copies)]
    xb, yb = ctx.upload(x), ctx.alloc(14336 * 4)

    def launch(i):
        ctx.gemv_f16(abs_[i % copies], xb, yb, 14336, 4096)

    n = max(3, min(steps, 100))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    for b in abs_ + [xb, yb]:
        b.free()
    gbs = GH_BYTES / per / 1e9
    return {"us_per_launch": round(per * 1e6, 2), "value": round(gbs, 2), "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("gemvh")}}


FFN = dict(hidden=4096, inter=14336, gs=32)


def ffn_bytes():
    h, i, gs = FFN["hidden"], FFN["inter"], FFN["gs"]
    w = 2 * i * h // 2 + 2 * i * (h // gs) * 2 + h * i // 2 + h * (i // gs) * 2  # int4 + fp16 scales
    act = h * 4 * 2 + h * 4 + i * 2 * 2 + h * 4  # x (twice), gamma, h (written, read), x_next
    return w + act


def bench_ffn(torch, W, ctx, steps, warmup):
    """One decode step of a gated FFN through the plugin: rms_norm (f32 -> f16) fused into
    the int4 g32 gate/up GEMV with the SILU_MUL epilogue (2 x 14336 x 4096,
    lux_hip_rms_norm_qmatmul), then the int4 g32 down GEMV (4096 x 14336) with the
    residual added in its ADD_RESIDUAL epilogue: two launches.  Weights rotate over copies
    beyond the MALL."""
    from util import int4_weights
    h, i, gs = FFN["hidden"], FFN["inter"], FFN["gs"]
    r = np.random.default_rng(45)
    _, Wgu, sgu = int4_weights(r, 2 * i, h, gs)
    _, Wd, sd = int4_weights(r, h, i, gs)
    copies = 3
    wgu = [ctx.upload(Wgu) for _ in range(copies)]
    s_gu = [ctx.upload(sgu) for _ in range(copies)]
    wd = [ctx.upload(Wd) for _ in range(copies)]
    s_d = [ctx.upload(sd) for _ in range(copies)]
    x = ctx.upload(r.standard_normal(h).astype(np.float32))
    gamma = ctx.upload(r.uniform(0.8, 1.2, h).astype(np.float32))
    hb, xn = ctx.alloc(i * 2), ctx.alloc(h * 4)
    d_gu = W.qdesc(2 * i, h, 1, 4, gs, 0, W.SCALE_F16, W.F16, W.F16)
    d_d = W.qdesc(h, i, 1, 4, gs, 0, W.SCALE_F16, W.F16, W.F32)

    def launch(j):
        k = j % copies
        ctx.rms_norm_qmatmul(x, gamma, 1e-6, W.F32, d_gu, wgu[k], s_gu[k], W.EPI_SILU_MUL, None, None, hb)
        ctx.qmatmul_ex(d_d, wd[k], s_d[k], hb, None, W.EPI_ADD_RESIDUAL, None, x, xn)

    n = max(3, min(steps, 60))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    for b in wgu + s_gu + wd + s_d + [x, gamma, hb, xn]:
        b.free()
    gbs = ffn_bytes() / per / 1e9
    return {"us_per_step": round(per * 1e6, 2), "value": round(gbs, 2), "unit": "GB/s",
            "workload": f"hidden {h}, intermediate {i}, int4 g{gs} fp16 scales, m = 1",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("ffn")}}


def bench_c5_fp(torch, W, ctx, steps, warmup):
    """Config 5 from fp32 activations: per-token int8 quantization (QUANTIZE_X) + W4A8."""
    from util import int4_weights
    r = np.random.default_rng(5)
    _, Wp, s = int4_weights(r, C5["n_out"], C5["k"], C5["gs"], 1)
    x = r.standard_normal((C5["m"], C5["k"])).astype(np.float32)
    wb, sb, xb = ctx.upload(Wp), ctx.upload(s), ctx.upload(x)
    yb = ctx.alloc(C5["m"] * C5["n_out"] * 2)
    d = W.qdesc(C5["n_out"], C5["k"], C5["m"], 4, C5["gs"], 1, W.SCALE_F16, W.F32, W.F16,
                W.QFLAG_QUANTIZE_X)
    ctx.qmatmul(d, wb, sb, xb, None, yb)  # sizes the workspace outside the capture

    def launch(i):
        ctx.qmatmul(d, wb, sb, xb, None, yb)

    n = max(3, min(steps, 100))
    per = timed_graph(torch, ctx, launch, n, max(1, warmup // 4)) / n
    tops = 2 * C5["m"] * C5["n_out"] * C5["k"] / per / 1e12
    return {"us_per_launch": round(per * 1e6, 2), "value": round(tops, 2), "unit": "TOP/s",
            "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_MFMA_PEAK_TOPS,
                         "unit": "TOP/s", "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4),
                         "traffic": None}}


def host_cpu():
    """CPU model string and the host's logical CPU count as this process sees them."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count()
    return model, os.cpu_count(), avail


CPU_LABEL = ("CPU restatement, not SwiftShader: oracle/lux_oracle.c (the reference WGSL's "
             "arithmetic in C, OpenMP); Dawn/SwiftShader is not in this image")


def cpu_baseline_c2(Wp, s, x, budget_s=10.0):
    import oracle
    sf = s.astype(np.float32).reshape(-1)
    xf = x.astype(np.float32).reshape(-1, 1)
    oracle.matmul_nax_grouped(Wp, sf, xf, C2["gs"])  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.matmul_nax_grouped(Wp, sf, xf, C2["gs"])
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 5000:
            break
    model, ncpu, avail = host_cpu()
    return {"value": round(C2_BYTES * n / el / 1e9, 3), "unit": "GB/s",
            "cores": oracle.num_threads(), "kind": "port", "label": CPU_LABEL,
            "cpu_model": model, "nproc": avail, "host_logical_cpus": ncpu,
            "sample": f"full config-2 GEMV (14336x4096 int4 g32) x{n} calls in {el:.1f} s, "
                      "lo_matmul_nax_grouped (matmul_nax_grouped, quantized_nax.wgsl:568-626)"}


C4_CPU_TOKENS = 32  # bounded CPU sample of config 4: 32 of the 2048 activation rows


def cpu_baseline_c4(budget_s=10.0):
    """Config 4 on the host: the oracle's matmul_nax_grouped over the full 14336 x 4096
    int4 g32 weights and a 32-token slice of the activations (the work per token is the
    same at any M, so TFLOP/s scales; 2048 tokens would take minutes)."""
    import oracle
    from util import int4_weights
    r = np.random.default_rng(4)
    _, Wp, s = int4_weights(r, C4["n_out"], C4["k"], C4["gs"])
    sf = s.astype(np.float32).reshape(-1)
    act = r.standard_normal((C4["k"], C4_CPU_TOKENS)).astype(np.float32)
    oracle.matmul_nax_grouped(Wp, sf, act, C4["gs"])  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.matmul_nax_grouped(Wp, sf, act, C4["gs"])
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 5000:
            break
    flops = 2 * C4_CPU_TOKENS * C4["n_out"] * C4["k"] * n
    model, ncpu, avail = host_cpu()
    return {"value": round(flops / el / 1e12, 5), "unit": "TFLOP/s",
            "cores": oracle.num_threads(), "kind": "port", "label": CPU_LABEL,
            "cpu_model": model, "nproc": avail, "host_logical_cpus": ncpu,
            "sample": f"config-4 weights (14336x4096 int4 g32) x {C4_CPU_TOKENS} of the 2048 tokens, "
                      f"x{n} calls in {el:.1f} s; TFLOP/s of that sample"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c4", "c5", "copy", "floor", "vendor", "quant", "dequant", "gemvb",
                                       "gemvt", "gemvh", "w8a8", "ffn", "gemm"],
                    default=None,
                    help="run one leg only and log its timing (profiling); the JSON line comes "
                         "from the full run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the path would shard over weight rows (output channels), each GPU running "
              "the same kernels on its rows with no communication",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import webgpu_amd as W

    plugin = W.Plugin()
    ctx = plugin.create_context(0)
    log(f"device: {ctx.info().name.decode()}")
    if args.only == "c4":
        c4 = bench_c4(torch, W, ctx, args.steps, args.warmup)
        log(f"  C4 {c4['per_launch_s']*1e6:.1f} us/launch, {c4['tflops']:.1f} TFLOP/s")
        return
    if args.only == "copy":
        # calibration for the FETCH_SIZE / WRITE_SIZE counters: a plain device copy
        # of known size (COPY_BYTES read + COPY_BYTES written per launch)
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"  copy {COPY_BYTES} bytes x5 done")
        return
    if args.only == "vendor":
        for k, v in bench_vendor(torch, args.steps, args.warmup).items():
            log(f"  hipBLASLt bf16 {k}: {v['us_per_launch']} us, {v['tflops']} TFLOP/s ({100 * v['frac']:.1f} % of 2.5 PF)")
        c4 = bench_c4(torch, W, ctx, args.steps, args.warmup)
        log(f"  C4 {c4['per_launch_s']*1e6:.1f} us/launch, {c4['tflops']:.1f} TFLOP/s")
        return
    if args.only == "floor":
        fl = bench_floor(torch, ctx, args.steps, args.warmup)
        for k, v in fl.items():
            log(f"  device copy, {v['bytes_per_launch']} bytes moved per launch: {v['us_per_launch']} us, "
                f"{v['gbs']} GB/s ({100 * v['frac']:.1f} % of 8 TB/s)")
        return
    if args.only == "c1":
        c1 = bench_c1(torch, W, ctx, args.steps, args.warmup)
        log(f"  C1 {c1['us_per_launch']} us/launch, {c1['value']} GB/s")
        return
    if args.only == "c3":
        for m in (8, 32):
            c3 = bench_c3(torch, W, ctx, m, args.steps, args.warmup)
            log(f"  C3 m={m} {c3['us_per_launch']} us/launch, {c3['value']} GB/s")
        return
    if args.only == "c5":
        c5 = bench_c5(torch, W, ctx, args.steps, args.warmup)
        log(f"  C5 {c5['us_per_launch']} us/launch, {c5['value']} TOP/s, {c5['hbm_gbs']} GB/s")
        c5f = bench_c5_fp(torch, W, ctx, args.steps, args.warmup)
        log(f"  C5 from fp32 activations {c5f['us_per_launch']} us/launch, {c5f['value']} TOP/s")
        return
    if args.only == "quant":
        qz = bench_quantize(torch, W, ctx, args.steps, args.warmup)
        log(f"  quantize {qz['us_per_launch']} us/launch, {qz['value']} GB/s")
        return
    if args.only == "dequant":
        dq = bench_dequantize(torch, W, ctx, args.steps, args.warmup)
        log(f"  dequantize {dq['us_per_launch']} us/launch, {dq['value']} GB/s")
        return
    if args.only == "ffn":
        ff = bench_ffn(torch, W, ctx, args.steps, args.warmup)
        log(f"  decode FFN step {ff['us_per_step']} us/step, {ff['value']} GB/s")
        return
    if args.only == "w8a8":
        w8 = bench_w8a8(torch, W, ctx, args.steps, args.warmup)
        log(f"  W8A8 {w8['us_per_launch']} us/launch, {w8['value']} TOP/s, {w8['hbm_gbs']} GB/s")
        return
    if args.only == "gemvh":
        gh = bench_gemv_f16(torch, W, ctx, args.steps, args.warmup)
        log(f"  gemv_f16 {gh['us_per_launch']} us/launch, {gh['value']} GB/s")
        return
    if args.only == "gemvt":
        gt = bench_gemv_t(torch, W, ctx, args.steps, args.warmup)
        log(f"  gemv_transpose {gt['us_per_launch']} us/launch, {gt['value']} GB/s")
        return
    if args.only == "gemvb":
        gb = bench_gemv_batched(torch, W, ctx, args.steps, args.warmup)
        log(f"  gemv_batched {gb['us_per_launch']} us/launch, {gb['value']} GB/s")
        return
    if args.only == "gemm":
        for n in (1024, 4096):
            gm = bench_gemm_f32(torch, W, ctx, n, args.steps, args.warmup)
            log(f"  gemm_f32 {n}^3 {gm['us_per_launch']} us/launch, {gm['value']} TFLOP/s")
        return
    log("bench: config 2 int4 GEMV")
    c2 = bench_c2(torch, W, ctx, args.steps, args.warmup)
    log(f"  C2 {c2['per_launch_s']*1e6:.2f} us/launch, {c2['gbs']:.1f} GB/s")
    if args.only == "c2":
        return
    c4 = None
    try:
        log("bench: config 4 int4 GEMM M=2048")
        c4 = bench_c4(torch, W, ctx, args.steps, args.warmup)
        log(f"  C4 {c4['per_launch_s']*1e6:.1f} us/launch, {c4['tflops']:.1f} TFLOP/s")
    except W.LuxError as e:
        log(f"  C4 skipped: {e}")
    c1, c3s, c5, c5f, qz, dq, gb, gt, gh, w8, ff = None, [], None, None, None, None, None, None, None, None, None
    gms = []
    try:
        log("bench: config 1 fp32 GEMV through op_matmul_f32")
        c1 = bench_c1(torch, W, ctx, args.steps, args.warmup)
        log(f"  C1 {c1['us_per_launch']} us/launch, {c1['value']} GB/s")
        log("bench: config 3 int8 GEMM M=8,32")
        for m in (8, 32):
            c3s.append(bench_c3(torch, W, ctx, m, args.steps, args.warmup))
            log(f"  C3 m={m} {c3s[-1]['us_per_launch']} us/launch, {c3s[-1]['value']} GB/s")
        log("bench: config 5 W4A8 M=256")
        c5 = bench_c5(torch, W, ctx, args.steps, args.warmup)
        log(f"  C5 {c5['us_per_launch']} us/launch, {c5['value']} TOP/s")
        log("bench: config 5 from fp32 activations (per-token quantization + W4A8)")
        c5f = bench_c5_fp(torch, W, ctx, args.steps, args.warmup)
        log(f"  C5 fp32-x {c5f['us_per_launch']} us/launch, {c5f['value']} TOP/s")
        log("bench: W8A8 at config 5's shape (int8 weights)")
        w8 = bench_w8a8(torch, W, ctx, args.steps, args.warmup)
        log(f"  W8A8 {w8['us_per_launch']} us/launch, {w8['value']} TOP/s")
        log("bench: int4 g32 quantizer on config-4 weights (fp32 -> int4 + fp16 scales)")
        qz = bench_quantize(torch, W, ctx, args.steps, args.warmup)
        log(f"  quantize {qz['us_per_launch']} us/launch, {qz['value']} GB/s")
        log("bench: int4 g32 dequantizer on config-4 weights (int4 + fp16 scales -> fp32)")
        dq = bench_dequantize(torch, W, ctx, args.steps, args.warmup)
        log(f"  dequantize {dq['us_per_launch']} us/launch, {dq['value']} GB/s")
        log("bench: batched fp32 GEMV, 64 x 4096 x 128")
        gb = bench_gemv_batched(torch, W, ctx, args.steps, args.warmup)
        log(f"  gemv_batched {gb['us_per_launch']} us/launch, {gb['value']} GB/s")
        log("bench: transposed fp32 GEMV, 4096 x 4096")
        gt = bench_gemv_t(torch, W, ctx, args.steps, args.warmup)
        log(f"  gemv_transpose {gt['us_per_launch']} us/launch, {gt['value']} GB/s")
        log("bench: fp16 GEMV, 14336 x 4096")
        gh = bench_gemv_f16(torch, W, ctx, args.steps, args.warmup)
        log(f"  gemv_f16 {gh['us_per_launch']} us/launch, {gh['value']} GB/s")
        log("bench: decode FFN step (rms_norm fused into gate/up + SILU_MUL, down + residual)")
        ff = bench_ffn(torch, W, ctx, args.steps, args.warmup)
        log(f"  decode FFN step {ff['us_per_step']} us/step, {ff['value']} GB/s")
        log("bench: fp32 GEMM through op_matmul_f32, 1024^3 and 4096^3")
        for n in (1024, 4096):
            gms.append(bench_gemm_f32(torch, W, ctx, n, args.steps, args.warmup))
            log(f"  gemm_f32 {n}^3 {gms[-1]['us_per_launch']} us/launch, {gms[-1]['value']} TFLOP/s")
    except W.LuxError as e:
        log(f"  C1/C3/C5 skipped: {e}")
    cpu, cpu4 = None, None
    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle)")
        cpu = cpu_baseline_c2(c2["W"], c2["s"], c2["x"], args.cpu_budget)
        log(f"  CPU {cpu['value']} GB/s on {cpu['cores']} threads")
        log("bench: CPU baseline, config 4 sample (oracle)")
        cpu4 = cpu_baseline_c4(args.cpu_budget)
        log(f"  CPU C4 sample {cpu4['value']} TFLOP/s on {cpu4['cores']} threads")

    gbs = c2["gbs"]
    out = {
        "metric": "int4 GEMV HBM GB/s (% of 8 TB/s) + int4 GEMM TFLOPS (% MFMA peak) @M=2048",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["per_launch_s"] * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights, fp16 activations/scales, fp32 accumulate",
        "data": "synthetic (seeded numpy, BASELINE.json config 2 distributions)",
        "config": {"workload": "config 2: int4 g32 weight-only GEMV, W 14336x4096 offset-binary, "
                               "fp16 scales U(0.005,0.02), x fp16 N(0,1), y fp16",
                   "n_out": 14336, "k": 4096, "m": 1, "group_size": 32,
                   "weight_copies_rotated": c2["copies"],
                   "timing": "one replay of a HIP graph of K launches, queued behind a device spin and an untimed replay; HIP events on the launch stream"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("c2")},
        "cpu_baseline": cpu,
        "int4_gemm_m2048": None if c4 is None else {
            "value": round(c4["tflops"], 2), "unit": "TFLOP/s",
            "us_per_launch": round(c4["per_launch_s"] * 1e6, 2),
            "roofline": {"bound": "mfma", "achieved": round(c4["tflops"], 2),
                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(c4["frac"], 4), "traffic": measured_traffic("c4"),
                         "mfma_busy": measured_mfma_busy("c4")},
            "cpu_baseline": cpu4},
        "fp32_gemv_c1": c1,
        "int8_gemm_c3": c3s or None,
        "w4a8_gemm_c5": c5,
        "w4a8_c5_from_fp32_activations": c5f,
        "w8a8_config5_shape": w8,
        "quantize_int4_g32_c4_weights": qz,
        "dequantize_int4_g32_c4_weights": dq,
        "gemv_f32_batched": gb,
        "gemv_f32_transpose": gt,
        "gemv_f16": gh,
        "decode_ffn_step": ff,
        "gemm_f32_op_matmul": gms or None,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
