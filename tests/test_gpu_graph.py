"""GPU: the asynchronous stream mode of the plugin under HIP graph capture.

A caller that sets lux_hip_context_set_synchronous(ctx, 0) and its own stream may capture
the plugin's launches in a graph (bench.py times every config that way).  One graph holds
a decode step (rms_norm -> int4 gate/up GEMM with SILU_MUL -> int4 down GEMV -> residual
op_add_f32), a large-m int4 GEMM with bf16 activations (pre-pass + MFMA GEMM, workspace),
a W4A8 GEMM with QUANTIZE_X (per-token quantizer + int8 MFMA, workspace) and the gate/up
GEMV with rms_norm in its prologue (lux_hip_rms_norm_qmatmul).  It is
replayed three times with new inputs written by eager torch work between the replays;
every replay must equal, bit for bit, the same ops run eagerly in synchronous mode (the
kernels are deterministic, so graph and eager results are identical).
"""
import numpy as np
import pytest

import webgpu_amd as W
from util import int4_weights, rng

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(plugin):
    import torch
    c = plugin.create_context(0)
    try:
        r = rng(4242)
        hidden, inter, gs = 1024, 512, 32
        x = torch.tensor(r.standard_normal(hidden), dtype=torch.float32, device="cuda")
        gamma = torch.tensor(r.uniform(0.8, 1.2, hidden), dtype=torch.float32, device="cuda")
        _, Wgu, sgu = int4_weights(r, 2 * inter, hidden, gs)
        _, Wd, sd = int4_weights(r, hidden, inter, gs)
        ml, nl, kl = 100, 256, 512                      # large-m int4 GEMM, bf16 activations
        _, Wl, sl = int4_weights(r, nl, kl, 32)
        xl = torch.tensor(r.standard_normal((ml, kl)), dtype=torch.bfloat16, device="cuda")
        mq, nq, kq = 64, 256, 512                       # W4A8 with per-token quantization
        _, Wq, sq = int4_weights(r, nq, kq, 128, 1)
        xq = torch.tensor(r.standard_normal((mq, kq)), dtype=torch.float32, device="cuda")

        xb, gb, xlb, xqb = c.wrap(x), c.wrap(gamma), c.wrap(xl), c.wrap(xq)
        wgu, s_gu, wd, s_d = c.upload(Wgu), c.upload(sgu), c.upload(Wd), c.upload(sd)
        wl, s_l, wq, s_q = c.upload(Wl), c.upload(sl), c.upload(Wq), c.upload(sq)
        nb, hb = c.alloc(hidden * 2), c.alloc(inter * 2)
        d_gu = W.qdesc(2 * inter, hidden, 1, 4, gs, 0, W.SCALE_F16, W.F16, W.F16)
        d_d = W.qdesc(hidden, inter, 1, 4, gs, 0, W.SCALE_F16, W.F16, W.F32)
        d_l = W.qdesc(nl, kl, ml, 4, 32, 0, W.SCALE_F16, W.BF16, W.BF16)
        d_q = W.qdesc(nq, kq, mq, 4, 128, 1, W.SCALE_F16, W.F32, W.F16, W.QFLAG_QUANTIZE_X)
        shapes = {"d": (hidden * 4, np.float32, (hidden,)), "res": (hidden * 4, np.float32, (hidden,)),
                  "large": (ml * nl * 2, np.uint16, (ml, nl)), "w4a8": (mq * nq * 2, np.uint16, (mq, nq)),
                  "fused": (inter * 2, np.float16, (inter,))}

        def outputs():
            return {k: c.alloc(v[0]) for k, v in shapes.items()}

        def run(o):
            c.rms_norm(xb, gb, nb, 1, hidden, 1e-6, W.F32, W.F16)
            c.qmatmul_ex(d_gu, wgu, s_gu, nb, None, W.EPI_SILU_MUL, None, None, hb)
            c.qmatmul(d_d, wd, s_d, hb, None, o["d"])
            c.binary_f32("add", xb, o["d"], o["res"], hidden)
            c.qmatmul(d_l, wl, s_l, xlb, None, o["large"])
            c.qmatmul(d_q, wq, s_q, xqb, None, o["w4a8"])
            c.rms_norm_qmatmul(xb, gb, 1e-6, W.F32, d_gu, wgu, s_gu, W.EPI_SILU_MUL, None, None, o["fused"])

        def fetch(o):
            return {k: c.download(o[k], v[1], v[2]) for k, v in shapes.items()}

        og, oe = outputs(), outputs()
        run(og)  # eager first: workspaces are sized outside the capture
        s = torch.cuda.Stream()
        c.set_stream(s.cuda_stream)
        c.set_synchronous(False)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            run(og)
        c.set_stream(None)
        c.set_synchronous(True)

        prev = None
        for i in range(3):
            # new inputs from eager torch work on the default stream
            x.mul_(1.25).add_(0.5 * (i + 1))
            xl.copy_(torch.tensor(r.standard_normal((ml, kl)), dtype=torch.bfloat16))
            xq.mul_(-0.75).add_(0.25)
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                g.replay()
            torch.cuda.synchronize()
            got = fetch(og)
            run(oe)  # the same ops, synchronous, on the context's own stream
            ref = fetch(oe)
            for k in shapes:
                assert np.array_equal(got[k].view(np.uint8), ref[k].view(np.uint8)), f"replay {i}: {k}"
            # rms_norm inside the gate/up GEMV gives the bits of the separate rms_norm
            assert np.array_equal(got["fused"].view(np.uint16), c.download(hb, np.float16, (inter,)).view(np.uint16))
            if prev is not None:  # the replay saw the new inputs
                assert not np.array_equal(got["res"], prev["res"])
                assert not np.array_equal(got["large"], prev["large"])
                assert not np.array_equal(got["w4a8"], prev["w4a8"])
            prev = got
    finally:
        c.close()


def test_graph_codecs_and_gemv_forms(plugin):
    """The dequantizer, the batched GEMV, the two-pass transposed GEMV (context workspace)
    and the fp16 batched dot in one graph: three replays with new inputs, each equal bit
    for bit to the same ops run eagerly."""
    import torch
    c = plugin.create_context(0)
    try:
        r = rng(4343)
        rows, k, gs = 512, 1024, 32
        _, Wq, sq = int4_weights(r, rows, k, gs)
        B, Mb, Nb = 8, 256, 128
        Ab = torch.tensor(r.standard_normal(B * Mb * Nb), dtype=torch.float32, device="cuda")
        xb_t = torch.tensor(r.standard_normal(B * Nb), dtype=torch.float32, device="cuda")
        Mt, Nt = 1000, 512
        At = torch.tensor(r.standard_normal((Mt, Nt)), dtype=torch.float32, device="cuda")
        xt_t = torch.tensor(r.standard_normal(Mt), dtype=torch.float32, device="cuda")
        nv, size = 64, 1024
        da = torch.tensor(r.standard_normal(nv * size), dtype=torch.float16, device="cuda")
        db = torch.tensor(r.standard_normal(nv * size), dtype=torch.float16, device="cuda")

        wq, s_q = c.upload(Wq), c.upload(sq)
        ab, xbb, at, xtb, dab, dbb = c.wrap(Ab), c.wrap(xb_t), c.wrap(At), c.wrap(xt_t), c.wrap(da), c.wrap(db)
        dq = W.quant_desc(rows, k, 4, gs, 0, W.SCALE_F16, W.F32)
        shapes = {"deq": (rows * k * 4, np.float32, (rows, k)), "gb": (B * Mb * 4, np.float32, (B * Mb,)),
                  "gt": (Nt * 4, np.float32, (Nt,)), "dot": (nv * 4, np.float32, (nv,))}

        def outputs():
            return {key: c.alloc(v[0]) for key, v in shapes.items()}

        def run(o):
            c.dequantize(dq, wq, s_q, o["deq"])
            c.gemv_f32_batched(ab, xbb, o["gb"], Mb, Nb, B, Mb * Nb, Nb, Mb)
            c.gemv_f32(at, xtb, o["gt"], Mt, Nt, trans=True)
            c.dot_f16(dab, dbb, o["dot"], size, nv, size)

        def fetch(o):
            return {key: c.download(o[key], v[1], v[2]) for key, v in shapes.items()}

        og, oe = outputs(), outputs()
        run(og)  # sizes the workspace outside the capture
        s = torch.cuda.Stream()
        c.set_stream(s.cuda_stream)
        c.set_synchronous(False)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            run(og)
        c.set_stream(None)
        c.set_synchronous(True)
        prev = None
        for i in range(3):
            Ab.mul_(-0.5).add_(0.25 * (i + 1))
            At.mul_(1.5).add_(-0.125)
            da.mul_(0.75)
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                g.replay()
            torch.cuda.synchronize()
            got = fetch(og)
            run(oe)
            ref = fetch(oe)
            for key in shapes:
                assert np.array_equal(got[key].view(np.uint8), ref[key].view(np.uint8)), f"replay {i}: {key}"
            if prev is not None:
                for key in ("gb", "gt", "dot"):
                    assert not np.array_equal(got[key], prev[key]), f"replay {i}: {key} unchanged"
            prev = got
    finally:
        c.close()


def test_graph_survives_workspace_growth(plugin):
    """A graph captured with the context's workspace keeps replaying correctly after an
    eager call on the same context grows the workspace: the old block is retired, not
    freed.  A call inside capture that would need a larger workspace is refused with
    NOT_SUPPORTED (hipMalloc is not allowed there) and launches nothing."""
    import torch
    c = plugin.create_context(0)
    try:
        r = rng(4444)
        m, n, k = 100, 256, 512                       # large-m int4 GEMM: small workspace
        _, Wl, sl = int4_weights(r, n, k, 32)
        xl = torch.tensor(r.standard_normal((m, k)), dtype=torch.bfloat16, device="cuda")
        wl, s_l, xlb = c.upload(Wl), c.upload(sl), c.wrap(xl)
        d = W.qdesc(n, k, m, 4, 32, 0, W.SCALE_F16, W.BF16, W.BF16)
        og, oe = c.alloc(m * n * 2), c.alloc(m * n * 2)
        c.qmatmul(d, wl, s_l, xlb, None, og)          # sizes the workspace eagerly
        s = torch.cuda.Stream()
        c.set_stream(s.cuda_stream)
        c.set_synchronous(False)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            c.qmatmul(d, wl, s_l, xlb, None, og)
        c.set_stream(None)
        c.set_synchronous(True)

        # an eager call with a much larger activation block grows the workspace
        M2, K2 = 2048, 4096
        _, W2, s2 = int4_weights(r, 256, K2, 32)
        x2 = torch.tensor(r.standard_normal((M2, K2)), dtype=torch.bfloat16, device="cuda")
        d2 = W.qdesc(256, K2, M2, 4, 32, 0, W.SCALE_F16, W.BF16, W.BF16)
        w2, sb2, x2b, y2 = c.upload(W2), c.upload(s2), c.wrap(x2), c.alloc(M2 * 256 * 2)
        c.qmatmul(d2, w2, sb2, x2b, None, y2)
        junk = torch.full((64 << 20,), 7, dtype=torch.uint8, device="cuda")  # reuse bait
        torch.cuda.synchronize()

        for i in range(3):
            xl.copy_(torch.tensor(r.standard_normal((m, k)), dtype=torch.bfloat16))
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                g.replay()
            torch.cuda.synchronize()
            c.qmatmul(d, wl, s_l, xlb, None, oe)
            got = c.download(og, np.uint16, (m, n))
            ref = c.download(oe, np.uint16, (m, n))
            assert np.array_equal(got, ref), f"replay {i} after workspace growth"

        # growth inside capture: refused, nothing launched
        M3 = 4096
        x3 = torch.zeros((M3, K2), dtype=torch.bfloat16, device="cuda")
        x3b, y3 = c.wrap(x3), c.alloc(M3 * 256 * 2)
        d3 = W.qdesc(256, K2, M3, 4, 32, 0, W.SCALE_F16, W.BF16, W.BF16)
        c.set_stream(s.cuda_stream)
        c.set_synchronous(False)
        g3 = torch.cuda.CUDAGraph()
        err = None
        with torch.cuda.graph(g3, stream=s):
            c.qmatmul(d, wl, s_l, xlb, None, og)      # fits: captured
            try:
                c.qmatmul(d3, w2, sb2, x3b, None, y3)
            except W.LuxError as e:
                err = e
        c.set_stream(None)
        c.set_synchronous(True)
        assert err is not None and err.code == W.LUX_BACKEND_ERROR_NOT_SUPPORTED, err
        del junk
    finally:
        c.close()
