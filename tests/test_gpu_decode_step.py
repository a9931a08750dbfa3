"""GPU parity: the ABI-v3 tensor slots around the matmul path (op_add/sub/mul/div_f32),
rms_norm, and one decode step of a gated FFN run end to end through the plugin.

Oracle: the elementwise ops are single IEEE fp32 operations (compared bit-for-bit with
numpy); rms_norm.wgsl and the FFN composition use oracle/lux_oracle.c (tolerance of the fp
paths).  The decode step is rms_norm -> int4 gate/up GEMM with the SILU_MUL epilogue ->
int4 down GEMV -> residual op_add_f32, i.e. the quantized path with its neighbours.
"""
import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import bf16_bits, bf16_to_f32, compare, int4_weights, rng, round_to

pytestmark = pytest.mark.gpu

NP = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide}


@pytest.mark.parametrize("n", [0, 1, 3, 4, 1027, 1 << 22])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_binary_slots_bit_exact(ctx, op, n):
    r = rng(n + len(op))
    a = r.standard_normal(n).astype(np.float32)
    b = r.standard_normal(n).astype(np.float32)
    if op == "div":
        b[np.abs(b) < 1e-3] = 0.5
    ab, bb, ob = ctx.upload(a), ctx.upload(b), ctx.alloc(max(4 * n, 4))
    ctx.binary_f32(op, ab, bb, ob, n)
    got = ctx.download(ob, np.float32, (n,))
    assert np.array_equal(got.view(np.uint32), NP[op](a, b).astype(np.float32).view(np.uint32))


def test_binary_slot_unaligned_and_in_place(ctx):
    """Buffers wrapped at a 4-byte offset take the scalar kernel; out may alias an input."""
    r = rng(77)
    a = r.standard_normal(4097).astype(np.float32)
    b = r.standard_normal(4097).astype(np.float32)
    big_a, big_b = ctx.upload(np.concatenate([[0.0], a]).astype(np.float32)), ctx.upload(np.concatenate([[0.0], b]).astype(np.float32))
    wa = ctx.plugin.lib.lux_hip_buffer_wrap(ctx.handle, big_a.ptr + 4, 4097 * 4)
    wb = ctx.plugin.lib.lux_hip_buffer_wrap(ctx.handle, big_b.ptr + 4, 4097 * 4)
    A, Bb = W.Buffer(ctx, wa, 4097 * 4), W.Buffer(ctx, wb, 4097 * 4)
    ctx.binary_f32("mul", A, Bb, A, 4097)
    got = ctx.download(big_a, np.float32, (4098,))[1:]
    assert np.array_equal(got, (a * b).astype(np.float32))
    with pytest.raises(W.LuxError):  # n beyond the buffers
        ctx.binary_f32("add", A, Bb, A, 5000)


@pytest.mark.parametrize("rows,hidden,xdt,ydt", [(1, 4096, "f32", "f16"), (64, 4096, "bf16", "f32"),
                                                 (3, 8192, "f32", "f32"), (5, 1000, "f16", "bf16")])
def test_rms_norm_matches_oracle(ctx, rows, hidden, xdt, ydt):
    r = rng(rows * hidden)
    x = (r.standard_normal((rows, hidden)) * 3).astype(np.float32)
    g = r.uniform(0.5, 1.5, hidden).astype(np.float32)
    codes = {"f32": W.F32, "f16": W.F16, "bf16": W.BF16}
    if xdt == "f16":
        xin = x.astype(np.float16)
        xf = xin.astype(np.float32)
    elif xdt == "bf16":
        xin = bf16_bits(x)
        xf = bf16_to_f32(xin)
    else:
        xin, xf = x, x
    ynp = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16}[ydt]
    xb, gb = ctx.upload(xin), ctx.upload(g)
    yb, rb = ctx.alloc(rows * hidden * np.dtype(ynp).itemsize), ctx.alloc(rows * 4)
    ctx.rms_norm(xb, gb, yb, rows, hidden, 1e-6, codes[xdt], codes[ydt], rb)
    got = ctx.download(yb, ynp, (rows, hidden))
    got = bf16_to_f32(got) if ydt == "bf16" else got.astype(np.float32)
    ref, rref = oracle.rms_norm(xf, g, 1e-6)
    compare(got.astype(np.float64), round_to(ref, ydt), f"rms_norm {xdt}->{ydt}")
    np.testing.assert_allclose(ctx.download(rb, np.float32, (rows,)), rref, rtol=1e-5)


def test_decode_step_end_to_end(ctx):
    """x <- x + W_down . (silu(W_gate . n) * (W_up . n)), n = rms_norm(x) * gamma, with int4
    g32 weights, fp16 activations between the ops and an fp32 residual stream."""
    r = rng(2024)
    hidden, inter, gs = 4096, 2048, 32
    x = r.standard_normal((1, hidden)).astype(np.float32)
    gamma = r.uniform(0.8, 1.2, hidden).astype(np.float32)
    _, Wgu, sgu = int4_weights(r, 2 * inter, hidden, gs)       # rows: gate then up
    _, Wd, sd = int4_weights(r, hidden, inter, gs)
    xb, gb = ctx.upload(x), ctx.upload(gamma)
    nb = ctx.alloc(hidden * 2)
    hb = ctx.alloc(inter * 2)
    db = ctx.alloc(hidden * 4)
    outb = ctx.alloc(hidden * 4)
    ctx.rms_norm(xb, gb, nb, 1, hidden, 1e-6, W.F32, W.F16)
    ctx.qmatmul_ex(W.qdesc(2 * inter, hidden, 1, 4, gs, 0, W.SCALE_F16, W.F16, W.F16),
                   ctx.upload(Wgu), ctx.upload(sgu), nb, None, W.EPI_SILU_MUL, None, None, hb)
    ctx.qmatmul(W.qdesc(hidden, inter, 1, 4, gs, 0, W.SCALE_F16, W.F16, W.F32),
                ctx.upload(Wd), ctx.upload(sd), hb, None, db)
    ctx.binary_f32("add", xb, db, outb, hidden)
    got = ctx.download(outb, np.float32, (1, hidden)).astype(np.float64)
    # oracle composition, rounding to fp16 where the plugin stores fp16
    n, _ = oracle.rms_norm(x, gamma, 1e-6)
    n16 = n.astype(np.float16).astype(np.float32)
    gu = oracle.qmatmul_f64(Wgu, sgu.astype(np.float32), n16, gs, 4).astype(np.float32)
    h16 = oracle.silu_mul(gu).astype(np.float16).astype(np.float32)
    d = oracle.qmatmul_f64(Wd, sd.astype(np.float32), h16, gs, 4).astype(np.float32)
    ref = (x + d).astype(np.float64)
    compare(got, ref, "decode step")
    # the FFN branch on its own (the residual would hide errors in it)
    compare(ctx.download(db, np.float32, (1, hidden)).astype(np.float64), d.astype(np.float64),
            "decode step FFN branch")
