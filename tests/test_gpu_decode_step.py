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
    # the same step in two launches (bench.py's form): rms_norm inside the gate/up GEMV,
    # the residual in the down GEMV's epilogue; the same bits as the four calls
    hb2, outb2 = ctx.alloc(inter * 2), ctx.alloc(hidden * 4)
    ctx.rms_norm_qmatmul(xb, gb, 1e-6, W.F32, W.qdesc(2 * inter, hidden, 1, 4, gs, 0, W.SCALE_F16, W.F16, W.F16),
                         ctx.upload(Wgu), ctx.upload(sgu), W.EPI_SILU_MUL, None, None, hb2)
    ctx.qmatmul_ex(W.qdesc(hidden, inter, 1, 4, gs, 0, W.SCALE_F16, W.F16, W.F32),
                   ctx.upload(Wd), ctx.upload(sd), hb2, None, W.EPI_ADD_RESIDUAL, None, xb, outb2)
    assert np.array_equal(ctx.download(outb2, np.float32, (1, hidden)).view(np.uint32),
                          got.astype(np.float32).view(np.uint32))
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


# ---- lux_hip_rms_norm_qmatmul: rms_norm fused ahead of the quantized matmul -------------
CODES = {"f32": W.F32, "f16": W.F16, "bf16": W.BF16}
YNP = {W.F32: np.float32, W.F16: np.float16, W.BF16: np.uint16}


def _norm_input(r, m, k, xdt):
    x = (r.standard_normal((m, k)) * 2).astype(np.float32)
    if xdt == "f16":
        return x.astype(np.float16)
    if xdt == "bf16":
        return bf16_bits(x)
    return x


def _fused_vs_two_calls(ctx, r, desc, xin, xdt, wp, s, epi, ydt):
    """Run lux_hip_rms_norm_qmatmul and lux_hip_rms_norm + lux_hip_qmatmul_ex on the same
    inputs; return both outputs as raw bits (they must be identical) and the normalised row."""
    m, k, n_out = desc.m, desc.k, desc.n_out
    ny = n_out // 2 if epi == W.EPI_SILU_MUL else n_out
    gamma = r.uniform(0.5, 1.5, k).astype(np.float32)
    bias = r.standard_normal(ny).astype(np.float32)
    resid = r.standard_normal((m, ny)).astype(np.float32)
    xb, gb, wb = ctx.upload(xin), ctx.upload(gamma), ctx.upload(wp)
    sb = ctx.upload(s) if s is not None else None
    bb = ctx.upload(bias) if epi == W.EPI_ADD_BIAS else None
    rb = ctx.upload(resid) if epi == W.EPI_ADD_RESIDUAL else None
    ynp = YNP[ydt]
    y1, y2 = ctx.alloc(m * ny * np.dtype(ynp).itemsize), ctx.alloc(m * ny * np.dtype(ynp).itemsize)
    nb = ctx.alloc(m * k * np.dtype(YNP[desc.x_dtype]).itemsize)
    ctx.rms_norm_qmatmul(xb, gb, 1e-6, CODES[xdt], desc, wb, sb, epi, bb, rb, y1)
    ctx.rms_norm(xb, gb, nb, m, k, 1e-6, CODES[xdt], desc.x_dtype)
    ctx.qmatmul_ex(desc, wb, sb, nb, None, epi, bb, rb, y2)
    got1 = ctx.download(y1, ynp, (m, ny))
    got2 = ctx.download(y2, ynp, (m, ny))
    return got1, got2, gamma


@pytest.mark.parametrize("k,xdt,epi,ydt,coding", [
    (4096, "f32", W.EPI_SILU_MUL, W.F16, 0),      # the decode FFN's gate/up call
    (4096, "f16", W.EPI_NONE, W.F32, 0),
    (4096, "bf16", W.EPI_ADD_BIAS, W.BF16, 1),
    (2048, "f32", W.EPI_ADD_RESIDUAL, W.F32, 0),  # one slice per lane
    (8192, "f32", W.EPI_SILU_MUL, W.F16, 1),      # four slices per lane: the largest fused k
    (4128, "f16", W.EPI_NONE, W.F16, 0),          # k not a multiple of 256: ragged last pass
    (96, "f32", W.EPI_NONE, W.F32, 0)])           # fewer elements than threads
def test_rms_norm_qmatmul_fused_gemv_bit_identical(ctx, k, xdt, epi, ydt, coding):
    """m = 1, int4, fp16 scales, fp16 activations: the GEMV normalises the row in its prologue
    (4160 rows: more than 16 per CU, so whole rows per wave). The output must equal rms_norm
    followed by qmatmul_ex bit for bit, and the oracle."""
    r = rng(k * 7 + len(xdt) + epi)
    n_out, gs = 4160, 32
    _, Wp, s = int4_weights(r, n_out, k, gs, coding)
    xin = _norm_input(r, 1, k, xdt)
    desc = W.qdesc(n_out, k, 1, 4, gs, coding, W.SCALE_F16, W.F16, ydt)
    got1, got2, gamma = _fused_vs_two_calls(ctx, r, desc, xin, xdt, Wp, s, epi, ydt)
    assert np.array_equal(got1.view(np.uint8), got2.view(np.uint8))
    if epi == W.EPI_NONE:  # and the oracle on the plain GEMV
        xf = xin.astype(np.float32) if xdt != "bf16" else bf16_to_f32(xin)
        n, _ = oracle.rms_norm(xf, gamma, 1e-6)
        n16 = n.astype(np.float16).astype(np.float32)
        ref = oracle.qmatmul_f64(Wp, s.astype(np.float32), n16, gs, 4)
        got = bf16_to_f32(got1) if ydt == W.BF16 else got1.astype(np.float32)
        yname = {W.F32: "f32", W.F16: "f16", W.BF16: "bf16"}[ydt]
        compare(got.astype(np.float64), round_to(ref.astype(np.float32), yname), f"rms_norm_qmatmul k{k}")


@pytest.mark.parametrize("case", ["small_m", "k16384", "k_halves", "scale_f32", "x_f32", "w8", "w4a8_qx"])
def test_rms_norm_qmatmul_two_launch_routes(ctx, case):
    """Descriptors outside the fused GEMV run rms_norm into the workspace, then the matmul:
    still bit-identical to the two separate calls."""
    r = rng(len(case) * 31)
    m, n_out, k, bits, gs, sf, xdt, ydt, flags, epi = 1, 512, 4096, 4, 32, W.SCALE_F16, W.F16, W.F16, 0, W.EPI_NONE
    if case == "small_m":
        m, epi = 5, W.EPI_SILU_MUL
    elif case == "k16384":  # outside the fused GEMV; the plain GEMV splits k in quarters
        k = 16384
    elif case == "k_halves":  # few long rows: the plain GEMV splits k, so both kernels run
        k = 8192
    elif case == "scale_f32":
        sf = W.SCALE_F32
    elif case == "x_f32":
        xdt, ydt = W.F32, W.F32
    elif case == "w8":
        bits, m, gs = 8, 3, k  # per-row int8 scales (config 3's format)
    elif case == "w4a8_qx":
        m, gs, flags, ydt, xdt = 33, 128, W.QFLAG_QUANTIZE_X, W.F32, W.F32
    if bits == 4:
        _, Wp, s = int4_weights(r, n_out, k, gs)
    else:
        q = r.integers(-127, 128, size=(n_out, k)).astype(np.int8)
        Wp, s = q, r.uniform(0.001, 0.01, size=(n_out, k // gs)).astype(np.float16)
    if sf == W.SCALE_F32:
        s = s.astype(np.float32)
    desc = W.qdesc(n_out, k, m, bits, gs, 0, sf, xdt, ydt)
    desc.flags = flags
    xin = _norm_input(r, m, k, "f32")
    got1, got2, _ = _fused_vs_two_calls(ctx, r, desc, xin, "f32", Wp, s, epi, ydt)
    assert np.array_equal(got1.view(np.uint8), got2.view(np.uint8))


def test_rms_norm_qmatmul_rejects(ctx):
    r = rng(5)
    k, n_out = 256, 64
    _, Wp, s = int4_weights(r, n_out, k, 32)
    xb, gb, wb, sb = ctx.upload(np.ones(k, np.float32)), ctx.upload(np.ones(k, np.float32)), ctx.upload(Wp), ctx.upload(s)
    yb = ctx.alloc(n_out * 2)
    d = W.qdesc(n_out, k, 1, 4, 32, 0, W.SCALE_F16, W.F16, W.F16)
    lib = ctx.plugin.lib

    def call(p, desc, gamma=gb):
        return lib.lux_hip_rms_norm_qmatmul(ctx.handle, W.byref(p), gamma.handle, W.byref(desc), wb.handle,
                                            sb.handle, xb.handle, W.EPI_NONE, None, None, yb.handle)
    assert call(W.RmsNormParams(1, k, 1e-6, W.F32, W.F16), d) == W.LUX_BACKEND_OK
    assert call(W.RmsNormParams(2, k, 1e-6, W.F32, W.F16), d) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT  # m
    assert call(W.RmsNormParams(1, k - 32, 1e-6, W.F32, W.F16), d) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT  # k
    assert call(W.RmsNormParams(1, k, 1e-6, W.F32, W.F32), d) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT  # y != x dtype
    assert call(W.RmsNormParams(1, k, 1e-6, W.I8, W.F16), d) == W.LUX_BACKEND_ERROR_NOT_SUPPORTED
    small = ctx.upload(np.ones(k // 2, np.float32))
    assert call(W.RmsNormParams(1, k, 1e-6, W.F32, W.F16), d, small) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
