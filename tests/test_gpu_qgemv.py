"""GPU parity: int4 weight-only GEMV (m == 1) through lux_hip_qmatmul.

Oracle: matmul_nax_grouped with N == 1 (quantized_nax.wgsl:568-626), restated in
oracle/lux_oracle.c.  Config 2 of BASELINE.json (W 14336 x 4096, g32, fp16 scales,
fp16 x, fp16 y) is checked at full size against the oracle rounded to fp16, and
ragged shapes cover the other kernel paths.
"""
import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import compare, int4_weights, rng, round_to

pytestmark = pytest.mark.gpu

YD = {"f16": (W.F16, np.float16), "f32": (W.F32, np.float32), "bf16": (W.BF16, np.uint16)}


def _run_gemv(ctx, Wp, s, x, n_out, K, gs, coding=0, scale_fmt=W.SCALE_F16, x_dtype=W.F16,
              y="f16"):
    ycode, ynp = YD[y]
    d = W.qdesc(n_out, K, 1, 4, gs, coding, scale_fmt, x_dtype, ycode)
    wb, sb, xb, yb = ctx.upload(Wp), ctx.upload(s), ctx.upload(x), ctx.alloc(n_out * np.dtype(ynp).itemsize)
    ctx.qmatmul(d, wb, sb, xb, None, yb)
    out = ctx.download(yb, ynp, n_out)
    if y == "bf16":
        out = (out.astype(np.uint32) << 16).view(np.float32)
    return out.astype(np.float64)


def _oracle(Wp, s_f32, x_f32, gs, coding=0):
    return oracle.matmul_nax_grouped(Wp, s_f32.reshape(-1), x_f32.reshape(-1, 1), gs, coding)[:, 0]


def test_config2_full(ctx):
    """C2: W 14336 x 4096 int4 g32 (offset-binary), fp16 scales U(0.005, 0.02), x fp16 N(0,1)."""
    r = rng(2)
    n_out, K, gs = 14336, 4096, 32
    q, Wp, s = int4_weights(r, n_out, K, gs)
    x = r.standard_normal(K).astype(np.float16)
    got = _run_gemv(ctx, Wp, s, x, n_out, K, gs)
    ref = _oracle(Wp, s.astype(np.float32), x.astype(np.float32), gs)
    st = compare(got, round_to(ref, "f16"), "C2 full")
    print(f"C2 rel-L2 {st['rel_l2']:.2e} max-abs {st['max_abs']:.2e}")


@pytest.mark.parametrize("n_out,K,gs", [(17, 32, 32), (64, 2080, 32), (33, 8192, 128),
                                        (8, 256, 64), (100, 14336, 32), (5, 4096, 4096)])
def test_int4_gemv_shapes(ctx, n_out, K, gs):
    r = rng(n_out * 31 + K)
    q, Wp, s = int4_weights(r, n_out, K, gs)
    x = r.standard_normal(K).astype(np.float16)
    got = _run_gemv(ctx, Wp, s, x, n_out, K, gs, y="f32")
    ref = _oracle(Wp, s.astype(np.float32), x.astype(np.float32), gs)
    compare(got, ref, f"gemv {n_out}x{K} g{gs}", rel_tol=1e-5, abs_frac=1e-5)


@pytest.mark.parametrize("n_out,K,gs,coding,y", [
    (4096, 14336, 32, 0, "f32"),     # the decode down-projection: quarters of 112 slices
    (4099, 8192, 64, 1, "f16"),      # halves; ragged last block: waves without rows run to the barrier
    (300, 4096, 32, 0, "bf16"),      # halves of one slice per lane
    (2048, 16384, 128, 1, "f32"),    # the largest k: quarters of two full slices per lane
    (1000, 4160, 32, 0, "f32"),      # halves of 65 slices: the second pass of each half ragged
    (1000, 8320, 32, 1, "f32"),      # quarters of 65 slices: the second pass of each quarter ragged
    (4099, 12288, 64, 0, "f16"),     # quarters, ragged last block
    (700, 8256, 32, 0, "f32")])      # k > 8192 but not a multiple of 128: halves of 129 slices
def test_int4_gemv_k_parts(ctx, n_out, K, gs, coding, y):
    """Few, long rows: two or four waves per row, one per part of k, their sums added in LDS."""
    r = rng(n_out + K + coding)
    q, Wp, s = int4_weights(r, n_out, K, gs, coding)
    x = r.standard_normal(K).astype(np.float16)
    got = _run_gemv(ctx, Wp, s, x, n_out, K, gs, coding=coding, y=y)
    ref = _oracle(Wp, s.astype(np.float32), x.astype(np.float32), gs, coding)
    if y == "f32":
        compare(got, ref, f"gemv k parts {n_out}x{K} g{gs}", rel_tol=1e-5, abs_frac=1e-5)
    else:
        compare(got, round_to(ref, y), f"gemv k parts {n_out}x{K} g{gs} {y}")


@pytest.mark.parametrize("scale_fmt", [W.SCALE_F32, W.SCALE_GROUPSCALE])
@pytest.mark.parametrize("coding", [0, 1])
def test_int4_gemv_formats(ctx, scale_fmt, coding):
    r = rng(10 + coding + scale_fmt)
    n_out, K, gs = 96, 1024, 32
    q, Wp, s16 = int4_weights(r, n_out, K, gs, coding)
    s32 = r.uniform(0.005, 0.02, size=s16.shape).astype(np.float32)
    if scale_fmt == W.SCALE_F32:
        sbuf = s32
    else:  # GroupScale {scale, zero_point, min, max}
        gsr = np.zeros(s32.shape + (4,), np.float32)
        gsr[..., 0] = s32
        gsr[..., 2] = -1.0
        gsr[..., 3] = 1.0
        sbuf = gsr
    x = r.standard_normal(K).astype(np.float16)
    got = _run_gemv(ctx, Wp, sbuf, x, n_out, K, gs, coding, scale_fmt, y="f32")
    ref = _oracle(Wp, s32, x.astype(np.float32), gs, coding)
    compare(got, ref, "formats", rel_tol=1e-5, abs_frac=1e-5)


@pytest.mark.parametrize("xd", ["f32", "bf16"])
@pytest.mark.parametrize("gs", [8, 32])
def test_int4_gemv_generic_x(ctx, xd, gs):
    r = rng(77 + gs)
    n_out, K = 70, 512
    q, Wp, s = int4_weights(r, n_out, K, gs)
    xf = r.standard_normal(K).astype(np.float32)
    if xd == "bf16":
        from util import bf16_bits, bf16_to_f32
        xb = bf16_bits(xf)
        xf = bf16_to_f32(xb)
        xin, xcode = xb, W.BF16
    else:
        xin, xcode = xf, W.F32
    got = _run_gemv(ctx, Wp, s, xin, n_out, K, gs, x_dtype=xcode, y="bf16")
    ref = _oracle(Wp, s.astype(np.float32), xf, gs)
    compare(got, round_to(ref, "bf16"), f"generic x={xd} g{gs}")


def test_int4_gemv_rejects(ctx):
    r = rng(3)
    q, Wp, s = int4_weights(r, 16, 64, 32)
    x = r.standard_normal(64).astype(np.float16)
    wb, sb, xb, yb = ctx.upload(Wp), ctx.upload(s), ctx.upload(x), ctx.alloc(16 * 2)
    with pytest.raises(W.LuxError) as e:  # scale buffer too small for g16
        ctx.qmatmul(W.qdesc(16, 64, 1, 4, 16), wb, sb, xb, None, yb)
    assert e.value.code == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    with pytest.raises(W.LuxError) as e:  # k not a multiple of 32
        ctx.qmatmul(W.qdesc(16, 40, 1, 4, 8), wb, sb, xb, None, yb)
    assert e.value.code == W.LUX_BACKEND_ERROR_NOT_SUPPORTED
    with pytest.raises(W.LuxError) as e:  # output too small
        ctx.qmatmul(W.qdesc(16, 64, 1, 4, 32, y_dtype=W.F32), wb, sb, xb, None, yb)
    assert e.value.code == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
