"""GPU parity: output epilogues fused into the quantized matmul stores
(lux_hip_qmatmul_ex).

Oracle: the fp64 ground truth of the matmul (oracle.qmatmul_f64), rounded to fp32, then
apply_epilogue / the silu_mul output stage of steel_gemm_fused.wgsl:80-127,452-558 as
restated in oracle/lux_oracle.c, then rounded to the output dtype.  Tolerance of the fp
paths (rel-L2 <= 1e-3, max-abs <= 1e-2 * ||ref||_inf, tests/util.py).  Each kernel family
is covered: the int4 GEMV (m = 1), the small-m kernel (int8 per-row and int4 group
weights, one and two 64-token passes) and the large-m int4 MFMA GEMM.
"""
import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import bf16_bits, bf16_to_f32, compare, int4_weights, int8_weights, rng, round_to

pytestmark = pytest.mark.gpu

YNP = {"f16": (W.F16, np.float16), "f32": (W.F32, np.float32), "bf16": (W.BF16, np.uint16)}


def _case(ctx, r, wbits, n_out, K, m, gs, xdt, ydt, epi):
    """Run one epilogue through the plugin; return (got, ref) as float64 [m, N]."""
    if wbits == 4:
        _, Wp, s = int4_weights(r, n_out, K, gs)
        sflat = s.astype(np.float32)
    else:
        Wp, s = int8_weights(r, n_out, K)
        gs = K
        sflat = s.astype(np.float32).reshape(n_out, 1)
    xf = r.standard_normal((m, K)).astype(np.float32)
    if xdt == "bf16":
        xin = bf16_bits(xf)
        xf = bf16_to_f32(xin)
        xcode = W.BF16
    else:
        xin = xf.astype(np.float16)
        xf = xin.astype(np.float32)
        xcode = W.F16
    ny = n_out // 2 if epi == W.EPI_SILU_MUL else n_out
    ycode, ynp = YNP[ydt]
    y0 = oracle.qmatmul_f64(Wp, sflat, xf, gs, wbits).astype(np.float32)  # [m, n_out]
    bias = r.standard_normal(ny).astype(np.float32)
    resid = r.standard_normal((m, ny)).astype(np.float32)
    if epi == W.EPI_SILU_MUL:
        ref = oracle.silu_mul(y0)
    else:
        ref = oracle.apply_epilogue(y0, epi, bias=bias, residual=resid)
    d = W.qdesc(n_out, K, m, wbits, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, xcode, ycode)
    wb, sb, xb = ctx.upload(Wp), ctx.upload(s), ctx.upload(xin)
    yb = ctx.alloc(m * ny * np.dtype(ynp).itemsize)
    bb = ctx.upload(bias) if epi == W.EPI_ADD_BIAS else None
    rb = ctx.upload(resid) if epi == W.EPI_ADD_RESIDUAL else None
    ctx.qmatmul_ex(d, wb, sb, xb, None, epi, bb, rb, yb)
    got = ctx.download(yb, ynp, (m, ny))
    got = bf16_to_f32(got) if ydt == "bf16" else got.astype(np.float32)
    return got.astype(np.float64), round_to(ref, ydt)


ALL = [W.EPI_RELU, W.EPI_GELU, W.EPI_SILU, W.EPI_TANH, W.EPI_SIGMOID, W.EPI_ADD_BIAS,
       W.EPI_ADD_RESIDUAL, W.EPI_SILU_MUL]


@pytest.mark.parametrize("epi", ALL)
def test_epilogue_int4_gemv(ctx, epi):
    """m = 1: the GEMV kernel (SILU_MUL reads the gate and up rows as interleaved pairs)."""
    got, ref = _case(ctx, rng(100 + epi), 4, 1024, 4096, 1, 32, "f16", "f16", epi)
    compare(got, ref, f"GEMV epilogue {epi}")


@pytest.mark.parametrize("wbits,m,xdt,epi", [
    (8, 8, "f16", W.EPI_GELU), (8, 8, "f16", W.EPI_ADD_RESIDUAL), (8, 32, "f16", W.EPI_SILU_MUL),
    (4, 20, "bf16", W.EPI_SILU), (4, 20, "bf16", W.EPI_ADD_BIAS), (4, 20, "bf16", W.EPI_SILU_MUL),
    (4, 70, "f16", W.EPI_ADD_RESIDUAL), (8, 70, "bf16", W.EPI_SILU_MUL)])
def test_epilogue_small_m(ctx, wbits, m, xdt, epi):
    """m <= 64 per pass: the small-m kernel; m = 70 runs two passes (the residual and the
    output advance with the pass)."""
    got, ref = _case(ctx, rng(200 + 7 * m + epi), wbits, 768, 2048, m, 128, xdt, "f16", epi)
    compare(got, ref, f"small-m epilogue w{wbits} m{m} {epi}")


@pytest.mark.parametrize("epi,ydt", [(W.EPI_RELU, "f32"), (W.EPI_ADD_BIAS, "bf16"),
                                     (W.EPI_ADD_RESIDUAL, "f32"), (W.EPI_TANH, "f32"),
                                     (W.EPI_SILU_MUL, "f32"), (W.EPI_SILU_MUL, "bf16")])
def test_epilogue_large_m(ctx, epi, ydt):
    """m > 64: the int4 MFMA GEMM; n_out = 1280 gives SILU_MUL 640 outputs, not a multiple
    of its 128-wide gate tiles, and m = 300 a partial 256-row tile."""
    got, ref = _case(ctx, rng(300 + epi), 4, 1280, 2048, 300, 32, "bf16", ydt, epi)
    compare(got, ref, f"large-m epilogue {epi} {ydt}")


def test_epilogue_rejects(ctx):
    r = rng(9)
    _, Wp, s = int4_weights(r, 64, 256, 32)
    x = r.standard_normal((4, 256)).astype(np.float16)
    wb, sb, xb, yb = ctx.upload(Wp), ctx.upload(s), ctx.upload(x), ctx.alloc(4 * 64 * 2)
    d = W.qdesc(64, 256, 4, 4, 32, 0, W.SCALE_F16, W.F16, W.F16)
    with pytest.raises(W.LuxError):  # bias missing
        ctx.qmatmul_ex(d, wb, sb, xb, None, W.EPI_ADD_BIAS, None, None, yb)
    with pytest.raises(W.LuxError):  # residual too small
        ctx.qmatmul_ex(d, wb, sb, xb, None, W.EPI_ADD_RESIDUAL, None, ctx.alloc(16), yb)
    with pytest.raises(W.LuxError):  # unknown epilogue
        ctx.qmatmul_ex(d, wb, sb, xb, None, 9, None, None, yb)
    d3 = W.qdesc(63, 256, 4, 4, 32, 0, W.SCALE_F16, W.F16, W.F16)
    with pytest.raises(W.LuxError):  # SILU_MUL needs gate and up rows in pairs
        ctx.qmatmul_ex(d3, wb, sb, xb, None, W.EPI_SILU_MUL, None, None, yb)


@pytest.mark.parametrize("epi,ydt", [(W.EPI_SILU_MUL, "f32"), (W.EPI_ADD_RESIDUAL, "f32"),
                                     (W.EPI_GELU, "f16")])
def test_epilogue_large_m_config4_shape(ctx, epi, ydt):
    """m = 2048 against 14336 weight rows (7168 SILU_MUL outputs), the grid of config 4
    (8 x 56 tiles of 256 x 256); K is cut to 256 to keep the oracle quick.  SILU_MUL is
    checked in f32: in bf16 the output rounding of two compounded operands alone reaches
    ~1e-3 rel-L2 against the rounded oracle."""
    got, ref = _case(ctx, rng(400 + epi), 4, 14336, 256, 2048, 32, "bf16", ydt, epi)
    compare(got, ref, f"config-4-shape epilogue {epi} {ydt}")


@pytest.mark.parametrize("n_out,K,gs,coding,sfmt,xdt", [
    (666, 512, 32, W.NIBBLE_TWOS_COMPLEMENT, W.SCALE_F32, "f16"),  # 333 pairs, xor-decoded nibbles
    (2 * 14336, 4096, 32, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, "f16"),  # 8 rows (4 pairs) per wave
    (512, 1024, 128, W.NIBBLE_OFFSET_BINARY, W.SCALE_GROUPSCALE, "f16"),
    (512, 1024, 32, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, "bf16"),  # no fast GEMV: small-m kernel
])
def test_silu_mul_gemv_pairs(ctx, n_out, K, gs, coding, sfmt, xdt):
    """SILU_MUL at m = 1 across codings, scale formats and pair counts, against
    silu_mul of the fp64 matmul (steel_gemm_fused.wgsl:452-558)."""
    r = rng(n_out + K + gs)
    _, Wp, s16 = int4_weights(r, n_out, K, gs, coding)
    sf = s16.astype(np.float32)
    if sfmt == W.SCALE_F16:
        sbuf = s16
    elif sfmt == W.SCALE_F32:
        sbuf = sf
    else:
        sbuf = np.zeros(sf.shape + (4,), np.float32)
        sbuf[..., 0] = sf
    xf = r.standard_normal((1, K)).astype(np.float32)
    if xdt == "bf16":
        xin = bf16_bits(xf)
        xf = bf16_to_f32(xin)
    else:
        xin = xf.astype(np.float16)
        xf = xin.astype(np.float32)
    w_ob = Wp if coding == W.NIBBLE_OFFSET_BINARY else Wp ^ np.uint32(0x88888888)
    ref = oracle.silu_mul(oracle.qmatmul_f64(w_ob, sf, xf, gs, 4).astype(np.float32))
    d = W.qdesc(n_out, K, 1, 4, gs, coding, sfmt, W.BF16 if xdt == "bf16" else W.F16, W.F32)
    yb = ctx.alloc(n_out // 2 * 4)
    ctx.qmatmul_ex(d, ctx.upload(Wp), ctx.upload(sbuf), ctx.upload(xin), None, W.EPI_SILU_MUL, None, None, yb)
    compare(ctx.download(yb, np.float32, (1, n_out // 2)).astype(np.float64), ref, f"SILU_MUL GEMV {n_out}x{K}")
