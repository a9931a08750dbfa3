"""GPU parity: weight-only quantized GEMM (m > 1) through lux_hip_qmatmul.

Oracle: matmul_nax_grouped (quantized_nax.wgsl:568-626) and the int8
dequantize + matmul composition (quantized_nax.wgsl:364-386 +
src/webgpu_plugin.cpp:138-205), restated in oracle/lux_oracle.c and evaluated in
the reference layout (act = X^T, out = Y^T).  Tolerance for every fp path:
rel-L2 <= 1e-3 and max-abs <= 1e-2 * ||ref||_inf against the oracle rounded (RNE)
to the output dtype.
"""
import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import bf16_bits, bf16_to_f32, compare, int4_weights, int8_weights, rng, round_to

pytestmark = pytest.mark.gpu

YD = {"f16": (W.F16, np.float16), "f32": (W.F32, np.float32), "bf16": (W.BF16, np.uint16)}


def _run(ctx, desc, Wp, s, X, n_out, m, y):
    ycode, ynp = YD[y]
    wb, sb, xb = ctx.upload(Wp), ctx.upload(s), ctx.upload(X)
    yb = ctx.alloc(m * n_out * np.dtype(ynp).itemsize)
    ctx.qmatmul(desc, wb, sb, xb, None, yb)
    out = ctx.download(yb, ynp, (m, n_out))
    if y == "bf16":
        out = bf16_to_f32(out)
    return out.astype(np.float64)


def _x(r, m, K, xd):
    xf = r.standard_normal((m, K)).astype(np.float32)
    if xd == "bf16":
        b = bf16_bits(xf)
        return b, bf16_to_f32(b), W.BF16
    h = xf.astype(np.float16)
    return h, h.astype(np.float32), W.F16


def test_config4_full(ctx):
    """C4: X 2048 x 4096 bf16 N(0,1), W 14336 x 4096 int4 g32 fp16 scales, bf16 out."""
    r = rng(4)
    n_out, K, m, gs = 14336, 4096, 2048, 32
    q, Wp, s = int4_weights(r, n_out, K, gs)
    X, Xf, xc = _x(r, m, K, "bf16")
    d = W.qdesc(n_out, K, m, 4, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, xc, W.BF16)
    got = _run(ctx, d, Wp, s, X, n_out, m, "bf16")
    ref = oracle.matmul_nax_grouped_tokens(Wp, s.astype(np.float32).reshape(-1), Xf, gs)
    st = compare(got, round_to(ref, "bf16"), "C4 full")
    print(f"C4 rel-L2 {st['rel_l2']:.3e} max-abs/inf {st['max_abs'] / st['ref_inf']:.3e}")


@pytest.mark.parametrize("n_out,K,m,gs,xd,y", [
    (256, 64, 2, 32, "bf16", "f32"),
    (300, 128, 5, 32, "f16", "f32"),
    (520, 512, 33, 128, "bf16", "bf16"),
    (256, 1024, 300, 64, "f16", "f16"),
    (1000, 256, 257, 32, "bf16", "f32"),
])
def test_int4_gemm_shapes(ctx, n_out, K, m, gs, xd, y):
    r = rng(n_out + K + m)
    q, Wp, s = int4_weights(r, n_out, K, gs)
    X, Xf, xc = _x(r, m, K, xd)
    d = W.qdesc(n_out, K, m, 4, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, xc, YD[y][0])
    got = _run(ctx, d, Wp, s, X, n_out, m, y)
    ref = oracle.matmul_nax_grouped_tokens(Wp, s.astype(np.float32).reshape(-1), Xf, gs)
    compare(got, round_to(ref, y), f"gemm {n_out}x{K} m{m} g{gs} {xd}->{y}")


@pytest.mark.parametrize("scale_fmt", [W.SCALE_F32, W.SCALE_GROUPSCALE])
@pytest.mark.parametrize("coding", [0, 1])
def test_int4_gemm_formats(ctx, scale_fmt, coding):
    r = rng(40 + 2 * scale_fmt + coding)
    n_out, K, m, gs = 384, 256, 70, 32
    q, Wp, _ = int4_weights(r, n_out, K, gs, coding)
    s32 = r.uniform(0.005, 0.02, size=(n_out, K // gs)).astype(np.float32)
    if scale_fmt == W.SCALE_F32:
        sbuf = s32
    else:
        sbuf = np.zeros(s32.shape + (4,), np.float32)
        sbuf[..., 0] = s32
    X, Xf, xc = _x(r, m, K, "bf16")
    d = W.qdesc(n_out, K, m, 4, gs, coding, scale_fmt, xc, W.F32)
    got = _run(ctx, d, Wp, sbuf, X, n_out, m, "f32")
    ref = oracle.matmul_nax_grouped_tokens(Wp, s32.reshape(-1), Xf, gs, coding)
    compare(got, ref, f"formats {scale_fmt} {coding}")


def test_int4_gemm_exact_grid(ctx):
    """Power-of-two scales and small-integer activations: every staged value and
    product is exact, so the GPU result must equal the oracle bit-for-bit."""
    r = rng(9)
    n_out, K, m, gs = 512, 512, 64, 32
    q = r.integers(-8, 8, size=(n_out, K))
    from util import pack_nibbles
    Wp = pack_nibbles(q, 0)
    s = (2.0 ** r.integers(-6, 0, size=(n_out, K // gs))).astype(np.float16)
    Xf = r.integers(-4, 5, size=(m, K)).astype(np.float32)
    X = Xf.astype(np.float16)
    d = W.qdesc(n_out, K, m, 4, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, W.F16, W.F32)
    got = _run(ctx, d, Wp, s, X, n_out, m, "f32")
    ref = oracle.matmul_nax_grouped_tokens(Wp, s.astype(np.float32).reshape(-1), Xf, gs)
    assert np.array_equal(got, ref.astype(np.float64))


# --------------------------------------------------------------------------- small m
@pytest.mark.parametrize("m", [8, 32])
def test_config3_int8_per_row(ctx, m):
    """C3: W 28672 x 8192 int8 U[-127,127], per-row fp16 scales U(0.001,0.01),
    X m x 8192 fp16 N(0,1), fp16 out; oracle = dequantize_nax_int8_group (gs = K)
    followed by the sequential-k matmul."""
    r = rng(30 + m)
    n_out, K = 28672, 8192
    q, s = int8_weights(r, n_out, K)
    X = r.standard_normal((m, K)).astype(np.float16)
    d = W.qdesc(n_out, K, m, 8, K, 0, W.SCALE_F16, W.F16, W.F16)
    got = _run(ctx, d, q, s, X, n_out, m, "f16")
    ref = oracle.matmul_int8_dequant_tokens(q, s.astype(np.float32).reshape(-1),
                                            X.astype(np.float32), K)
    st = compare(got, round_to(ref, "f16"), f"C3 m={m}")
    print(f"C3 m={m} rel-L2 {st['rel_l2']:.3e}")


@pytest.mark.parametrize("n_out,K,m,gs,xd,y", [
    (100, 256, 1, 256, "f16", "f32"),
    (1000, 512, 5, 512, "bf16", "bf16"),
    (513, 1024, 64, 128, "f16", "f32"),
    (300, 512, 45, 64, "bf16", "f16"),   # group scales: a 32-token pass, then 13 tokens
    (256, 768, 70, 768, "f32", "f16"),
])
def test_int8_small_shapes(ctx, n_out, K, m, gs, xd, y):
    r = rng(n_out + 3 * K + m)
    q, _ = int8_weights(r, n_out, K)
    s = r.uniform(0.001, 0.01, size=(n_out, K // gs)).astype(np.float16)
    if xd == "f32":
        Xf = r.standard_normal((m, K)).astype(np.float32)
        X, xc = Xf, W.F32
    else:
        X, Xf, xc = _x(r, m, K, xd)
    d = W.qdesc(n_out, K, m, 8, gs, 0, W.SCALE_F16, xc, YD[y][0])
    got = _run(ctx, d, q, s, X, n_out, m, y)
    # f32 activations are staged as fp16 by this kernel (relative error <= 2^-11 per
    # activation); the comparison is still against the unrounded fp32 oracle.
    ref = oracle.matmul_int8_dequant_tokens(q, s.astype(np.float32).reshape(-1),
                                            Xf.astype(np.float32), gs)
    compare(got, round_to(ref, y), f"int8 small {n_out}x{K} m{m} g{gs}")


@pytest.mark.parametrize("n_out,K,m,gs", [(14336, 4096, 8, 32), (300, 512, 17, 128), (256, 256, 64, 32)])
def test_int4_small_m(ctx, n_out, K, m, gs):
    r = rng(n_out + K + 7 * m)
    q, Wp, s = int4_weights(r, n_out, K, gs)
    X, Xf, xc = _x(r, m, K, "f16")
    d = W.qdesc(n_out, K, m, 4, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, xc, W.F16)
    got = _run(ctx, d, Wp, s, X, n_out, m, "f16")
    ref = oracle.matmul_nax_grouped_tokens(Wp, s.astype(np.float32).reshape(-1), Xf, gs)
    compare(got, round_to(ref, "f16"), f"int4 small m {n_out}x{K} m{m}")


@pytest.mark.parametrize("m,xd", [(300, "bf16"), (8, "bf16"), (8, "f32"), (70, "f32")])
def test_int4_wide_range_activations(ctx, m, xd):
    """Rows far outside fp16's normal range (x 3e5 with one element at 3e6, and x 1e-7).
    bf16 / fp32 activations are staged as fp16 after dividing each row by a power of
    two, so every row keeps its precision; checked row by row."""
    r = rng(77 + m)
    n_out, K, gs = 512, 1024, 32
    q, Wp, s = int4_weights(r, n_out, K, gs)
    xf = r.standard_normal((m, K)).astype(np.float32)
    xf[0] *= 3e5
    xf[1] *= 1e-7
    xf[2, 5] = 3e6
    if xd == "bf16":
        X = bf16_bits(xf)
        Xf, xc = bf16_to_f32(X), W.BF16
    else:
        X, Xf, xc = xf, xf, W.F32
    d = W.qdesc(n_out, K, m, 4, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, xc, W.F32)
    got = _run(ctx, d, Wp, s, X, n_out, m, "f32")
    ref = oracle.matmul_nax_grouped_tokens(Wp, s.astype(np.float32).reshape(-1), Xf, gs)
    assert np.all(np.isfinite(got))
    for i in range(m):
        compare(got[i], ref[i].astype(np.float64), f"wide-range row {i} m{m} {xd}")


# ------------------------------------------------------------------ scale range
# The reference dequantizes f32(q) * scale in fp32 (quantized_nax.wgsl:589-608), and its
# producer (compute_group_scales, :157-232) writes fp32 scales of any magnitude.  The m > 1
# int4 kernels stage q * s as fp16 after dividing each weight row's scales by a power of
# two (the row's scale fold), so tiny, fp16-subnormal and huge scales must give the
# oracle's result.  m = 1 is the GEMV (fp32 scales), m = 8 / 64 the small-m MFMA kernel,
# m = 2048 the large-m MFMA kernel.
SCALE_RANGES = {"tiny": (1e-9, 1e-7), "f16sub": (2.0 ** -24, 2.0 ** -14), "huge": (1e4, 1e5)}


def _scale_buffer(s32, fmt):
    """Scales in the requested storage and the fp32 values the oracle must use."""
    if fmt == W.SCALE_F16:
        s16 = np.minimum(s32, 60000.0).astype(np.float16)
        return s16, s16.astype(np.float32)
    if fmt == W.SCALE_F32:
        return s32, s32
    gsb = np.zeros(s32.shape + (4,), np.float32)
    gsb[..., 0] = s32
    return gsb, s32


@pytest.mark.parametrize("rname", list(SCALE_RANGES))
@pytest.mark.parametrize("fmt", [W.SCALE_F32, W.SCALE_GROUPSCALE, W.SCALE_F16])
@pytest.mark.parametrize("m", [1, 8, 64, 2048])
def test_int4_scale_range(ctx, m, fmt, rname):
    r = rng(1000 + m + 10 * fmt + len(rname))
    n_out, K, gs = 256, 512, 32
    q, Wp, _ = int4_weights(r, n_out, K, gs)
    lo, hi = SCALE_RANGES[rname]
    sbuf, sref = _scale_buffer(r.uniform(lo, hi, size=(n_out, K // gs)).astype(np.float32), fmt)
    X, Xf, xc = _x(r, m, K, "bf16" if m == 2048 else "f16")
    d = W.qdesc(n_out, K, m, 4, gs, W.NIBBLE_OFFSET_BINARY, fmt, xc, W.F32)
    got = _run(ctx, d, Wp, sbuf, X, n_out, m, "f32")
    ref = oracle.matmul_nax_grouped_tokens(Wp, sref.reshape(-1), Xf, gs).astype(np.float64)
    assert np.all(np.isfinite(got))
    st = compare(got, ref, f"scale range {rname} fmt {fmt} m {m}")
    for i in range(0, m, max(1, m // 16)):  # token rows
        compare(got[i], ref[i], f"scale range {rname} fmt {fmt} m {m} token {i}")
    print(f"scale range {rname} fmt {fmt} m {m}: rel-L2 {st['rel_l2']:.2e}")


@pytest.mark.parametrize("fmt", [W.SCALE_F32, W.SCALE_GROUPSCALE])
@pytest.mark.parametrize("m", [8, 64, 300])
def test_int4_scales_vary_per_weight_row(ctx, m, fmt):
    """Each weight row's scales sit at their own magnitude, 10^U(-9, 5): every row gets
    its own fold; checked weight row by weight row (output column by column)."""
    r = rng(2000 + m + fmt)
    n_out, K, gs = 320, 512, 64
    q, Wp, _ = int4_weights(r, n_out, K, gs)
    mag = 10.0 ** r.uniform(-9, 5, size=(n_out, 1))
    s32 = (r.uniform(0.5, 1.0, size=(n_out, K // gs)) * mag).astype(np.float32)
    sbuf, sref = _scale_buffer(s32, fmt)
    X, Xf, xc = _x(r, m, K, "bf16")
    d = W.qdesc(n_out, K, m, 4, gs, W.NIBBLE_OFFSET_BINARY, fmt, xc, W.F32)
    got = _run(ctx, d, Wp, sbuf, X, n_out, m, "f32")
    ref = oracle.matmul_nax_grouped_tokens(Wp, sref.reshape(-1), Xf, gs).astype(np.float64)
    for n in range(n_out):
        compare(got[:, n], ref[:, n], f"per-row magnitude m {m} fmt {fmt} weight row {n}")


@pytest.mark.parametrize("fmt", [W.SCALE_F32, W.SCALE_GROUPSCALE])
@pytest.mark.parametrize("coding", [0, 1])
def test_int4_small_m_formats(ctx, fmt, coding):
    """The small-m kernel with fp32 and GroupScale scales, both nibble codings."""
    r = rng(60 + 2 * fmt + coding)
    n_out, K, m, gs = 384, 512, 24, 64
    q, Wp, _ = int4_weights(r, n_out, K, gs, coding)
    sbuf, sref = _scale_buffer(r.uniform(0.005, 0.02, size=(n_out, K // gs)).astype(np.float32), fmt)
    X, Xf, xc = _x(r, m, K, "f16")
    d = W.qdesc(n_out, K, m, 4, gs, coding, fmt, xc, W.F16)
    got = _run(ctx, d, Wp, sbuf, X, n_out, m, "f16")
    ref = oracle.matmul_nax_grouped_tokens(Wp, sref.reshape(-1), Xf, gs, coding)
    compare(got, round_to(ref, "f16"), f"small-m formats {fmt} {coding}")


@pytest.mark.parametrize("n_out,K,m,sf,y", [
    (1000, 2048, 1, "f16", "f16"),      # rows not a multiple of 16, one token
    (4099, 4096, 5, "f32", "f32"),
    (333, 2048, 16, "gs", "bf16"),      # GroupScale records, a full m-tile
    (777, 2048, 17, "none", "f32"),     # no scales, two m-tiles with one token in the second
    (1024, 6144, 32, "f16", "f16"),     # three 1024-k super-chunks per call
    (2051, 3072, 9, "f16", "f16"),      # k not a multiple of 2048 at m <= 16: the general kernel
])
def test_int8_per_row_fp16_x(ctx, n_out, K, m, sf, y):
    """int8 weights with one scale per row and fp16 activations, m <= 32: the kernel that
    stages X in super-chunks and decodes int8 with SDWA conversions, against the oracle
    (dequantize_nax_int8_group with gs = K, then the sequential-k matmul)."""
    r = rng(n_out + K + 11 * m)
    q, s16 = int8_weights(r, n_out, K)
    s32 = s16.astype(np.float32).reshape(-1)
    if sf == "f16":
        s, code = s16, W.SCALE_F16
    elif sf == "f32":
        s32 = r.uniform(1e-3, 1e-2, size=n_out).astype(np.float32)
        s, code = s32, W.SCALE_F32
    elif sf == "gs":
        s32 = r.uniform(1e-3, 1e-2, size=n_out).astype(np.float32)
        s = np.zeros((n_out, 4), np.float32)
        s[:, 0] = s32
        code = W.SCALE_GROUPSCALE
    else:
        s32 = np.ones(n_out, np.float32)
        s, code = np.zeros(4, np.float32), W.SCALE_NONE
    X, Xf, xc = _x(r, m, K, "f16")
    d = W.qdesc(n_out, K, m, 8, K, 0, code, xc, YD[y][0])
    got = _run(ctx, d, q, s, X, n_out, m, y)
    ref = oracle.matmul_int8_dequant_tokens(q, s32, Xf, K)
    compare(got, round_to(ref, y), f"int8 per-row {n_out}x{K} m{m} {sf}")
