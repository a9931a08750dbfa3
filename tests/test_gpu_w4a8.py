"""GPU parity: W4A8 (int4 weights x int8 activations) through lux_hip_qmatmul.

Oracle: matmul_int4_int8 (quantized.wgsl:590-647, two's-complement nibbles) restated
in oracle/lux_oracle.c, and its per-group form.  Integer results are compared
bit-for-bit; the scaled fp output (config 5's group scales and per-token activation
scales) against the fp64 ground truth rounded to the output dtype.
"""
import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import bf16_to_f32, compare, int4_weights, int8_weights, quantize_rows_int8, rng, round_to

pytestmark = pytest.mark.gpu


def _inputs(r, n_out, K, m, gs, coding):
    q, Wp, s = int4_weights(r, n_out, K, gs, coding)
    a8, ascale = quantize_rows_int8(r.standard_normal((m, K)).astype(np.float32))
    return q, Wp, s, a8, ascale


@pytest.mark.parametrize("n_out,K,m,coding", [(11008, 4096, 256, 1), (40, 256, 3, 1),
                                              (97, 512, 300, 0), (64, 128, 17, 1)])
def test_w4a8_full_k_int32_exact(ctx, n_out, K, m, coding):
    """Full-K int32 sums (the reference kernel's output), bit-exact."""
    r = rng(n_out + K + m)
    q, Wp, s, a8, _ = _inputs(r, n_out, K, m, 128, coding)
    d = W.qdesc(n_out, K, m, 4, 128, coding, W.SCALE_NONE, W.I8, W.I32)
    wb, xb, yb = ctx.upload(Wp), ctx.upload(a8), ctx.alloc(m * n_out * 4)
    ctx.qmatmul(d, wb, None, xb, None, yb)
    got = ctx.download(yb, np.int32, (m, n_out))
    ref = oracle.matmul_int4_int8(Wp, np.ascontiguousarray(a8.T), coding).T  # [m, n]
    assert np.array_equal(got, ref)
    if n_out * m < 10**6:  # an independent int64 check on the small shapes
        assert np.array_equal(got, (a8.astype(np.int64) @ q.T).astype(np.int32))


@pytest.mark.parametrize("n_out,K,m,gs", [(512, 4096, 256, 128), (70, 512, 20, 256)])
def test_w4a8_group_partials_exact(ctx, n_out, K, m, gs):
    """Per-group int32 partial sums, bit-exact against brute force."""
    r = rng(7 * n_out + m)
    q, Wp, s, a8, _ = _inputs(r, n_out, K, m, gs, 1)
    d = W.qdesc(n_out, K, m, 4, gs, 1, W.SCALE_F16, W.I8, W.I32, W.QFLAG_GROUP_PARTIALS)
    wb, sb, xb = ctx.upload(Wp), ctx.upload(s), ctx.upload(a8)
    yb = ctx.alloc(m * n_out * (K // gs) * 4)
    ctx.qmatmul(d, wb, sb, xb, None, yb)
    got = ctx.download(yb, np.int32, (m, n_out, K // gs))
    ref = oracle.w4a8_group_partials(Wp, a8, gs, 1)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("y", ["f16", "f32"])
def test_config5_scaled(ctx, y):
    """C5: W 11008 x 4096 int4 g128 fp16 scales, A 256 x 4096 per-token int8."""
    r = rng(5)
    n_out, K, m, gs = 11008, 4096, 256, 128
    q, Wp, s, a8, ascale = _inputs(r, n_out, K, m, gs, 1)
    ycode, ynp = {"f16": (W.F16, np.float16), "f32": (W.F32, np.float32)}[y]
    d = W.qdesc(n_out, K, m, 4, gs, 1, W.SCALE_F16, W.I8, ycode)
    wb, sb, xb, asb = ctx.upload(Wp), ctx.upload(s), ctx.upload(a8), ctx.upload(ascale)
    yb = ctx.alloc(m * n_out * np.dtype(ynp).itemsize)
    ctx.qmatmul(d, wb, sb, xb, asb, yb)
    got = ctx.download(yb, ynp, (m, n_out)).astype(np.float64)
    P = oracle.w4a8_group_partials(Wp, a8, gs, 1).astype(np.float64)      # [m, n, G]
    ref = (P * s.astype(np.float64)[None, :, :]).sum(axis=2) * ascale.astype(np.float64)[:, None]
    st = compare(got, round_to(ref.astype(np.float32), y), f"C5 scaled {y}")
    print(f"C5 {y} rel-L2 {st['rel_l2']:.3e}")


@pytest.mark.parametrize("n_out,K,m,gs,sfmt,y", [
    (70, 512, 20, 256, W.SCALE_F32, "bf16"),       # groups of two stages, ragged rows
    (200, 1024, 65, 128, W.SCALE_GROUPSCALE, "f32"),  # a second 64-token block of one token
    (64, 256, 9, 128, W.SCALE_F16, "f16"),         # two stages: fewer than the prefetch depth
    (130, 384, 3, 128, W.SCALE_F16, "f32")])       # three stages, rows past the last block
def test_w4a8_scaled_shapes(ctx, n_out, K, m, gs, sfmt, y):
    """Scaled output on ragged shapes and every scale format: y = a_s[m] * sum_g s[n,g] P_g,
    P_g from the brute-force int64 group sums."""
    r = rng(n_out * 3 + K + m)
    q, Wp, s16, a8, ascale = _inputs(r, n_out, K, m, gs, 1)
    s32 = r.uniform(0.005, 0.02, size=s16.shape).astype(np.float32)
    if sfmt == W.SCALE_F16:
        sbuf, sref = s16, s16.astype(np.float64)
    elif sfmt == W.SCALE_F32:
        sbuf, sref = s32, s32.astype(np.float64)
    else:  # GroupScale {scale, zero_point, min, max}
        sbuf = np.zeros(s32.shape + (4,), np.float32)
        sbuf[..., 0], sbuf[..., 2], sbuf[..., 3] = s32, -1.0, 1.0
        sref = s32.astype(np.float64)
    ycode, ynp = {"f16": (W.F16, np.float16), "f32": (W.F32, np.float32), "bf16": (W.BF16, np.uint16)}[y]
    d = W.qdesc(n_out, K, m, 4, gs, 1, sfmt, W.I8, ycode)
    yb = ctx.alloc(m * n_out * np.dtype(ynp).itemsize)
    ctx.qmatmul(d, ctx.upload(Wp), ctx.upload(sbuf), ctx.upload(a8), ctx.upload(ascale), yb)
    got = ctx.download(yb, ynp, (m, n_out))
    got = (bf16_to_f32(got) if y == "bf16" else got.astype(np.float32)).astype(np.float64)
    qg = q.reshape(n_out, K // gs, gs).astype(np.int64)
    ag = a8.reshape(m, K // gs, gs).astype(np.int64)
    P = np.einsum("ngk,mgk->mng", qg, ag).astype(np.float64)              # exact group sums
    ref = (P * sref[None, :, :]).sum(axis=2) * ascale.astype(np.float64)[:, None]
    compare(got, round_to(ref.astype(np.float32), y), f"W4A8 scaled {n_out}x{K} m{m} g{gs} {y}")


@pytest.mark.parametrize("n_out,K,m,coding,y", [(11008, 4096, 256, 1, "f16"), (11008, 4096, 256, 0, "f32"),
                                                (11000, 4096, 250, 0, "bf16"), (130, 384, 65, 0, "bf16"),
                                                (64, 128, 3, 1, "f32")])
def test_w4a8_fp16_scales_same_bits_as_fp32_scales(ctx, n_out, K, m, coding, y):
    """g128 with fp16 scales decodes nibbles to 16 q and stages s / 16 (config-5-sized shapes:
    in 11-wave blocks, the group scaling a stage late); fp32 scales of the same values take
    the plain decode in 4-wave blocks. Both feed every fma the same product in the same group
    order, so the outputs must agree bit for bit; and the fp16-scale result matches the exact
    group sums. 11000 x 250: a partial last row block and a partial last token block."""
    r = rng(n_out * 5 + K + m + coding)
    q, Wp, s16, a8, ascale = _inputs(r, n_out, K, m, 128, coding)
    ycode, ynp = {"f16": (W.F16, np.float16), "f32": (W.F32, np.float32), "bf16": (W.BF16, np.uint16)}[y]
    wb, xb, asb = ctx.upload(Wp), ctx.upload(a8), ctx.upload(ascale)
    outs = []
    for sfmt, sbuf in ((W.SCALE_F16, s16), (W.SCALE_F32, s16.astype(np.float32))):
        yb = ctx.alloc(m * n_out * np.dtype(ynp).itemsize)
        ctx.qmatmul(W.qdesc(n_out, K, m, 4, 128, coding, sfmt, W.I8, ycode), wb, ctx.upload(sbuf), xb, asb, yb)
        outs.append(ctx.download(yb, ynp, (m, n_out)))
    assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8))
    got = (bf16_to_f32(outs[0]) if y == "bf16" else outs[0].astype(np.float32)).astype(np.float64)
    P = oracle.w4a8_group_partials(Wp, a8, 128, coding).astype(np.float64)      # [m, n, G]
    ref = (P * s16.astype(np.float64)[None, :, :]).sum(axis=2) * ascale.astype(np.float64)[:, None]
    compare(got, round_to(ref.astype(np.float32), y), f"W4A8 fp16 scales {n_out}x{K} m{m} coding {coding}")


def test_w4a8_rejects(ctx):
    r = rng(1)
    q, Wp, s, a8, ascale = _inputs(r, 32, 128, 4, 128, 1)
    wb, sb, xb, yb = ctx.upload(Wp), ctx.upload(s), ctx.upload(a8), ctx.alloc(4 * 32 * 4)
    with pytest.raises(W.LuxError) as e:  # fp output needs per-token activation scales
        ctx.qmatmul(W.qdesc(32, 128, 4, 4, 128, 1, W.SCALE_F16, W.I8, W.F32), wb, sb, xb, None, yb)
    assert e.value.code == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    s64 = ctx.upload(np.ones((32, 2), np.float16))
    with pytest.raises(W.LuxError) as e:  # group of 64 does not hold whole 128-k stages
        ctx.qmatmul(W.qdesc(32, 128, 4, 4, 64, 1, W.SCALE_F16, W.I8, W.F32), wb, s64, xb,
                    ctx.upload(ascale), yb)
    assert e.value.code == W.LUX_BACKEND_ERROR_NOT_SUPPORTED


@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_w4a8_quantize_x(ctx, xdt):
    """QUANTIZE_X: fp activations quantized per token on the GPU (the W4A8 prologue), then
    the int8 MFMA.  Bit-identical to feeding the host-quantized int8 activations and their
    scales (compute_group_scales NAX_INT8_SYM + quantize_nax_int8_group with gs = K), and
    within tolerance of the oracle's scaled group sums."""
    from util import bf16_bits, bf16_to_f32
    r = rng(55)
    n_out, K, m, gs = 1024, 4096, 256, 128
    q, Wp, s = int4_weights(r, n_out, K, gs, 1)[0:3]
    x = r.standard_normal((m, K)).astype(np.float32)
    if xdt == "bf16":
        xin = bf16_bits(x)
        xf = bf16_to_f32(xin)
        code = W.BF16
    else:
        xin, xf, code = x, x, W.F32
    a8, ascale = quantize_rows_int8(xf)
    wb, sb = ctx.upload(Wp), ctx.upload(s)
    y1, y2 = ctx.alloc(m * n_out * 2), ctx.alloc(m * n_out * 2)
    ctx.qmatmul(W.qdesc(n_out, K, m, 4, gs, 1, W.SCALE_F16, code, W.F16, W.QFLAG_QUANTIZE_X),
                wb, sb, ctx.upload(xin), None, y1)
    ctx.qmatmul(W.qdesc(n_out, K, m, 4, gs, 1, W.SCALE_F16, W.I8, W.F16), wb, sb, ctx.upload(a8),
                ctx.upload(ascale), y2)
    got = ctx.download(y1, np.float16, (m, n_out))
    assert np.array_equal(got.view(np.uint16), ctx.download(y2, np.float16, (m, n_out)).view(np.uint16))
    P = oracle.w4a8_group_partials(Wp, a8, gs, 1).astype(np.float64)
    ref = (P * s.astype(np.float64)[None, :, :]).sum(axis=2) * ascale.astype(np.float64)[:, None]
    compare(got.astype(np.float64), round_to(ref.astype(np.float32), "f16"), f"W4A8 QUANTIZE_X {xdt}")
    with pytest.raises(W.LuxError):  # x_scales must not be passed with QUANTIZE_X
        ctx.qmatmul(W.qdesc(n_out, K, m, 4, gs, 1, W.SCALE_F16, code, W.F16, W.QFLAG_QUANTIZE_X),
                    wb, sb, ctx.upload(xin), ctx.upload(ascale), y1)


@pytest.mark.parametrize("n_out,K,m,gs,xdt,y", [
    (11008, 4096, 256, 128, "f32", "f16"),  # config 5
    (64, 4096, 1000, 128, "f16", "f32"),    # many token blocks, fp16 activations
    (300, 8192, 70, 256, "bf16", "bf16"),   # long rows, ragged rows and tokens
    (130, 128, 5, 128, "f32", "f32"),       # one stage
    (1024, 2048, 64, 2048, "f32", "f16"),   # per-output-channel weight scales
])
def test_w4a8_quantize_x_shapes(ctx, n_out, K, m, gs, xdt, y):
    """QUANTIZE_X over shapes and activation dtypes is bit-identical to the host-quantized
    int8 path (quantize_rows_int8 = compute_group_scales NAX_INT8_SYM +
    quantize_nax_int8_group with gs = K, quantized_nax.wgsl:204-212, 336-362).  Two calls
    in a row, the second with other data and fewer tokens (the workspace is reused)."""
    from util import bf16_bits
    r = rng(n_out + K + m)
    _, Wp, s = int4_weights(r, n_out, K, gs, 1)[0:3]
    xcode = {"f32": W.F32, "f16": W.F16, "bf16": W.BF16}[xdt]
    ycode, ynp = {"f16": (W.F16, np.float16), "f32": (W.F32, np.float32), "bf16": (W.BF16, np.uint16)}[y]
    ybytes = 4 if y == "f32" else 2
    wb, sb = ctx.upload(Wp), ctx.upload(s)
    for rows, seed in ((m, 1), (max(1, m // 2 - 3), 2)):
        x = rng(seed).standard_normal((rows, K)).astype(np.float32) * 3.0
        if xdt == "bf16":
            xin = bf16_bits(x)
            xf = bf16_to_f32(xin)
        elif xdt == "f16":
            xin = x.astype(np.float16)
            xf = xin.astype(np.float32)
        else:
            xin = xf = x
        a8, ascale = quantize_rows_int8(xf)
        y1, y2 = ctx.alloc(rows * n_out * ybytes), ctx.alloc(rows * n_out * ybytes)
        ctx.qmatmul(W.qdesc(n_out, K, rows, 4, gs, 1, W.SCALE_F16, xcode, ycode, W.QFLAG_QUANTIZE_X),
                    wb, sb, ctx.upload(xin), None, y1)
        ctx.qmatmul(W.qdesc(n_out, K, rows, 4, gs, 1, W.SCALE_F16, W.I8, ycode), wb, sb, ctx.upload(a8),
                    ctx.upload(ascale), y2)
        got = ctx.download(y1, ynp, (rows, n_out)).view(np.uint8)
        assert np.array_equal(got, ctx.download(y2, ynp, (rows, n_out)).view(np.uint8)), f"rows {rows}"


# --------------------------------------------------------------------------- W8A8
@pytest.mark.parametrize("n_out,K,m", [(512, 4096, 256), (97, 512, 300), (40, 256, 3)])
def test_w8a8_full_k_int32_exact(ctx, n_out, K, m):
    """int8 weights x int8 activations, full-K int32 sums: matmul_int8
    (quantized.wgsl:497-555) restated in oracle/lux_oracle.c, bit-exact; an independent
    int64 numpy product on top."""
    r = rng(3 * n_out + K + m)
    q, _ = int8_weights(r, n_out, K)
    a8, _ = quantize_rows_int8(r.standard_normal((m, K)).astype(np.float32))
    d = W.qdesc(n_out, K, m, 8, K, 0, W.SCALE_NONE, W.I8, W.I32)
    yb = ctx.alloc(m * n_out * 4)
    ctx.qmatmul(d, ctx.upload(q), None, ctx.upload(a8), None, yb)
    got = ctx.download(yb, np.int32, (m, n_out))
    ref = oracle.matmul_int8(q, np.ascontiguousarray(a8.T)).T  # [m, n]
    assert np.array_equal(got, ref)
    assert np.array_equal(got, (a8.astype(np.int64) @ q.astype(np.int64).T).astype(np.int32))


@pytest.mark.parametrize("n_out,K,m,gs,sfmt,y", [
    (1024, 4096, 256, 4096, W.SCALE_F16, "f16"),  # per-output-channel scales
    (300, 1024, 70, 128, W.SCALE_F32, "bf16"),    # group scales, ragged rows and tokens
])
def test_w8a8_scaled(ctx, n_out, K, m, gs, sfmt, y):
    """Scaled output y = a_s[m] * sum_g s[n,g] P_g[m,n] with int8 weights, P_g exact."""
    r = rng(n_out + 5 * m)
    q, _ = int8_weights(r, n_out, K)
    s = r.uniform(0.001, 0.01, size=(n_out, K // gs)).astype(np.float32)
    sbuf = s.astype(np.float16) if sfmt == W.SCALE_F16 else s
    sref = sbuf.astype(np.float64)
    a8, ascale = quantize_rows_int8(r.standard_normal((m, K)).astype(np.float32))
    ycode, ynp = {"f16": (W.F16, np.float16), "bf16": (W.BF16, np.uint16)}[y]
    d = W.qdesc(n_out, K, m, 8, gs, 0, sfmt, W.I8, ycode)
    yb = ctx.alloc(m * n_out * 2)
    ctx.qmatmul(d, ctx.upload(q), ctx.upload(sbuf), ctx.upload(a8), ctx.upload(ascale), yb)
    got = ctx.download(yb, ynp, (m, n_out))
    got = (bf16_to_f32(got) if y == "bf16" else got.astype(np.float32)).astype(np.float64)
    qg = q.reshape(n_out, K // gs, gs).astype(np.int64)
    ag = a8.reshape(m, K // gs, gs).astype(np.int64)
    P = np.einsum("ngk,mgk->mng", qg, ag).astype(np.float64)
    ref = (P * sref[None, :, :]).sum(axis=2) * ascale.astype(np.float64)[:, None]
    compare(got, round_to(ref.astype(np.float32), y), f"W8A8 scaled {n_out}x{K} m{m} g{gs}")


@pytest.mark.parametrize("m,y", [(256, "f16"), (250, "f32")])
def test_w8a8_config5_shape_wide_blocks(ctx, m, y):
    """W8A8 at config 5's shape with g128 fp16 scales runs in 11-wave blocks with the group
    scaling a stage late; fp32 scales of the same values run in 4-wave blocks. Same products,
    same group order: bit-identical outputs, and both match the exact group sums."""
    r = rng(90 + m)
    n_out, K, gs = 11008, 4096, 128
    q, _ = int8_weights(r, n_out, K)
    s16 = r.uniform(0.001, 0.01, size=(n_out, K // gs)).astype(np.float16)
    a8, ascale = quantize_rows_int8(r.standard_normal((m, K)).astype(np.float32))
    ycode, ynp = {"f16": (W.F16, np.float16), "f32": (W.F32, np.float32)}[y]
    wb, xb, asb = ctx.upload(q), ctx.upload(a8), ctx.upload(ascale)
    outs = []
    for sfmt, sbuf in ((W.SCALE_F16, s16), (W.SCALE_F32, s16.astype(np.float32))):
        yb = ctx.alloc(m * n_out * np.dtype(ynp).itemsize)
        ctx.qmatmul(W.qdesc(n_out, K, m, 8, gs, 0, sfmt, W.I8, ycode), wb, ctx.upload(sbuf), xb, asb, yb)
        outs.append(ctx.download(yb, ynp, (m, n_out)))
    assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8))
    # exact group sums in float64 (|P_g| <= 127 * 127 * 128, far inside 2^53)
    ref = np.zeros((m, n_out))
    qf, af, sf = q.astype(np.float64), a8.astype(np.float64), s16.astype(np.float64)
    for g in range(K // gs):
        ref += (af[:, g * gs:(g + 1) * gs] @ qf[:, g * gs:(g + 1) * gs].T) * sf[None, :, g]
    ref *= ascale.astype(np.float64)[:, None]
    compare(outs[0].astype(np.float64), round_to(ref.astype(np.float32), y), f"W8A8 config-5 shape m{m} {y}")


def test_w8a8_quantize_x(ctx):
    """QUANTIZE_X with int8 weights: bit-identical to the host-quantized int8 path."""
    r = rng(88)
    n_out, K, m = 512, 2048, 64
    q, s = int8_weights(r, n_out, K)
    x = r.standard_normal((m, K)).astype(np.float32)
    a8, ascale = quantize_rows_int8(x)
    wb, sb = ctx.upload(q), ctx.upload(s)
    y1, y2 = ctx.alloc(m * n_out * 4), ctx.alloc(m * n_out * 4)
    ctx.qmatmul(W.qdesc(n_out, K, m, 8, K, 0, W.SCALE_F16, W.F32, W.F32, W.QFLAG_QUANTIZE_X),
                wb, sb, ctx.upload(x), None, y1)
    ctx.qmatmul(W.qdesc(n_out, K, m, 8, K, 0, W.SCALE_F16, W.I8, W.F32), wb, sb, ctx.upload(a8),
                ctx.upload(ascale), y2)
    got = ctx.download(y1, np.float32, (m, n_out))
    assert np.array_equal(got.view(np.uint32), ctx.download(y2, np.float32, (m, n_out)).view(np.uint32))
    ref = (a8.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64).T * ascale.astype(np.float64)[:, None]
    compare(got.astype(np.float64), ref, "W8A8 QUANTIZE_X")
