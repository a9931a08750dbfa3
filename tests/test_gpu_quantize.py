"""GPU parity: producers and codecs of the matmul inputs (lux_hip_quantize, lux_hip_dequantize,
lux_hip_convert_nibbles, lux_hip_convert_scales, lux_hip_requantize_i32).

Oracle: compute_group_scales (quantized_nax.wgsl:157-232), quantize_nax_int4_sym
(:238-262), quantize_nax_int8_group (:336-362) and requantize_int32_to_int8
(quantized.wgsl:572-580) restated in oracle/lux_oracle.c.  Everything here is integer
or a single correctly rounded fp32 operation, so the comparison is bit-for-bit.  With
fp16 scale storage the oracle composition is: scales from compute_group_scales,
rounded to binary16, then the quantizer run with the rounded scales.
"""
import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import bf16_bits, bf16_to_f32, compare, pack_nibbles, quantize_rows_int8, rng, round_to

pytestmark = pytest.mark.gpu

XD = {"f32": W.F32, "f16": W.F16, "bf16": W.BF16}


def _input(r, rows, k, xdt, scale=1.0):
    x = (r.standard_normal((rows, k)) * scale).astype(np.float32)
    if xdt == "f16":
        xs = x.astype(np.float16)
        return xs, xs.astype(np.float32)
    if xdt == "bf16":
        b = bf16_bits(x)
        return b, bf16_to_f32(b)
    return x, x


def _oracle_quant(xf, gs, bits, scale_format):
    """Scales as stored and the packed words the oracle produces with them."""
    fmt = oracle.NAX_INT4_SYM if bits == 4 else oracle.NAX_INT8_SYM
    s, zp, mn, mx = oracle.compute_group_scales(xf, gs, fmt)
    sq = s.astype(np.float16).astype(np.float32) if scale_format == W.SCALE_F16 else s
    words = (oracle.quantize_int4_sym(xf, gs, sq) if bits == 4 else oracle.quantize_int8_group(xf, gs, sq))
    return s, zp, mn, mx, words


def _run(ctx, x, rows, k, bits, gs, coding, sfmt, xdt):
    d = W.quant_desc(rows, k, bits, gs, coding, sfmt, XD[xdt])
    xb = ctx.upload(x)
    qb = ctx.alloc(rows * k * bits // 8)
    sb = ctx.alloc(rows * (k // gs) * {W.SCALE_F16: 2, W.SCALE_F32: 4, W.SCALE_GROUPSCALE: 16}[sfmt])
    ctx.quantize(d, xb, qb, sb)
    q = ctx.download(qb, np.uint32, (rows * k * bits // 32,))
    if sfmt == W.SCALE_GROUPSCALE:
        sraw = ctx.download(sb, np.uint32, (rows * (k // gs), 4))
    else:
        sraw = ctx.download(sb, np.float16 if sfmt == W.SCALE_F16 else np.float32, (rows * (k // gs),))
    return q, sraw


@pytest.mark.parametrize("rows,k,gs,xdt,sfmt", [
    (14336, 4096, 32, "f32", W.SCALE_F16),     # config 2/4 weights
    (300, 512, 128, "bf16", W.SCALE_F32),
    (64, 1024, 64, "f16", W.SCALE_GROUPSCALE),
    (33, 256, 8, "f32", W.SCALE_F16),          # 1056 chunks: a partly filled last wave
    (10, 160, 16, "bf16", W.SCALE_GROUPSCALE),  # 4 lanes per group
    (24, 768, 256, "f16", W.SCALE_F16),        # a group fills one half of a wave
    (40, 1024, 512, "f32", W.SCALE_F32),       # a group spans both halves of a wave
    (16, 8192, 1024, "f32", W.SCALE_F32),      # groups longer than 512: one wave each
    (7, 4096, 4096, "bf16", W.SCALE_F16),      # per-row int4
])
def test_quantize_int4_matches_oracle(ctx, rows, k, gs, xdt, sfmt):
    r = rng(rows + k + gs)
    x, xf = _input(r, rows, k, xdt, scale=0.05)
    q, sraw = _run(ctx, x, rows, k, 4, gs, W.NIBBLE_OFFSET_BINARY, sfmt, xdt)
    s, zp, mn, mx, words = _oracle_quant(xf, gs, 4, sfmt)
    assert np.array_equal(q, words)
    if sfmt == W.SCALE_GROUPSCALE:
        assert np.array_equal(sraw[:, 0], s.view(np.uint32))
        assert np.array_equal(sraw[:, 1], np.zeros_like(zp, np.uint32))
        assert np.array_equal(sraw[:, 2], mn.view(np.uint32))
        assert np.array_equal(sraw[:, 3], mx.view(np.uint32))
    elif sfmt == W.SCALE_F16:
        assert np.array_equal(sraw.view(np.uint16), s.astype(np.float16).view(np.uint16))
    else:
        assert np.array_equal(sraw.view(np.uint32), s.view(np.uint32))


def test_quantize_int4_twos_complement(ctx):
    """Two's-complement output is the offset-binary words with every nibble xor 8."""
    r = rng(11)
    x, xf = _input(r, 40, 256, "f32")
    q, _ = _run(ctx, x, 40, 256, 4, 32, W.NIBBLE_TWOS_COMPLEMENT, W.SCALE_F32, "f32")
    *_, words = _oracle_quant(xf, 32, 4, W.SCALE_F32)
    assert np.array_equal(q, words ^ np.uint32(0x88888888))


@pytest.mark.parametrize("rows,k,gs,xdt", [(256, 4096, 4096, "f32"),   # config 5 activations
                                           (28672 // 16, 8192, 8192, "f16"),  # config 3 rows
                                           (100, 512, 32, "bf16"),
                                           (30, 1024, 512, "f32"),
                                           (11, 88, 8, "f16"),
                                           (9, 16384, 16384, "f32"),   # 8 chunks per thread
                                           (5, 32768, 32768, "bf16")])  # one wave per group
def test_quantize_int8_matches_oracle(ctx, rows, k, gs, xdt):
    r = rng(3 * rows + k)
    x, xf = _input(r, rows, k, xdt)
    q, sraw = _run(ctx, x, rows, k, 8, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F32, xdt)
    s, _, _, _, words = _oracle_quant(xf, gs, 8, W.SCALE_F32)
    assert np.array_equal(q, words)
    assert np.array_equal(sraw.view(np.uint32), s.view(np.uint32))
    if gs == k:  # the per-token quantizer the W4A8 tests use on the host
        q8, s8 = quantize_rows_int8(xf)
        assert np.array_equal(q.view(np.int8).reshape(rows, k), q8)
        assert np.array_equal(sraw, s8)


def test_quantize_edge_values(ctx):
    """All-zero groups (scale 1), exact ties (round half to even), clamping."""
    k, gs = 64, 32
    x = np.zeros((3, k), np.float32)
    x[1, :gs] = np.arange(gs, dtype=np.float32) - 16.0  # absmax 16 -> s = 16/7
    ties = [7.0, -0.5, 0.5, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5, 4.5, -4.5, 5.5, -5.5, 6.5, -6.5, 0.0]
    x[1, gs:] = np.array(ties * 2, np.float32)  # absmax 7 -> s = 1: q = rint(x)
    x[2, :] = np.linspace(-1e4, 3e4, k, dtype=np.float32)
    q, sraw = _run(ctx, x, 3, k, 4, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F32, "f32")
    s, _, _, _, words = _oracle_quant(x, gs, 4, W.SCALE_F32)
    assert np.array_equal(q, words)
    assert np.array_equal(sraw, s)
    assert sraw[0] == 1.0 and sraw[1] == 1.0 and sraw[3] == 1.0  # zero groups; the tie group
    deq = oracle.dequantize_int4(q.reshape(3, k // 8), sraw.reshape(3, k // gs), gs)
    want = [7, 0, 0, 2, -2, 2, -2, 4, -4, 4, -4, 6, -6, 6, -6, 0] * 2
    assert deq[1, gs:].tolist() == want


@pytest.mark.parametrize("bits,sfmt", [(4, W.SCALE_F32), (4, W.SCALE_F16), (8, W.SCALE_F32),
                                       (8, W.SCALE_F16)])
def test_quantize_near_ties_and_tiny_scales(ctx, bits, sfmt):
    """Values whose quotient v / s lies within a few ulps of a half-integer (where a
    reciprocal-multiply would round the other way than the correctly rounded quotient),
    and groups with subnormal scales or a scale whose reciprocal overflows.  Bit-exact
    against the oracle, which divides."""
    r = rng(77 + bits + sfmt)
    gs, groups = 32, 2048
    qmax = 7 if bits == 4 else 127
    amax = r.uniform(0.05, 300.0, groups).astype(np.float32)
    if sfmt == W.SCALE_F32:
        amax[-64:] = (10.0 ** r.uniform(-44, -36, 64)).astype(np.float32)  # subnormal / tiny s
    s = (amax / np.float32(qmax)).astype(np.float32)
    s = s.astype(np.float16).astype(np.float32) if sfmt == W.SCALE_F16 else s
    x = np.zeros((groups, gs), np.float32)
    x[:, 0] = amax
    n = r.integers(-qmax, qmax, size=(groups, gs - 1))
    v = ((n + 0.5) * s[:, None]).astype(np.float32)
    for _ in range(3):  # walk up to 3 ulps either way of (n + 1/2) * s
        step = r.integers(-1, 2, size=v.shape)
        v = np.where(step > 0, np.nextafter(v, np.float32(np.inf)),
                     np.where(step < 0, np.nextafter(v, np.float32(-np.inf)), v)).astype(np.float32)
    x[:, 1:] = np.clip(v, -amax[:, None], amax[:, None])
    rows, k = groups // 8, 8 * gs
    x = x.reshape(rows, k)
    q, sraw = _run(ctx, x, rows, k, bits, gs, W.NIBBLE_OFFSET_BINARY, sfmt, "f32")
    so, _, _, _, words = _oracle_quant(x, gs, bits, sfmt)
    assert np.array_equal(q, words)


def test_quantize_roundtrip_through_gemv(ctx):
    """Quantize fp32 weights on the GPU, then run the int4 GEMV on them: the result
    matches the oracle GEMV of the same packed weights and scales (tolerance of the fp
    paths), and the dequantised weights are within s/2 of the originals."""
    r = rng(21)
    n_out, k, gs = 2048, 4096, 32
    x, xf = _input(r, n_out, k, "f32", scale=0.02)
    q, s16 = _run(ctx, x, n_out, k, 4, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, "f32")
    Wp = q.reshape(n_out, k // 8)
    sc = s16.reshape(n_out, k // gs)
    deq = oracle.dequantize_int4(Wp, sc.astype(np.float32), gs)
    err = np.abs(deq - xf) - 0.5 * np.repeat(sc.astype(np.float32), gs, axis=1)
    assert err.max() <= 1e-6 * np.abs(xf).max()
    v = r.standard_normal(k).astype(np.float16)
    d = W.qdesc(n_out, k, 1, 4, gs, W.NIBBLE_OFFSET_BINARY, W.SCALE_F16, W.F16, W.F16)
    wb, sb, vb, yb = ctx.upload(Wp), ctx.upload(sc), ctx.upload(v), ctx.alloc(n_out * 2)
    ctx.qmatmul(d, wb, sb, vb, None, yb)
    got = ctx.download(yb, np.float16, n_out).astype(np.float64)
    ref = oracle.matmul_nax_grouped(Wp, sc.astype(np.float32).reshape(-1), v.astype(np.float32).reshape(-1, 1), gs)[:, 0]
    compare(got, round_to(ref, "f16"), "quantize -> GEMV")


def test_convert_nibbles(ctx):
    r = rng(5)
    qv = r.integers(-8, 8, size=(37, 64))
    ob, tc = pack_nibbles(qv, 0), pack_nibbles(qv, 1)
    for src, sc, dc, want in [(ob, 0, 1, tc), (tc, 1, 0, ob), (ob, 0, 0, ob)]:
        ib, obuf = ctx.upload(src), ctx.alloc(src.nbytes)
        ctx.convert_nibbles(ib, obuf, src.size, sc, dc)
        assert np.array_equal(ctx.download(obuf, np.uint32, src.shape), want)
    # odd word count and in place
    src = ob.reshape(-1)[:1001].copy()
    ib = ctx.upload(src)
    ctx.convert_nibbles(ib, ib, src.size, 0, 1)
    assert np.array_equal(ctx.download(ib, np.uint32, src.shape), src ^ np.uint32(0x88888888))


def test_convert_scales(ctx):
    r = rng(6)
    s32 = r.uniform(0.001, 0.05, size=777).astype(np.float32)
    b32 = ctx.upload(s32)
    b16, bgs, back = ctx.alloc(777 * 2), ctx.alloc(777 * 16), ctx.alloc(777 * 4)
    ctx.convert_scales(b32, W.SCALE_F32, b16, W.SCALE_F16, 777)
    got16 = ctx.download(b16, np.float16, 777)
    assert np.array_equal(got16.view(np.uint16), s32.astype(np.float16).view(np.uint16))
    ctx.convert_scales(b16, W.SCALE_F16, bgs, W.SCALE_GROUPSCALE, 777)
    gs = ctx.download(bgs, np.uint32, (777, 4))
    assert np.array_equal(gs[:, 0], got16.astype(np.float32).view(np.uint32))
    assert not gs[:, 1:].any()
    ctx.convert_scales(bgs, W.SCALE_GROUPSCALE, back, W.SCALE_F32, 777)
    assert np.array_equal(ctx.download(back, np.float32, 777), got16.astype(np.float32))


def test_requantize_matches_oracle(ctx):
    r = rng(8)
    x = r.integers(-200000, 200000, size=10001).astype(np.int32)
    x[:6] = [0, 1, -1, 5, -5, 2**31 - 1]
    for s_in, s_out, zp in [(0.001, 0.01, 0), (1.0, 2.0, 3), (0.5, 1.0, -7)]:
        ib, ob = ctx.upload(x), ctx.alloc(x.nbytes)
        ctx.requantize(ib, ob, x.size, s_in, s_out, zp)
        got = ctx.download(ob, np.int32, x.shape)
        assert np.array_equal(got, oracle.requantize_int32_to_int8(x, s_in, s_out, zp))
    # half-even ties: 1*1/2 = 0.5 -> 0, 3/2 = 1.5 -> 2, 5/2 -> 2
    t = np.array([1, 3, 5, -1, -3], np.int32)
    ib, ob = ctx.upload(t), ctx.alloc(t.nbytes)
    ctx.requantize(ib, ob, t.size, 1.0, 2.0, 0)
    assert ctx.download(ob, np.int32, t.shape).tolist() == [0, 2, 2, 0, -2]


@pytest.mark.parametrize("size,stride", [(10001, 7), (4096 * 64, 4096), (1023, 1), (333, 1000)])
@pytest.mark.parametrize("quant_type", [0, 1])
def test_int8_per_channel_matches_oracle(ctx, size, stride, quant_type):
    """quantize_int8_per_channel / dequantize_int8_per_channel (quantized.wgsl:264-297),
    one i32 per element, bit-exact against the oracle; ragged sizes, a channel per element,
    one channel for everything; half-even ties, saturation and NaN in the first elements."""
    r = rng(size + stride)
    C = -(-size // stride)
    s = r.uniform(0.01, 0.1, size=C).astype(np.float32)
    zp = r.integers(-20, 20, size=C).astype(np.int32)
    ch = oracle.channel_scales(s, zp)
    x = (r.standard_normal(size) * 8 * np.repeat(s, stride)[:size]).astype(np.float32)
    x[:5] = [2.5 * s[0], -3.5 * s[0], 1e30, np.nan, -np.inf]  # ties exact in channel 0 (stride >= 2)
    cb, xb, qb, ob = ctx.upload(ch), ctx.upload(x), ctx.alloc(size * 4), ctx.alloc(size * 4)
    ctx.quantize_int8_per_channel(xb, cb, qb, size, stride, quant_type)
    q = ctx.download(qb, np.int32, size)
    assert np.array_equal(q, oracle.quantize_int8_per_channel(x, ch, stride, quant_type))
    qi = r.integers(-128, 128, size=size).astype(np.int32)
    qi[:2] = [-2**31, 2**31 - 1]  # the asymmetric subtraction wraps
    ctx.dequantize_int8_per_channel(ctx.upload(qi), cb, ob, size, stride, quant_type)
    got = ctx.download(ob, np.float32, size)
    assert np.array_equal(got.view(np.uint32),
                          oracle.dequantize_int8_per_channel(qi, ch, stride, quant_type).view(np.uint32))


def test_int8_per_channel_unaligned_and_rejects(ctx):
    """Buffers that are 4- but not 16-byte aligned take the element-wise path; bad
    arguments are refused before any launch."""
    import torch
    size, stride = 1001, 10
    r = rng(77)
    ch = oracle.channel_scales(r.uniform(0.01, 0.1, size=-(-size // stride)).astype(np.float32))
    x = r.standard_normal(size).astype(np.float32)
    xt = torch.zeros(size + 1, dtype=torch.float32, device="cuda")
    xt[1:] = torch.from_numpy(x).cuda()
    qt = torch.zeros(size + 1, dtype=torch.int32, device="cuda")
    cb = ctx.upload(ch)
    ctx.quantize_int8_per_channel(ctx.wrap(xt[1:]), cb, ctx.wrap(qt[1:]), size, stride, 0)
    torch.cuda.synchronize()
    assert np.array_equal(qt[1:].cpu().numpy(), oracle.quantize_int8_per_channel(x, ch, stride, 0))
    xb, qb = ctx.upload(x), ctx.alloc(size * 4)
    with pytest.raises(W.LuxError) as e:
        ctx.quantize_int8_per_channel(xb, cb, qb, size, 0, 0)
    assert e.value.code == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    with pytest.raises(W.LuxError) as e:  # one PerChannelScale short
        ctx.quantize_int8_per_channel(xb, ctx.upload(ch[:-1]), qb, size, stride, 0)
    assert e.value.code == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT


def test_quantize_rejects(ctx):
    x = np.zeros((4, 96), np.float32)
    xb, qb, sb = ctx.upload(x), ctx.alloc(4 * 96), ctx.alloc(4 * 96 * 4)
    for bad in [dict(group_size=48), dict(group_size=4), dict(weight_bits=2),
                dict(x_dtype=W.I8), dict(scale_format=W.SCALE_NONE)]:
        kw = dict(rows=4, k=96, weight_bits=4, group_size=32, nibble_coding=0,
                  scale_format=W.SCALE_F32, x_dtype=W.F32)
        kw.update(bad)
        with pytest.raises(W.LuxError):
            ctx.quantize(W.quant_desc(**kw), xb, qb, sb)
    with pytest.raises(W.LuxError):  # output buffer too small
        ctx.quantize(W.quant_desc(4, 96, 8, 32, 0, W.SCALE_F32, W.F32), xb, ctx.alloc(16), sb)


# --------------------------------------------------------------------------- dequantize
def _scale_buffers(r, rows, groups, sfmt):
    """Scales in the requested storage and as the f32 values the dequantizer reads."""
    s32 = r.uniform(0.005, 0.02, size=(rows, groups)).astype(np.float32)
    if sfmt == W.SCALE_F16:
        s16 = s32.astype(np.float16)
        return s16, s16.astype(np.float32)
    if sfmt == W.SCALE_F32:
        return s32, s32
    gsr = np.zeros((rows, groups, 4), np.float32)  # GroupScale {scale, zero_point, min, max}
    gsr[..., 0], gsr[..., 2], gsr[..., 3] = s32, -1.0, 1.0
    return gsr, s32


@pytest.mark.parametrize("bits,rows,k,gs,coding,sfmt,odt", [
    (4, 14336, 4096, 32, 0, W.SCALE_F16, "f32"),   # config 2/4 weights, offset-binary
    (4, 100, 512, 128, 1, W.SCALE_F32, "f16"),     # two's complement nibbles
    (4, 37, 256, 64, 0, W.SCALE_GROUPSCALE, "bf16"),
    (8, 2048, 8192, 8192, 0, W.SCALE_F16, "f32"),  # config 3 per-row int8 (a slice of rows)
    (8, 96, 1024, 64, 0, W.SCALE_F32, "bf16"),
    (4, 50, 960, 96, 1, W.SCALE_F16, "f32"),       # 12 chunks per group: not a power of two
    (8, 20, 720, 24, 0, W.SCALE_F32, "f16"),
])
def test_dequantize_matches_oracle(ctx, bits, rows, k, gs, coding, sfmt, odt):
    """dequantize_nax_int4_sym / dequantize_nax_int8_group: f32 output bit-exact against
    the oracle; f16/bf16 output equal to the oracle's f32 rounded to nearest-even."""
    r = rng(bits * rows + k + gs)
    sbuf, sf = _scale_buffers(r, rows, k // gs, sfmt)
    if bits == 4:
        q = r.integers(-8, 8, size=(rows, k))
        qb = pack_nibbles(q, coding)
        ref = oracle.dequantize_int4(qb.reshape(-1), sf.reshape(-1), gs, coding).reshape(rows, k)
    else:
        qb = r.integers(-128, 128, size=(rows, k)).astype(np.int8)
        ref = oracle.dequantize_int8(qb.reshape(-1), sf.reshape(-1), gs).reshape(rows, k)
    onp = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16}[odt]
    ob = ctx.alloc(rows * k * np.dtype(onp).itemsize)
    ctx.dequantize(W.quant_desc(rows, k, bits, gs, coding, sfmt, XD[odt]), ctx.upload(qb), ctx.upload(sbuf), ob)
    got = ctx.download(ob, onp, (rows, k))
    if odt == "f32":
        assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))
    elif odt == "f16":
        assert np.array_equal(got.view(np.uint16), ref.astype(np.float32).astype(np.float16).view(np.uint16))
    else:
        assert np.array_equal(got, bf16_bits(ref.astype(np.float32)))


def test_dequantize_roundtrip_and_rejects(ctx):
    """quantize then dequantize reproduces the input to within half a step of its group's
    scale (the symmetric grid), and bad descriptors are refused."""
    r = rng(321)
    rows, k, gs = 256, 1024, 32
    x = r.standard_normal((rows, k)).astype(np.float32)
    d = W.quant_desc(rows, k, 4, gs, 0, W.SCALE_F32, W.F32)
    qb, sb, ob = ctx.alloc(rows * k // 2), ctx.alloc(rows * (k // gs) * 4), ctx.alloc(rows * k * 4)
    ctx.quantize(d, ctx.upload(x), qb, sb)
    ctx.dequantize(d, qb, sb, ob)
    back = ctx.download(ob, np.float32, (rows, k))
    s = ctx.download(sb, np.float32, (rows, k // gs))
    err = np.abs(back - x).reshape(rows, k // gs, gs).max(axis=2)
    assert np.all(err <= 0.5 * s * (1 + 1e-6))
    with pytest.raises(W.LuxError):  # group size not a multiple of 8
        ctx.dequantize(W.quant_desc(rows, k, 4, 12, 0, W.SCALE_F32, W.F32), qb, sb, ob)
    with pytest.raises(W.LuxError):  # output too small
        ctx.dequantize(d, qb, sb, ctx.alloc(16))
    with pytest.raises(W.LuxError):  # an integer output type
        ctx.dequantize(W.quant_desc(rows, k, 4, gs, 0, W.SCALE_F32, W.I8), qb, sb, ob)


def test_device_and_host_codecs_agree(ctx):
    """lux_hip_convert_scales / convert_nibbles on the device and the host packers give the
    same bits: binary16 rounding of subnormals, ties and overflow included."""
    r = rng(99)
    f = np.concatenate([r.standard_normal(4096), r.standard_normal(4096) * 1e-6,
                        (np.arange(2048) + 0.5) * 2.0 ** -24, r.uniform(6e4, 7e4, 512),
                        [0.0, -0.0, 65504.0, 65520.0, 2.0 ** -25]]).astype(np.float32)
    n = f.size
    b32, b16 = ctx.upload(f), ctx.alloc(n * 2)
    ctx.convert_scales(b32, W.SCALE_F32, b16, W.SCALE_F16, n)
    assert np.array_equal(ctx.download(b16, np.uint16, n), W.convert_scales_host(f, W.SCALE_F32, W.SCALE_F16))
    q = r.integers(-8, 8, size=4096).astype(np.int8)
    words = W.pack_int4_host(q, W.NIBBLE_OFFSET_BINARY)
    wb, tb = ctx.upload(words), ctx.alloc(words.nbytes)
    ctx.convert_nibbles(wb, tb, words.size, W.NIBBLE_OFFSET_BINARY, W.NIBBLE_TWOS_COMPLEMENT)
    assert np.array_equal(ctx.download(tb, np.uint32, words.size), W.pack_int4_host(q, W.NIBBLE_TWOS_COMPLEMENT))
