"""Pins for the CPU oracle (oracle/lux_oracle.c).

The reference holds no golden vectors for this path, so each oracle function is
pinned by something that does not restate its own formula:
  - library routines (numpy float16 / torch bfloat16 casts, numpy integer matmul);
  - exhaustive enumeration (all 65,536 fp16 patterns, all nibbles and bytes);
  - exact arithmetic: integer-valued inputs with power-of-two scales make every
    fp32 product and partial sum exact, so the result must equal an int64/fp64
    computation bit-for-bit -- a wrong group index, nibble position, sign or
    transposed operand changes the answer;
  - fp64 ground truth within fp32 error bounds for random inputs;
  - invariants (round trips, sum of group partials == full sum).
"""
import numpy as np
import pytest

import oracle as O
from util import pack_nibbles, rng, unpack_nibbles


# --------------------------------------------------------------------------- fp16 / bf16
def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = O.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def _edge_f32():
    r = rng(11)
    v = np.concatenate([
        r.standard_normal(200000).astype(np.float32),
        (r.standard_normal(100000) * 1e-5).astype(np.float32),    # f16 subnormal range
        (r.standard_normal(100000) * 3e4).astype(np.float32),     # near overflow
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 2.0**-24, 2.0**-25,
                  3 * 2.0**-26, 2.0**-14, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf,
                  1e-40, 6.0e-8], np.float32)])
    # exact ties between neighbouring f16 values
    h = np.arange(1, 0x7BFF, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    h2 = np.arange(2, 0x7C00, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    ties = ((h + h2[: len(h)]) / 2).astype(np.float32)
    return np.concatenate([v, ties])


@pytest.mark.filterwarnings("ignore:overflow")
def test_f32_to_f16_rne_matches_numpy():
    v = _edge_f32()
    assert np.array_equal(O.f32_to_f16_rne(v), v.astype(np.float16).view(np.uint16))


@pytest.mark.filterwarnings("ignore:overflow")
def test_f32_to_f16_wgsl_quirks():
    """fp_quantized.wgsl:65-128 equals IEEE RNE except: f32 denormal inputs flush to
    zero and f16-denormal results round half *up* in magnitude."""
    v = _edge_f32()
    got = O.f32_to_f16_wgsl(v)
    ref = v.astype(np.float16).view(np.uint16)
    a = np.abs(v.astype(np.float64))
    normal_out = (a >= 2.0**-14) & np.isfinite(v)
    assert np.array_equal(got[normal_out], ref[normal_out])
    sub = (a < 2.0**-14) & (v.view(np.uint32) & 0x7F800000 != 0)
    mag = np.floor(a[sub] / 2.0**-24 + 0.5).astype(np.uint16)  # round half up
    mag = np.where(a[sub] < 2.0**-25, 0, mag)  # below exponent -25 flushes (:97-99)
    sign = (v[sub].view(np.uint32) >> 16 & 0x8000).astype(np.uint16)
    assert np.array_equal(got[sub], sign | mag)
    den = (v.view(np.uint32) & 0x7F800000) == 0
    assert np.array_equal(got[den], (v[den].view(np.uint32) >> 16 & 0x8000).astype(np.uint16))
    assert O.lib().lo_f32_to_f16_wgsl(np.float32(np.nan)) & 0x7E00 == 0x7E00


def test_bf16_rne_matches_torch():
    torch = pytest.importorskip("torch")
    v = _edge_f32()
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16_rne(v)
    fin = np.isfinite(v)
    assert np.array_equal(got[fin], ref[fin])
    assert np.array_equal(O.bf16_to_f32(got[fin]), torch.from_numpy(ref[fin].view(np.int16))
                          .view(torch.bfloat16).float().numpy())


# --------------------------------------------------------------------------- int codecs
def test_int4_codecs_exhaustive():
    for pos in range(8):
        for v in range(-8, 8):
            vals = np.zeros(8, np.int32)
            vals[pos] = v
            ob = O.lib().lo_pack_int4_ob(vals.ctypes.data_as(O._P))
            tc = O.lib().lo_pack_int4_tc(vals.ctypes.data_as(O._P))
            assert (ob >> (4 * pos)) & 0xF == v + 8          # stored q + 8
            assert (tc >> (4 * pos)) & 0xF == (v & 0xF)      # stored two's complement
            assert ob == tc ^ 0x88888888                     # ob = tc ^ 0x8 per nibble
            assert list(O.unpack_int4(np.array([ob], np.uint32), 0)) == list(vals)
            assert list(O.unpack_int4(np.array([tc], np.uint32), 1)) == list(vals)


def test_int4_pack_matches_vectorised_helper():
    q = rng(1).integers(-8, 8, size=(3, 64))
    for coding in (0, 1):
        assert np.array_equal(O.pack_int4(q, coding), pack_nibbles(q, coding))
        assert np.array_equal(unpack_nibbles(pack_nibbles(q, coding), coding), q)


def test_int8x4_codec_exhaustive():
    L = O.lib()
    for pos in range(4):
        for v in range(-128, 128):
            vals = np.zeros(4, np.int32)
            vals[pos] = v
            w = L.lo_pack_int8x4(vals.ctypes.data_as(O._P))
            assert w == int(np.array(vals, np.int8).view(np.uint32)[0])  # little-endian bytes
            out = np.empty(4, np.int32)
            L.lo_unpack_int8x4(w, out.ctypes.data_as(O._P))
            assert list(out) == list(vals)


# --------------------------------------------------------------------------- fp32 paths
def test_matmul_f32_exact_integers_and_random():
    r = rng(2)
    A = r.integers(-8, 8, size=(37, 70)).astype(np.float32)
    B = r.integers(-8, 8, size=(70, 19)).astype(np.float32)
    assert np.array_equal(O.matmul_f32(A, B), (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32))
    A = r.standard_normal((33, 300)).astype(np.float32)
    B = r.standard_normal((300, 21)).astype(np.float32)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    bound = 300 * 6e-8 * (np.abs(A) @ np.abs(B))
    assert np.all(np.abs(O.matmul_f32(A, B) - ref) <= bound)


@pytest.mark.parametrize("fn", ["gemv_row_parallel", "gemv_vec4"])
def test_gemv_exact_and_alpha_beta(fn):
    r = rng(3)
    M, N = 21, 1003  # N not a multiple of 4 or 256: exercises remainder and tree paths
    A = r.integers(-4, 5, size=(M, N)).astype(np.float32)
    x = r.integers(-4, 5, size=N).astype(np.float32)
    y0 = r.integers(-4, 5, size=M).astype(np.float32)
    exact = (A.astype(np.int64) @ x.astype(np.int64)) * 2 - 3 * y0.astype(np.int64)
    got = getattr(O, fn)(A, x, y0, alpha=2.0, beta=-3.0)
    assert np.array_equal(got, exact.astype(np.float32))
    # e_k extracts column k
    e = np.zeros(N, np.float32)
    e[517] = 1.0
    Ar = r.standard_normal((M, N)).astype(np.float32)
    assert np.array_equal(getattr(O, fn)(Ar, e), Ar[:, 517])


def test_gemv_batched_pinned():
    """gemv_batched: exact on small integers (closed form per batch), batch b equal to
    gemv_row_parallel on its own slice, and stride 0 for A or x shares one operand."""
    r = rng(31)
    B, M, N, lda = 5, 13, 301, 307
    sa, sx, sy = M * lda + 11, N + 3, M + 2
    A = r.integers(-4, 5, size=(B - 1) * sa + M * lda).astype(np.float32)
    x = r.integers(-4, 5, size=(B - 1) * sx + N).astype(np.float32)
    y0 = r.integers(-4, 5, size=(B - 1) * sy + M).astype(np.float32)
    got = O.gemv_batched(A, x, y0, M, N, B, sa, sx, sy, alpha=2.0, beta=-1.0, lda=lda)
    want = y0.copy()  # gaps between the y vectors stay untouched
    for b in range(B):
        Ab = A[b * sa:b * sa + M * lda].reshape(M, lda)[:, :N].astype(np.int64)
        xb = x[b * sx:b * sx + N].astype(np.int64)
        want[b * sy:b * sy + M] = (2 * (Ab @ xb) - y0[b * sy:b * sy + M].astype(np.int64)).astype(np.float32)
    assert np.array_equal(got, want)
    Ar = r.standard_normal(M * N).astype(np.float32)
    xr = r.standard_normal(B * N).astype(np.float32)
    got = O.gemv_batched(Ar, xr, np.zeros(B * M, np.float32), M, N, B, 0, N, M)
    for b in range(B):
        assert np.array_equal(got[b * M:(b + 1) * M], O.gemv_row_parallel(Ar.reshape(M, N), xr[b * N:(b + 1) * N]))


def test_dot_product_fp16_pinned():
    """dot_product_fp16_fp32: small integers are exact, so each vector's result is the int64
    dot product of its pairs; an odd size drops the last pair's second element; an odd
    stride starts odd vectors one element early (word base / 2); one vector per row of a
    matrix with x repeated equals the shared-x GEMV restatement."""
    r = rng(41)
    size, nv, stride = 301, 9, 306
    n = (nv - 1) * stride + 302
    a = r.integers(-6, 7, n).astype(np.float16)
    b = r.integers(-6, 7, n).astype(np.float16)
    got = O.dot_product_fp16_fp32(a.view(np.uint16), b.view(np.uint16), size, nv, stride)
    ai, bi = a.astype(np.int64), b.astype(np.int64)
    want = [int(ai[v * stride:v * stride + size] @ bi[v * stride:v * stride + size]) for v in range(nv)]
    assert np.array_equal(got, np.array(want, np.float32))
    stride = 305  # odd: vector v starts at element 2 * (v * 305 // 2)
    got = O.dot_product_fp16_fp32(a.view(np.uint16), b.view(np.uint16), size, nv, stride)
    st = [2 * (v * stride // 2) for v in range(nv)]
    want = [int(ai[s0:s0 + size] @ bi[s0:s0 + size]) for s0 in st]
    assert np.array_equal(got, np.array(want, np.float32))
    A = r.standard_normal((7, 64)).astype(np.float16)
    x = r.standard_normal(64).astype(np.float16)
    got = O.dot_product_fp16_fp32(A.view(np.uint16), np.tile(x, 7).view(np.uint16), 64, 7, 64)
    assert np.array_equal(got, O.gemv_f16_f32(A.view(np.uint16), x.view(np.uint16)))


def test_gemv_transpose_and_fp16():
    r = rng(4)
    A = r.integers(-4, 5, size=(300, 41)).astype(np.float32)
    x = r.integers(-4, 5, size=300).astype(np.float32)
    assert np.array_equal(O.gemv_transpose(A, x), (A.T.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))
    Ah = r.standard_normal((13, 777)).astype(np.float16)
    xh = r.standard_normal(777).astype(np.float16)
    ref = Ah.astype(np.float64) @ xh.astype(np.float64)
    got = O.gemv_f16_f32(Ah.view(np.uint16), xh.view(np.uint16))
    assert np.all(np.abs(got - ref) <= 777 * 6e-8 * (np.abs(Ah.astype(np.float64)) @ np.abs(xh.astype(np.float64))))
    Ai = r.integers(-3, 4, size=(5, 33)).astype(np.float16)  # odd length: tail element
    xi = r.integers(-3, 4, size=33).astype(np.float16)
    assert np.array_equal(O.gemv_f16_f32(Ai.view(np.uint16), xi.view(np.uint16)),
                          (Ai.astype(np.int64) @ xi.astype(np.int64)).astype(np.float32))


# --------------------------------------------------------------------------- grouped int4
@pytest.mark.parametrize("coding", [0, 1])
@pytest.mark.parametrize("gs", [8, 32, 128])
def test_matmul_nax_grouped_exact(coding, gs):
    """Power-of-two scales that differ per group + small integer activations: all
    fp32 arithmetic is exact, so the oracle must equal the int64 computation."""
    r = rng(5 + gs + coding)
    M, K, N = 23, 256, 9
    q = r.integers(-8, 8, size=(M, K))
    Wp = pack_nibbles(q, coding)
    e = r.integers(-6, 1, size=(M, K // gs))
    s = (2.0 ** e).astype(np.float32)
    act = r.integers(-5, 6, size=(K, N)).astype(np.float32)
    wf = q * np.repeat(2.0 ** e, gs, axis=1)
    ref = wf @ act.astype(np.float64)
    got = O.matmul_nax_grouped(Wp, s.reshape(-1), act, gs, coding)
    assert np.array_equal(got.astype(np.float64), ref)
    # the dequant codec agrees with the same closed form
    assert np.array_equal(O.dequantize_int4(Wp, s.reshape(-1), gs, coding).astype(np.float64), wf)


def test_matmul_nax_grouped_random_vs_f64():
    r = rng(6)
    M, K, N, gs = 40, 1024, 7, 32
    q = r.integers(-8, 8, size=(M, K))
    Wp = pack_nibbles(q, 0)
    s = r.uniform(0.005, 0.02, size=(M, K // gs)).astype(np.float16).astype(np.float32)
    X = r.standard_normal((N, K)).astype(np.float16).astype(np.float32)
    ref = O.qmatmul_f64(Wp, s, X, gs, 4)                       # [N, M]
    got = O.matmul_nax_grouped_tokens(Wp, s.reshape(-1), X, gs)  # [N, M]
    wabs = np.abs(q) * np.repeat(s, gs, axis=1)
    bound = K * 6e-8 * (np.abs(X.astype(np.float64)) @ wabs.T) + 1e-30
    assert np.all(np.abs(got - ref) <= bound)
    # fp64 ground truth itself vs an independent numpy dequant + matmul
    wf = q * np.repeat(s.astype(np.float64), gs, axis=1)
    assert np.allclose(ref, X.astype(np.float64) @ wf.T, rtol=1e-12, atol=1e-12)


def test_int8_dequant_paths():
    r = rng(7)
    M, K, N = 19, 128, 5
    q = r.integers(-127, 128, size=(M, K)).astype(np.int8)
    e = r.integers(-7, 0, size=(M, 1))
    s = (2.0 ** e).astype(np.float32)
    act = r.integers(-4, 5, size=(K, N)).astype(np.float32)
    ref = (q.astype(np.float64) * 2.0 ** e) @ act
    assert np.array_equal(O.matmul_int8_dequant(q, s.reshape(-1), act, K).astype(np.float64), ref)
    assert np.array_equal(O.dequantize_int8(q, s.reshape(-1), K).astype(np.float64), q * 2.0 ** e)
    # group size 32: a scale per 32 consecutive elements of the flat index
    s32 = (2.0 ** r.integers(-5, 1, size=(M, K // 32))).astype(np.float32)
    assert np.array_equal(O.dequantize_int8(q, s32.reshape(-1), 32).astype(np.float64),
                          q * np.repeat(s32.astype(np.float64), 32, axis=1))


# --------------------------------------------------------------------------- integer
@pytest.mark.parametrize("coding", [0, 1])
def test_matmul_int4_int8_brute_force(coding):
    r = rng(8 + coding)
    M, K, N = 29, 512, 13
    q = r.integers(-8, 8, size=(M, K))
    a = r.integers(-128, 128, size=(K, N)).astype(np.int8)
    got = O.matmul_int4_int8(pack_nibbles(q, coding), a, coding)
    assert np.array_equal(got, q @ a.astype(np.int64))


def test_matmul_int8_and_w4a8_partials():
    r = rng(9)
    A = r.integers(-128, 128, size=(11, 96)).astype(np.int8)
    B = r.integers(-128, 128, size=(96, 17)).astype(np.int8)
    assert np.array_equal(O.matmul_int8(A, B), A.astype(np.int64) @ B.astype(np.int64))
    n_out, K, M, gs = 10, 512, 6, 128
    q = r.integers(-8, 8, size=(n_out, K))
    Wp = pack_nibbles(q, 1)
    X = r.integers(-128, 128, size=(M, K)).astype(np.int8)
    P = O.w4a8_group_partials(Wp, X, gs, 1)
    ref = np.einsum("mgk,ngk->mng", X.reshape(M, K // gs, gs).astype(np.int64),
                    q.reshape(n_out, K // gs, gs))
    assert np.array_equal(P, ref)
    # invariant: the group partials sum to matmul_int4_int8's full-K result
    full = O.matmul_int4_int8(Wp, np.ascontiguousarray(X.T), 1)  # [n_out, M]
    assert np.array_equal(P.sum(axis=2).T, full)


def test_requantize():
    x = np.array([0, 1, 2, 3, 5, -5, 1000, -1000, 250, -250, 7], np.int32)
    got = O.requantize_int32_to_int8(x, 0.5, 1.0, 0)
    # 0.5*x rounded half-to-even, clamped to int8
    assert list(got) == [0, 0, 1, 2, 2, -2, 127, -128, 125, -125, 4]
    assert list(O.requantize_int32_to_int8(np.array([4, -300], np.int32), 1.0, 2.0, 3)) == [5, -128]


def test_int8_per_channel_hand_vectors():
    """quantize/dequantize_int8_per_channel (quantized.wgsl:264-297) on hand-computed
    values: channel = i / stride (distinct scales per channel catch a wrong index), the
    zero point's sign in both directions, half-to-even ties, i32 saturation, NaN -> 0 and
    the wrapping i32 subtraction."""
    ch = O.channel_scales([0.5, 2.0, 1.0], [3, -5, 1])
    x = np.array([1.25, 1.75, -1.25, 5.0, 300.0, -1e30, np.nan], np.float32)
    # x / s: 2.5, 3.5, -2.5 | 2.5, 150, -5e29 | NaN
    assert O.quantize_int8_per_channel(x, ch, 3, 0).tolist() == [2, 4, -2, 2, 127, -128, 0]
    assert O.quantize_int8_per_channel(x, ch, 3, 1).tolist() == [5, 7, 1, -3, 127, -128, 0]
    assert O.quantize_int8_per_channel(x, ch, 3, 2).tolist() == [5, 7, 1, -3, 127, -128, 0]  # != 0: asym
    q = np.array([2, -3, 127, 5, -128, 0, -2**31], np.int32)
    assert O.dequantize_int8_per_channel(q, ch, 3, 0).tolist() == [1.0, -1.5, 63.5, 10.0, -256.0, 0.0,
                                                                  -2147483648.0]
    # asym: (q - zp) * s; -2^31 - 1 wraps to 2^31 - 1, whose f32 is 2^31
    assert O.dequantize_int8_per_channel(q, ch, 3, 1).tolist() == [-0.5, -3.0, 62.0, 20.0, -246.0, 10.0,
                                                                  2147483648.0]
    # stride 1: every element its own channel; stride >= size: one channel
    ch1 = O.channel_scales([1.0, 0.25, 4.0])
    assert O.quantize_int8_per_channel(np.array([3.0, 3.0, 3.0], np.float32), ch1, 1).tolist() == [3, 12, 1]
    assert O.quantize_int8_per_channel(np.array([3.0, 3.0, 3.0], np.float32), ch1, 100).tolist() == [3, 3, 3]


def test_int8_per_channel_round_trip():
    """Symmetric round trip: |dequantize(quantize(x)) - x| <= s / 2 for |x / s| <= 127."""
    r = rng(12)
    stride, C = 37, 11
    s = r.uniform(0.01, 0.1, size=C).astype(np.float32)
    x = (r.uniform(-120, 120, size=stride * C) * np.repeat(s, stride)).astype(np.float32)
    ch = O.channel_scales(s)
    back = O.dequantize_int8_per_channel(O.quantize_int8_per_channel(x, ch, stride), ch, stride)
    assert np.all(np.abs(back.astype(np.float64) - x) <= np.repeat(s, stride).astype(np.float64) * 0.5 * (1 + 1e-6))


# --------------------------------------------------------------------------- producers
def test_group_scales_and_quantizers():
    r = rng(10)
    x = r.standard_normal(32 * 20).astype(np.float32)
    x[64:96] = 0.0  # an all-zero group -> scale 1 (quantized_nax.wgsl:228)
    s, zp, mn, mx = O.compute_group_scales(x, 32, O.NAX_INT4_SYM)
    g = x.reshape(20, 32)
    assert np.array_equal(mn, g.min(1)) and np.array_equal(mx, g.max(1))
    amax = np.maximum(np.abs(g.max(1)), np.abs(g.min(1)))
    exp = np.where(amax == 0, 1.0, amax / np.float32(7.0)).astype(np.float32)
    assert np.array_equal(s, exp) and np.all(zp == 0)
    w = O.quantize_int4_sym(x, 32, s)
    deq = O.dequantize_int4(w, s, 32)
    assert np.all(np.abs(deq - x) <= np.repeat(s, 32) / 2 * (1 + 1e-6))
    # values on the grid quantize exactly; clamp at +/-8..7
    grid = (np.arange(-8, 8, dtype=np.float32) * np.float32(0.25)).repeat(2)
    wq = O.quantize_int4_sym(grid, 32, np.array([0.25], np.float32))
    assert np.array_equal(O.dequantize_int4(wq, np.array([0.25], np.float32), 32), grid)
    big = np.array([100.0, -100.0] * 4, np.float32)
    assert list(unpack_nibbles(O.quantize_int4_sym(big, 8, np.array([1.0], np.float32)))) == [7, -8] * 4
    # int8 symmetric, per 128
    s8, _, _, _ = O.compute_group_scales(x, 128, O.NAX_INT8_SYM)
    q8 = O.quantize_int8_group(x, 128, s8).view(np.int8)[: x.size]
    assert np.array_equal(q8, np.clip(np.rint(x / np.repeat(s8, 128)), -128, 127).astype(np.int8))
    # asymmetric int4: zero point = clamp(round(-min/scale), 0, 15)
    sa, za, mna, mxa = O.compute_group_scales(x, 32, O.NAX_INT4_ASYM)
    rng_ = (mxa - mna) / np.float32(15.0)
    rng_ = np.where(rng_ == 0, 1.0, rng_).astype(np.float32)
    assert np.array_equal(sa, rng_)


# ------------------------------------------------------------------ GEMM epilogues
def test_epilogue_activations_pinned():
    """apply_epilogue (steel_gemm_fused.wgsl:80-127) against library routines and closed
    forms: relu exact, sigmoid/silu against scipy's expit, tanh against numpy, gelu's tanh
    form within its known distance of the erf definition, bias/residual exact adds."""
    from scipy.special import erf, expit
    x = np.linspace(-12, 12, 4001, dtype=np.float32).reshape(1, -1)
    xd = x.astype(np.float64)
    assert np.array_equal(O.apply_epilogue(x, O.EPI_RELU), np.maximum(x, 0))
    sig = O.apply_epilogue(x, O.EPI_SIGMOID).astype(np.float64)
    np.testing.assert_allclose(sig, expit(xd), rtol=2e-6, atol=1e-7)
    assert O.apply_epilogue(np.zeros((1, 1), np.float32), O.EPI_SIGMOID)[0, 0] == 0.5
    silu = O.apply_epilogue(x, O.EPI_SILU).astype(np.float64)
    np.testing.assert_allclose(silu, xd * expit(xd), rtol=2e-6, atol=1e-6)
    th = O.apply_epilogue(x, O.EPI_TANH).astype(np.float64)
    np.testing.assert_allclose(th, np.tanh(xd), rtol=1e-6, atol=1e-7)
    gelu = O.apply_epilogue(x, O.EPI_GELU).astype(np.float64)
    exact = 0.5 * xd * (1 + erf(xd / np.sqrt(2)))
    assert np.abs(gelu - exact).max() < 1e-3          # tanh approximation of GELU
    assert np.abs(gelu - exact).max() > 1e-5          # ... and not the erf form itself
    r = np.random.default_rng(3)
    y = r.standard_normal((7, 9)).astype(np.float32)
    b = r.standard_normal(9).astype(np.float32)
    res = r.standard_normal((7, 9)).astype(np.float32)
    assert np.array_equal(O.apply_epilogue(y, O.EPI_ADD_BIAS, bias=b), y + b[None, :])
    assert np.array_equal(O.apply_epilogue(y, O.EPI_ADD_RESIDUAL, residual=res), y + res)
    assert np.array_equal(O.apply_epilogue(y, O.EPI_NONE), y)


def test_silu_mul_pinned():
    """steel_gemm_silu_mul output stage: gate columns first, up columns second."""
    from scipy.special import expit
    r = np.random.default_rng(4)
    g = r.standard_normal((5, 6)).astype(np.float32)
    u = r.standard_normal((5, 6)).astype(np.float32)
    out = O.silu_mul(np.concatenate([g, u], axis=1)).astype(np.float64)
    gd = g.astype(np.float64)
    np.testing.assert_allclose(out, gd * expit(gd) * u, rtol=3e-6, atol=1e-7)
    # halves are not interchangeable: up = 1 gives silu(gate), gate = 0 gives 0
    assert np.array_equal(O.silu_mul(np.concatenate([g, np.ones_like(g)], 1)),
                          O.apply_epilogue(g, O.EPI_SILU))
    assert not O.silu_mul(np.concatenate([np.zeros_like(g), u], 1)).any()


# ------------------------------------------------------------------ around the path
def test_rms_norm_pinned():
    """rms_norm.wgsl restated: against an fp64 evaluation of the definition, and the closed
    forms of constant rows (r = 1/sqrt(c^2 + eps)) and zero rows (r = 1/sqrt(eps))."""
    r = np.random.default_rng(12)
    x = r.standard_normal((5, 3000)).astype(np.float32)
    g = r.uniform(0.5, 1.5, 3000).astype(np.float32)
    y, rms = O.rms_norm(x, g, 1e-6)
    xd = x.astype(np.float64)
    rd = 1.0 / np.sqrt((xd * xd).mean(axis=1) + 1e-6)
    np.testing.assert_allclose(rms, rd, rtol=2e-6)
    np.testing.assert_allclose(y, xd * rd[:, None] * g, rtol=5e-6, atol=1e-7)
    c = np.full((2, 512), 0.75, np.float32)
    c[1] = 0.0
    yc, rc = O.rms_norm(c, np.ones(512, np.float32), 1e-5)
    assert abs(rc[0] - 1 / np.sqrt(0.5625 + 1e-5)) < 1e-6 * rc[0]
    assert abs(rc[1] - 1 / np.sqrt(1e-5)) < 1e-6 * rc[1]
    assert not yc[1].any()
