"""GPU parity: fp32 / fp16 GEMV and op_matmul_f32 through the plugin's C-ABI.

Oracle: gemv_row_parallel / gemv_transpose / gemv_batched / WGSL_MATMUL restated in oracle/
(gemv.wgsl:49-149,297-354, src/webgpu_plugin.cpp:138-205).  Config 1 of BASELINE.json is
the 4096 x 4096 case; the rest are ragged shapes and the alpha/beta/lda paths.
"""
import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import compare, rng

pytestmark = pytest.mark.gpu


def _c1(seed=1, M=4096, K=4096):
    r = rng(seed)
    A = (r.standard_normal((M, K)) * 0.02).astype(np.float32)
    x = r.standard_normal(K).astype(np.float32)
    return A, x


def test_config1_matmul_f32_gemv(ctx):
    """C1: op_matmul_f32 with N == 1 (the vtable hot path) vs the oracle."""
    A, x = _c1()
    ref = oracle.matmul_f32(A, x[:, None])[:, 0]
    a, b, c = ctx.upload(A), ctx.upload(x), ctx.alloc(4096 * 4)
    ctx.matmul_f32(a, b, c, 4096, 4096, 1)
    got = ctx.download(c, np.float32, 4096)
    st = compare(got, ref, "C1 matmul N=1")
    assert st["rel_l2"] < 1e-5  # fp32 vs fp32: reassociation only
    ref2 = oracle.gemv_row_parallel(A, x)
    compare(got, ref2, "C1 vs gemv_row_parallel", rel_tol=1e-5)


@pytest.mark.parametrize("M,K", [(4096, 4096), (1, 7), (5, 1000), (129, 4099), (300, 64)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 2.0)])
def test_gemv_f32_row(ctx, M, K, alpha, beta):
    r = rng(M * 7 + K)
    A = r.standard_normal((M, K)).astype(np.float32)
    x = r.standard_normal(K).astype(np.float32)
    y0 = r.standard_normal(M).astype(np.float32)
    ref = oracle.gemv_row_parallel(A, x, y0, alpha, beta)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.upload(y0)
    ctx.gemv_f32(a, xb, yb, M, K, alpha, beta)
    compare(ctx.download(yb, np.float32, M), ref, f"gemv {M}x{K}", rel_tol=1e-5)


def test_gemv_f32_lda_and_transpose(ctx):
    r = rng(5)
    M, N, lda = 200, 300, 333
    A = r.standard_normal((M, lda)).astype(np.float32)
    x = r.standard_normal(N).astype(np.float32)
    ref = oracle.gemv_row_parallel(A, x, None, 1.0, 0.0, lda=lda, rows=M, cols=N)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.alloc(M * 4)
    ctx.gemv_f32(a, xb, yb, M, N, lda=lda)
    compare(ctx.download(yb, np.float32, M), ref, "gemv lda", rel_tol=1e-5)
    # y[N] = A^T x over an [M x N] matrix
    A2 = r.standard_normal((M, N)).astype(np.float32)
    x2 = r.standard_normal(M).astype(np.float32)
    y2 = r.standard_normal(N).astype(np.float32)
    ref2 = oracle.gemv_transpose(A2, x2, y2, 2.0, -1.0)
    a2, xb2, yb2 = ctx.upload(A2), ctx.upload(x2), ctx.upload(y2)
    ctx.gemv_f32(a2, xb2, yb2, M, N, 2.0, -1.0, trans=True)
    compare(ctx.download(yb2, np.float32, N), ref2, "gemv_transpose", rel_tol=1e-5)


@pytest.mark.parametrize("M,N,lda", [(33, 2047, 2052), (1, 1024, 1024), (8192, 1030, 1032)])
def test_gemv_f32_rows_split_between_waves(ctx, M, N, lda):
    """Few long rows: each row's two halves go to two waves (16-B aligned split, K % 4 tail
    in the second half); odd M leaves one wave pair of the last block idle."""
    r = rng(M + N)
    A = r.standard_normal((M, lda)).astype(np.float32)
    x = r.standard_normal(N).astype(np.float32)
    y0 = r.standard_normal(M).astype(np.float32)
    ref = oracle.gemv_row_parallel(A, x, y0, 0.75, -0.5, lda=lda, rows=M, cols=N)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.upload(y0)
    ctx.gemv_f32(a, xb, yb, M, N, 0.75, -0.5, lda=lda)
    compare(ctx.download(yb, np.float32, M), ref, f"gemv split {M}x{N}", rel_tol=1e-5)


@pytest.mark.parametrize("M,K,lda", [(4096, 4096, 4096), (8192, 4096, 4100), (2048, 2048, 2048),
                                     (3000, 2048, 2052), (1024, 1024, 1024), (1500, 4096, 4096)])
def test_gemv_f32_rows_in_k_quarters(ctx, M, K, lda):
    """Few rows with k in {1024, 2048, 4096}: four waves per row set, one per quarter of k,
    each wave 4, 8 or 16 rows; ragged last row sets (1500, 3000) compute clamped rows and
    store only their own."""
    r = rng(M * 3 + K)
    A = r.standard_normal((M, lda)).astype(np.float32)
    x = r.standard_normal(K).astype(np.float32)
    y0 = r.standard_normal(M).astype(np.float32)
    ref = oracle.gemv_row_parallel(A, x, y0, 1.25, 0.5, lda=lda, rows=M, cols=K)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.upload(y0)
    ctx.gemv_f32(a, xb, yb, M, K, 1.25, 0.5, lda=lda)
    compare(ctx.download(yb, np.float32, M), ref, f"gemv quarters {M}x{K}", rel_tol=1e-5)


@pytest.mark.parametrize("M,K,N", [(64, 64, 64), (100, 37, 70), (1, 512, 300), (257, 129, 3),
                                   (512, 1024, 256)])
def test_matmul_f32_general(ctx, M, K, N):
    r = rng(M + K + N)
    A = r.standard_normal((M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    ref = oracle.matmul_f32(A, B)
    a, b, c = ctx.upload(A), ctx.upload(B), ctx.alloc(M * N * 4)
    ctx.matmul_f32(a, b, c, M, K, N)
    compare(ctx.download(c, np.float32, (M, N)), ref, f"matmul {M}x{K}x{N}", rel_tol=1e-5)


def test_matmul_f32_empty_and_errors(ctx):
    a, b, c = ctx.alloc(64), ctx.alloc(64), ctx.alloc(64)
    ctx.matmul_f32(a, b, c, 0, 4, 4)  # empty: OK, nothing written
    with pytest.raises(W.LuxError) as e:
        ctx.matmul_f32(a, b, c, 16, 16, 16)  # buffers too small
    assert e.value.code == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    # K == 0 -> zeros
    c2 = ctx.upload(np.full(4, 7.0, np.float32))
    ctx.matmul_f32(a, b, c2, 2, 0, 2)
    assert np.all(ctx.download(c2, np.float32, 4) == 0)


@pytest.mark.parametrize("M,K", [(4096, 4096), (33, 1000), (7, 8), (64, 4095)])
def test_gemv_f16(ctx, M, K):
    r = rng(M + 3 * K)
    A = r.standard_normal((M, K)).astype(np.float16)
    x = r.standard_normal(K).astype(np.float16)
    ref = oracle.gemv_f16_f32(A.view(np.uint16), x.view(np.uint16))
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.alloc(M * 4)
    ctx.gemv_f16(a, xb, yb, M, K)
    compare(ctx.download(yb, np.float32, M), ref, f"gemv_f16 {M}x{K}", rel_tol=1e-5)


@pytest.mark.parametrize("M,K,lda", [(14336, 4096, 4096), (3000, 2048, 2056), (1024, 512, 512),
                                     (20000, 1024, 1024), (2049, 4096, 4104)])
def test_gemv_f16_rows_per_wave(ctx, M, K, lda):
    """Whole rows of 512-4096 halves, 1-8 rows per wave at 8 waves per CU: ragged last waves
    (3000, 2049 rows) compute clamped rows and store only their own; padded lda."""
    r = rng(M + 5 * K)
    A = r.standard_normal((M, lda)).astype(np.float16)
    x = r.standard_normal(K).astype(np.float16)
    ref = oracle.gemv_f16_f32(np.ascontiguousarray(A[:, :K]).view(np.uint16), x.view(np.uint16))
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.alloc(M * 4)
    ctx.gemv_f16(a, xb, yb, M, K, lda=lda)
    compare(ctx.download(yb, np.float32, M), ref, f"gemv_f16 rows {M}x{K} lda {lda}", rel_tol=1e-5)


# --------------------------------------------------------------------------- gemv_batched
@pytest.mark.parametrize("B,M,N,lda,pad_a,pad_x,pad_y", [
    (32, 2048, 128, 128, 0, 0, 0),    # 32 heads x 2048 keys x head dim 128, vector path
    (5, 13, 301, 307, 11, 3, 2),      # ragged: odd strides take the scalar path
    (70000, 3, 8, 8, 0, 0, 0),        # more batches than one grid dimension holds
    (3, 1000, 64, 64, 0, 0, 0),       # short rows, 4 per wave
    (4, 77, 37, 40, 8, 3, 1),         # short rows with a K % 4 tail and ragged rows
    (2, 5000, 100, 100, 0, 0, 0),     # short rows, 25 of 32 lanes per row busy
    (2, 999, 7, 8, 4, 1, 0),          # shortest rows: 8 per wave
])
def test_gemv_f32_batched(ctx, B, M, N, lda, pad_a, pad_x, pad_y):
    """gemv_batched vs the oracle (gemv.wgsl:297-354), rel-L2 <= 1e-5 (fp32, reassociated
    sums); elements between the y vectors are left untouched."""
    r = rng(B + M + N)
    sa, sx, sy = M * lda + pad_a, N + pad_x, M + pad_y
    A = r.standard_normal((B - 1) * sa + M * lda).astype(np.float32)
    x = r.standard_normal((B - 1) * sx + N).astype(np.float32)
    y0 = r.standard_normal((B - 1) * sy + M).astype(np.float32)
    alpha, beta = (0.5, 2.0) if pad_y else (1.0, 0.0)
    ref = oracle.gemv_batched(A, x, y0, M, N, B, sa, sx, sy, alpha, beta, lda=lda)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.upload(y0)
    ctx.gemv_f32_batched(a, xb, yb, M, N, B, sa, sx, sy, alpha, beta, lda=lda)
    got = ctx.download(yb, np.float32, y0.size)
    compare(got, ref, f"gemv_batched {B}x{M}x{N}", rel_tol=1e-5)
    gaps = np.ones(y0.size, bool)
    for b in range(B):
        gaps[b * sy:b * sy + M] = False
    assert np.array_equal(got[gaps], y0[gaps])


def test_gemv_f32_batched_shared_operands_and_errors(ctx):
    """stride 0 shares one matrix (or one vector) across batches; integer inputs make the
    result exact.  Overlapping y vectors, short buffers and empty batches."""
    r = rng(77)
    B, M, N = 6, 40, 520
    A = r.integers(-4, 5, size=M * N).astype(np.float32)
    x = r.integers(-4, 5, size=B * N).astype(np.float32)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.alloc(B * M * 4)
    ctx.gemv_f32_batched(a, xb, yb, M, N, B, 0, N, M)            # one A, B vectors
    want = (x.reshape(B, N).astype(np.int64) @ A.reshape(M, N).T.astype(np.int64)).astype(np.float32)
    assert np.array_equal(ctx.download(yb, np.float32, (B, M)), want)
    A2 = r.integers(-4, 5, size=B * M * N).astype(np.float32)
    a2 = ctx.upload(A2)
    ctx.gemv_f32_batched(a2, xb, yb, M, N, B, M * N, 0, M)       # B matrices, one x
    want2 = (A2.reshape(B, M, N).astype(np.int64) @ x[:N].astype(np.int64)).astype(np.float32)
    assert np.array_equal(ctx.download(yb, np.float32, (B, M)), want2)
    with pytest.raises(W.LuxError):  # y vectors overlap
        ctx.gemv_f32_batched(a2, xb, yb, M, N, B, M * N, N, M - 1)
    with pytest.raises(W.LuxError):  # A holds B-1 matrices only
        ctx.gemv_f32_batched(a, xb, yb, M, N, B, M * N, N, M)
    ctx.gemv_f32_batched(a, xb, yb, M, N, 0, 0, 0, 0)            # empty batch: no-op
    assert np.array_equal(ctx.download(yb, np.float32, (B, M)), want2)


def test_gemv_f32_more_rows_than_one_grid_pass(ctx):
    """2^22 + 37 rows: beyond 2^20 blocks of 4 rows, waves stride over the rest.  Small
    integers make every row exact, so numpy's int64 product is the check."""
    r = rng(78)
    M, N = (1 << 22) + 37, 4
    A = r.integers(-4, 5, size=(M, N)).astype(np.float32)
    x = r.integers(-4, 5, size=N).astype(np.float32)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.alloc(M * 4)
    ctx.gemv_f32(a, xb, yb, M, N)
    want = (A.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)
    assert np.array_equal(ctx.download(yb, np.float32, M), want)


@pytest.mark.parametrize("size,nv,stride", [(4096, 512, 4096),   # vector path
                                            (301, 9, 306),       # odd size, scalar path
                                            (301, 9, 305),       # odd stride: odd vectors start early
                                            (64, 3, 0),          # stride 0: one pair of vectors
                                            (0, 4, 8)])          # empty vectors: zeros
def test_dot_f16(ctx, size, nv, stride):
    """dot_product_fp16_fp32 (fp_quantized.wgsl:418-469) vs the oracle; rel-L2 <= 1e-5
    (exact fp16 products, fp32 sums reassociated)."""
    r = rng(size + nv + stride)
    n = max(2 * (((nv - 1) * stride) // 2) + size, 1)
    a = r.standard_normal(n).astype(np.float16)
    b = r.standard_normal(n).astype(np.float16)
    ref = oracle.dot_product_fp16_fp32(a.view(np.uint16), b.view(np.uint16), size, nv, stride)
    ab, bb, rb = ctx.upload(a), ctx.upload(b), ctx.alloc(nv * 4)
    ctx.dot_f16(ab, bb, rb, size, nv, stride)
    got = ctx.download(rb, np.float32, nv)
    if size == 0:
        assert np.array_equal(got, np.zeros(nv, np.float32))
    else:
        compare(got, ref, f"dot_f16 {size}x{nv}/{stride}", rel_tol=1e-5)
    with pytest.raises(W.LuxError):  # b one element short
        ctx.dot_f16(ab, ctx.upload(b[:n - 1]) if n > 1 else ctx.alloc(0), rb, size + 1, nv, stride)


@pytest.mark.parametrize("M,N,lda", [(4096, 4096, 4096),   # the config-1 matrix, 16-B loads
                                     (1000, 301, 301),     # scalar path, ragged strip
                                     (20000, 64, 68),      # 256 row chunks of 79 rows
                                     (37, 1024, 1024)])    # one partly filled chunk
def test_gemv_f32_transpose_two_pass(ctx, M, N, lda):
    """gemv_transpose (gemv.wgsl:103-149) through the two-pass kernel vs the oracle."""
    r = rng(M + N)
    A = r.standard_normal((M, lda)).astype(np.float32)
    x = r.standard_normal(M).astype(np.float32)
    y0 = r.standard_normal(N).astype(np.float32)
    ref = oracle.gemv_transpose(np.ascontiguousarray(A[:, :N]), x, y0, 1.5, 0.5)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.upload(y0)
    ctx.gemv_f32(a, xb, yb, M, N, 1.5, 0.5, lda=lda, trans=True)
    compare(ctx.download(yb, np.float32, N), ref, f"gemv_t {M}x{N}", rel_tol=1e-5)


def test_gemv_f32_transpose_inf_and_empty(ctx):
    """An inf in A gives inf in its column (no 0 * inf from the padding of a partly filled
    chunk); M = 0 leaves y = beta * y."""
    M, N = 37, 256
    A = np.ones((M, N), np.float32)
    A[0, 5] = np.inf
    x = np.ones(M, np.float32)
    a, xb, yb = ctx.upload(A), ctx.upload(x), ctx.alloc(N * 4)
    ctx.gemv_f32(a, xb, yb, M, N, trans=True)
    got = ctx.download(yb, np.float32, N)
    assert got[5] == np.inf and np.all(got[np.arange(N) != 5] == M)
    y0 = np.full(N, 2.0, np.float32)
    yb2 = ctx.upload(y0)
    ctx.gemv_f32(a, xb, yb2, 0, N, 1.0, 3.0, trans=True)
    assert np.all(ctx.download(yb2, np.float32, N) == 6.0)


@pytest.mark.parametrize("M,K,N", [(1024, 1024, 1024), (129, 260, 68), (2, 4, 4), (300, 1000, 516),
                                   (1000, 36, 2000)])
def test_matmul_f32_mfma(ctx, M, K, N):
    """op_matmul_f32 on the fp32 matrix cores (rows 16-byte aligned: K, N multiples of 4),
    both tile sizes and ragged edges, against the oracle's sequential-k matmul."""
    r = rng(M * 3 + K + N)
    A = r.standard_normal((M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    ref = oracle.matmul_f32(A, B)
    a, b, c = ctx.upload(A), ctx.upload(B), ctx.alloc(M * N * 4)
    ctx.matmul_f32(a, b, c, M, K, N)
    compare(ctx.download(c, np.float32, (M, N)), ref, f"matmul mfma {M}x{K}x{N}", rel_tol=1e-5)
