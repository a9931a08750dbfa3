"""GPU parity: fp32 / fp16 GEMV and op_matmul_f32 through the plugin's C-ABI.

Oracle: gemv_row_parallel / gemv_transpose / WGSL_MATMUL restated in oracle/
(gemv.wgsl:49-149, src/webgpu_plugin.cpp:138-205).  Config 1 of BASELINE.json is
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
