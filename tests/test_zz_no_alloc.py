"""GPU: lux_hip_qmatmul_noalloc (staging in the library's fixed per-device scratch, no
allocation) against lux_hip_qmatmul_ex (the context workspace) on the same inputs.

Both run the same kernels, so the results must be identical bit for bit.  Each case is
two calls in a row, the second with a smaller input, so the second reuses the scratch
that the first left behind.  The cases cover every kernel that stages through scratch:
the large-m int4 GEMM (fp16-restaged activations, row factors, scale folds), the small-m
int4 GEMM (scale folds, bf16 row factors) and W4A8 with QUANTIZE_X (per-token int8
activations and scales).  A shape above the scratch maximum is refused with
NOT_SUPPORTED.
"""
import numpy as np
import pytest

import webgpu_amd as W
from util import bf16_bits, int4_weights, rng

pytestmark = pytest.mark.gpu


def _pair(ctx, d, Wp, s, X, ybytes, epi=W.EPI_NONE):
    wb, sb, xb = ctx.upload(Wp), ctx.upload(s), ctx.upload(X)
    ya, yb = ctx.alloc(ybytes), ctx.alloc(ybytes)
    ctx.qmatmul_ex(d, wb, sb, xb, None, epi, None, None, ya)
    ctx.qmatmul_noalloc(d, wb, sb, xb, None, epi, None, None, yb)
    a = ctx.download(ya, np.uint8, (ybytes,))
    b = ctx.download(yb, np.uint8, (ybytes,))
    for buf in (wb, sb, xb, ya, yb):
        buf.free()
    return a, b


CASES = {
    # name: [(n_out, k, m, gs, x_dtype, y_dtype, flags, coding), second smaller call]
    "large_m_int4": [(4096, 4096, 2048, 32, "bf16", W.BF16, 0, 0), (512, 1024, 300, 64, "bf16", W.F32, 0, 0)],
    "small_m_int4": [(4096, 4096, 64, 32, "bf16", W.F16, 0, 0), (256, 512, 9, 32, "f32", W.F32, 0, 0)],
    "w4a8_quantize_x": [(4096, 4096, 256, 128, "f32", W.F16, W.QFLAG_QUANTIZE_X, 1),
                        (512, 1024, 40, 128, "f32", W.F32, W.QFLAG_QUANTIZE_X, 1)],
}


def _x(r, m, k, xd):
    x = r.standard_normal((m, k)).astype(np.float32)
    if xd == "bf16":
        return bf16_bits(x), W.BF16
    if xd == "f16":
        return x.astype(np.float16), W.F16
    return x, W.F32


@pytest.mark.parametrize("case", list(CASES))
def test_noalloc_matches_workspace_path(ctx, case):
    r = rng(7100 + len(case))
    for i, (n, k, m, gs, xd, yd, flags, coding) in enumerate(CASES[case]):
        _, Wp, s = int4_weights(r, n, k, gs, coding)
        X, xc = _x(r, m, k, xd)
        d = W.qdesc(n, k, m, 4, gs, coding, W.SCALE_F16, xc, yd, flags)
        ybytes = m * n * (4 if yd == W.F32 else 2)
        a, b = _pair(ctx, d, Wp, s, X, ybytes)
        assert np.array_equal(a, b), f"{case} call {i}: noalloc differs from the workspace path"


def test_noalloc_refuses_oversize(ctx):
    r = rng(7199)
    n, k, m = 256, 8192, 4096  # large-m staging needs 64 MiB + rows: above the maximum
    _, Wp, s = int4_weights(r, n, k, 32)
    X = np.zeros((m, k), np.uint16)
    wb, sb, xb, yb = ctx.upload(Wp), ctx.upload(s), ctx.upload(X), ctx.alloc(m * n * 2)
    d = W.qdesc(n, k, m, 4, 32, 0, W.SCALE_F16, W.BF16, W.BF16)
    with pytest.raises(W.LuxError) as ei:
        ctx.qmatmul_noalloc(d, wb, sb, xb, None, 0, None, None, yb)
    assert ei.value.code == W.LUX_BACKEND_ERROR_NOT_SUPPORTED
    assert "scratch" in str(ei.value)
    for buf in (wb, sb, xb, yb):
        buf.free()
