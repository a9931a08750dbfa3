"""CPU oracle for the quantized-matmul path -- TEST INFRASTRUCTURE ONLY.

A C restatement (``lux_oracle.c``) of the luxcpp/webgpu WGSL arithmetic, wrapped
with ctypes for numpy arrays.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the reported CPU baseline; the HIP plugin never depends on it.

Every wrapper keeps the reference's layouts: weights ``[rows, K]`` packed along K,
grouped/int activations ``[K, N]`` and outputs ``[rows, N]``.  Token-major helpers
(``*_tokens``) transpose at the numpy level only.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblux_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

_SIGS = {
    "lo_f32_to_f16_wgsl": (ctypes.c_uint32, [_F]),
    "lo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint32]),
    "lo_f32_to_f16_rne": (ctypes.c_uint16, [_F]),
    "lo_f32_to_bf16_rne": (ctypes.c_uint16, [_F]),
    "lo_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "lo_pack_int4_ob": (ctypes.c_uint32, [_P]),
    "lo_unpack_int4_ob": (None, [ctypes.c_uint32, _P]),
    "lo_pack_int4_tc": (ctypes.c_uint32, [_P]),
    "lo_unpack_int4_tc": (None, [ctypes.c_uint32, _P]),
    "lo_pack_int8x4": (ctypes.c_uint32, [_P]),
    "lo_unpack_int8x4": (None, [ctypes.c_uint32, _P]),
    "lo_f16_to_f32_array": (None, [_P, _P, _SZ]),
    "lo_f32_to_f16_rne_array": (None, [_P, _P, _SZ]),
    "lo_f32_to_f16_wgsl_array": (None, [_P, _P, _SZ]),
    "lo_bf16_to_f32_array": (None, [_P, _P, _SZ]),
    "lo_f32_to_bf16_rne_array": (None, [_P, _P, _SZ]),
    "lo_matmul_f32": (None, [_P, _P, _P, _I, _I, _I]),
    "lo_gemv_row_parallel": (None, [_P, _P, _P, _I, _I, _I, _F, _F]),
    "lo_gemv_transpose": (None, [_P, _P, _P, _I, _I, _I, _F, _F]),
    "lo_gemv_batched": (None, [_P, _P, _P, _I, _I, _I, _F, _F, _I, ctypes.c_long, ctypes.c_long,
                               ctypes.c_long]),
    "lo_gemv_vec4": (None, [_P, _P, _P, _I, _I, _I, _F, _F]),
    "lo_gemv_f16_f32": (None, [_P, _P, _P, _I, _I, _I]),
    "lo_dot_product_fp16_fp32": (None, [_P, _P, _P, _I, _I, _I]),
    "lo_matmul_nax_grouped": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "lo_dequantize_nax_int4_sym": (None, [_P, _P, _P, _SZ, _I, _I]),
    "lo_dequantize_nax_int8_group": (None, [_P, _P, _P, _SZ, _I]),
    "lo_matmul_int8_dequant": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "lo_matmul_int4_int8": (None, [_P, _P, _P, _I, _I, _I, _I]),
    "lo_matmul_int8": (None, [_P, _P, _P, _I, _I, _I]),
    "lo_requantize_int32_to_int8": (None, [_P, _P, _SZ, _F, _F, ctypes.c_int32]),
    "lo_quantize_int8_per_channel": (None, [_P, _P, _P, _SZ, ctypes.c_uint32, ctypes.c_uint32]),
    "lo_dequantize_int8_per_channel": (None, [_P, _P, _P, _SZ, ctypes.c_uint32, ctypes.c_uint32]),
    "lo_apply_epilogue": (None, [_P, _I, _I, _I, _P, _P]),
    "lo_silu_mul": (None, [_P, _P, _I, _I]),
    "lo_rms_norm": (None, [_P, _P, _P, _P, _I, _I, _F]),
    "lo_w4a8_group_partials": (None, [_P, _P, _P, _I, _I, _I, _I, _I]),
    "lo_compute_group_scales": (None, [_P, _SZ, _I, _I, _P, _P, _P, _P]),
    "lo_quantize_nax_int4_sym": (None, [_P, _SZ, _I, _P, _P]),
    "lo_quantize_nax_int8_group": (None, [_P, _SZ, _I, _P, _P]),
    "lo_qmatmul_f64": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "lo_num_threads": (_I, []),
}

NIBBLE_OFFSET_BINARY = 0
NIBBLE_TWOS_COMPLEMENT = 1
NAX_INT4_SYM, NAX_INT4_ASYM, NAX_INT8_SYM, NAX_INT8_ASYM = 0, 1, 2, 3


def build(force: bool = False) -> str:
    """Compile liblux_oracle.so with oracle/Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE] + (["-B"] if force else []), check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------- codecs
def f16_to_f32(bits) -> np.ndarray:
    b = _c(bits, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().lo_f16_to_f32_array(_p(b), _p(out), b.size)
    return out


def f32_to_f16_rne(x) -> np.ndarray:
    a = _c(x, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().lo_f32_to_f16_rne_array(_p(a), _p(out), a.size)
    return out


def f32_to_f16_wgsl(x) -> np.ndarray:
    a = _c(x, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().lo_f32_to_f16_wgsl_array(_p(a), _p(out), a.size)
    return out


def bf16_to_f32(bits) -> np.ndarray:
    b = _c(bits, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().lo_bf16_to_f32_array(_p(b), _p(out), b.size)
    return out


def f32_to_bf16_rne(x) -> np.ndarray:
    a = _c(x, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().lo_f32_to_bf16_rne_array(_p(a), _p(out), a.size)
    return out


def pack_int4(q, coding: int = NIBBLE_OFFSET_BINARY) -> np.ndarray:
    """Pack int values in [-8, 7] (shape [..., K], K % 8 == 0) 8 per u32."""
    q = _c(q, np.int32)
    flat = q.reshape(-1, 8)
    fn = lib().lo_pack_int4_ob if coding == NIBBLE_OFFSET_BINARY else lib().lo_pack_int4_tc
    out = np.empty(flat.shape[0], np.uint32)
    for i in range(flat.shape[0]):
        row = np.ascontiguousarray(flat[i])
        out[i] = fn(_p(row))
    return out.reshape(q.shape[:-1] + (q.shape[-1] // 8,))


def unpack_int4(words, coding: int = NIBBLE_OFFSET_BINARY) -> np.ndarray:
    w = _c(words, np.uint32)
    fn = lib().lo_unpack_int4_ob if coding == NIBBLE_OFFSET_BINARY else lib().lo_unpack_int4_tc
    out = np.empty(w.shape + (8,), np.int32)
    o2 = out.reshape(-1, 8)
    for i, v in enumerate(w.reshape(-1)):
        row = np.empty(8, np.int32)
        fn(int(v), _p(row))
        o2[i] = row
    return out.reshape(w.shape[:-1] + (w.shape[-1] * 8,)) if w.ndim else out


# --------------------------------------------------------------------------- fp32
def matmul_f32(A, B) -> np.ndarray:
    A = _c(A, np.float32)
    B = _c(B, np.float32)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    C = np.empty((M, N), np.float32)
    lib().lo_matmul_f32(_p(A), _p(B), _p(C), M, K, N)
    return C


def _gemv(fn, A, x, y, alpha, beta, lda=None, rows=None, cols=None):
    A = _c(A, np.float32)
    x = _c(x, np.float32)
    M = rows if rows is not None else A.shape[0]
    N = cols if cols is not None else A.shape[1]
    lda = lda if lda is not None else A.shape[1]
    y = _c(np.zeros(M if fn != "lo_gemv_transpose" else N, np.float32) if y is None else y,
           np.float32).copy()
    getattr(lib(), fn)(_p(A), _p(x), _p(y), M, N, lda, float(alpha), float(beta))
    return y


def gemv_row_parallel(A, x, y=None, alpha=1.0, beta=0.0, lda=None, rows=None, cols=None):
    return _gemv("lo_gemv_row_parallel", A, x, y, alpha, beta, lda, rows, cols)


def gemv_transpose(A, x, y=None, alpha=1.0, beta=0.0):
    return _gemv("lo_gemv_transpose", A, x, y, alpha, beta)


def gemv_batched(A, x, y, M, N, batch, stride_a, stride_x, stride_y, alpha=1.0, beta=0.0,
                 lda=None):
    """gemv_batched over flat buffers A, x, y (strides and lda in elements); returns the new y."""
    A = _c(A, np.float32).reshape(-1)
    x = _c(x, np.float32).reshape(-1)
    y = _c(y, np.float32).reshape(-1).copy()
    lda = N if lda is None else lda
    if batch > 0 and M > 0:
        assert A.size >= (batch - 1) * stride_a + (M - 1) * lda + N
        assert x.size >= (batch - 1) * stride_x + N and y.size >= (batch - 1) * stride_y + M
    lib().lo_gemv_batched(_p(A), _p(x), _p(y), M, N, lda, float(alpha), float(beta), batch,
                          stride_a, stride_x, stride_y)
    return y


def gemv_vec4(A, x, y=None, alpha=1.0, beta=0.0):
    return _gemv("lo_gemv_vec4", A, x, y, alpha, beta)


def gemv_f16_f32(A_bits, x_bits) -> np.ndarray:
    A = _c(A_bits, np.uint16)
    x = _c(x_bits, np.uint16)
    M, N = A.shape
    y = np.empty(M, np.float32)
    lib().lo_gemv_f16_f32(_p(A), _p(x), _p(y), M, N, N)
    return y


def dot_product_fp16_fp32(a_bits, b_bits, size, num_vectors, stride) -> np.ndarray:
    """dot_product_fp16_fp32 over flat f16 bit arrays (stride in elements)."""
    a = _c(a_bits, np.uint16).reshape(-1)
    b = _c(b_bits, np.uint16).reshape(-1)
    if num_vectors > 0:
        need = 2 * (((num_vectors - 1) * stride) // 2) + size  # elements read
        assert a.size >= need and b.size >= need
    out = np.empty(num_vectors, np.float32)
    lib().lo_dot_product_fp16_fp32(_p(a), _p(b), _p(out), size, num_vectors, stride)
    return out


# --------------------------------------------------------------------------- grouped
def matmul_nax_grouped(W, scale, act, gs, coding=NIBBLE_OFFSET_BINARY) -> np.ndarray:
    """out[M, N] = dequant(W)[M, K] @ act[K, N] (quantized_nax.wgsl:568-626)."""
    W = _c(W, np.uint32)
    scale = _c(scale, np.float32)
    act = _c(act, np.float32)
    M = W.shape[0]
    K = W.shape[1] * 8
    N = act.shape[1]
    assert act.shape[0] == K and scale.size == M * K // gs
    out = np.empty((M, N), np.float32)
    lib().lo_matmul_nax_grouped(_p(W), _p(scale), _p(act), _p(out), M, N, K, gs, coding)
    return out


def matmul_nax_grouped_tokens(W, scale, X, gs, coding=NIBBLE_OFFSET_BINARY) -> np.ndarray:
    """Token-major form: Y[m, n] for X[m, K] (transposes around the reference layout)."""
    act = np.ascontiguousarray(np.asarray(X, np.float32).T)
    return np.ascontiguousarray(matmul_nax_grouped(W, scale, act, gs, coding).T)


def dequantize_int4(W, scale, gs, coding=NIBBLE_OFFSET_BINARY) -> np.ndarray:
    W = _c(W, np.uint32)
    scale = _c(scale, np.float32)
    out = np.empty(W.size * 8, np.float32)
    lib().lo_dequantize_nax_int4_sym(_p(W), _p(scale), _p(out), out.size, gs, coding)
    return out.reshape(W.shape[:-1] + (W.shape[-1] * 8,))


def dequantize_int8(W, scale, gs) -> np.ndarray:
    W = _c(W, np.int8)
    scale = _c(scale, np.float32)
    out = np.empty(W.size, np.float32)
    lib().lo_dequantize_nax_int8_group(_p(W), _p(scale), _p(out), out.size, gs)
    return out.reshape(W.shape)


def matmul_int8_dequant(W, scale, act, gs) -> np.ndarray:
    W = _c(W, np.int8)
    scale = _c(scale, np.float32)
    act = _c(act, np.float32)
    M, K = W.shape
    N = act.shape[1]
    out = np.empty((M, N), np.float32)
    lib().lo_matmul_int8_dequant(_p(W), _p(scale), _p(act), _p(out), M, N, K, gs)
    return out


def matmul_int8_dequant_tokens(W, scale, X, gs) -> np.ndarray:
    act = np.ascontiguousarray(np.asarray(X, np.float32).T)
    return np.ascontiguousarray(matmul_int8_dequant(W, scale, act, gs).T)


# --------------------------------------------------------------------------- integer
def matmul_int4_int8(W, act, coding=NIBBLE_TWOS_COMPLEMENT) -> np.ndarray:
    """out[M, N] i32 = w4[M, K] @ a8[K, N] (quantized.wgsl:590-647)."""
    W = _c(W, np.uint32)
    act = _c(act, np.int8)
    M = W.shape[0]
    K = W.shape[1] * 8
    N = act.shape[1]
    out = np.empty((M, N), np.int32)
    lib().lo_matmul_int4_int8(_p(W), _p(act), _p(out), M, N, K, coding)
    return out


def matmul_int8(A, B) -> np.ndarray:
    A = _c(A, np.int8)
    B = _c(B, np.int8)
    M, K = A.shape
    N = B.shape[1]
    out = np.empty((M, N), np.int32)
    lib().lo_matmul_int8(_p(A), _p(B), _p(out), M, N, K)
    return out


def requantize_int32_to_int8(x, in_scale, out_scale, out_zp=0) -> np.ndarray:
    x = _c(x, np.int32)
    out = np.empty(x.shape, np.int32)
    lib().lo_requantize_int32_to_int8(_p(x), _p(out), x.size, float(in_scale),
                                      float(out_scale), int(out_zp))
    return out


def channel_scales(scale, zero_point=None) -> np.ndarray:
    """PerChannelScale array (quantized.wgsl:51-56): [C, 4] u32 words {f32 scale, i32
    zero_point, 0, 0}."""
    scale = np.asarray(scale, np.float32).ravel()
    zp = np.zeros(scale.size, np.int32) if zero_point is None else np.asarray(zero_point, np.int32).ravel()
    out = np.zeros((scale.size, 4), np.uint32)
    out[:, 0] = scale.view(np.uint32)
    out[:, 1] = zp.view(np.uint32)
    return out


def quantize_int8_per_channel(x, channels, stride, quant_type=0) -> np.ndarray:
    """quantize_int8_per_channel (quantized.wgsl:264-280): i32 per element."""
    x = _c(x, np.float32)
    ch = _c(channels, np.uint32)
    assert ch.shape[-1] == 4 and ch.shape[0] >= -(-x.size // stride)
    out = np.empty(x.shape, np.int32)
    lib().lo_quantize_int8_per_channel(_p(x), _p(ch), _p(out), x.size, int(stride), int(quant_type))
    return out


def dequantize_int8_per_channel(q, channels, stride, quant_type=0) -> np.ndarray:
    """dequantize_int8_per_channel (quantized.wgsl:282-297): f32 per element."""
    q = _c(q, np.int32)
    ch = _c(channels, np.uint32)
    assert ch.shape[-1] == 4 and ch.shape[0] >= -(-q.size // stride)
    out = np.empty(q.shape, np.float32)
    lib().lo_dequantize_int8_per_channel(_p(q), _p(ch), _p(out), q.size, int(stride), int(quant_type))
    return out


def w4a8_group_partials(W, A, gs, coding=NIBBLE_TWOS_COMPLEMENT) -> np.ndarray:
    """P[m, n, g] int32 for token-major A[m, K] int8."""
    W = _c(W, np.uint32)
    A = _c(A, np.int8)
    n_out = W.shape[0]
    K = W.shape[1] * 8
    M = A.shape[0]
    P = np.empty((M, n_out, K // gs), np.int32)
    lib().lo_w4a8_group_partials(_p(W), _p(A), _p(P), n_out, M, K, gs, coding)
    return P


# --------------------------------------------------------------------------- producers
def compute_group_scales(x, gs, fmt=NAX_INT4_SYM):
    x = _c(x, np.float32).reshape(-1)
    ng = (x.size + gs - 1) // gs
    s = np.empty(ng, np.float32)
    zp = np.empty(ng, np.int32)
    mn = np.empty(ng, np.float32)
    mx = np.empty(ng, np.float32)
    lib().lo_compute_group_scales(_p(x), x.size, gs, fmt, _p(s), _p(zp), _p(mn), _p(mx))
    return s, zp, mn, mx


def quantize_int4_sym(x, gs, scale) -> np.ndarray:
    x = _c(x, np.float32)
    scale = _c(scale, np.float32)
    out = np.empty((x.size + 7) // 8, np.uint32)
    lib().lo_quantize_nax_int4_sym(_p(x.reshape(-1)), x.size, gs, _p(scale), _p(out))
    return out


def quantize_int8_group(x, gs, scale) -> np.ndarray:
    x = _c(x, np.float32)
    scale = _c(scale, np.float32)
    out = np.empty((x.size + 3) // 4, np.uint32)
    lib().lo_quantize_nax_int8_group(_p(x.reshape(-1)), x.size, gs, _p(scale), _p(out))
    return out


# --------------------------------------------------------------------------- epilogues
EPI_NONE, EPI_RELU, EPI_GELU, EPI_SILU, EPI_TANH, EPI_SIGMOID, EPI_ADD_BIAS, EPI_ADD_RESIDUAL = range(8)


def apply_epilogue(y, kind, bias=None, residual=None) -> np.ndarray:
    """apply_epilogue of steel_gemm_fused.wgsl:96-127 on y [m, n] (float32 copy)."""
    y = np.array(y, np.float32, order="C", copy=True)
    m, n = y.shape
    b = _c(bias, np.float32) if bias is not None else np.zeros(1, np.float32)
    r = _c(residual, np.float32) if residual is not None else np.zeros(1, np.float32)
    lib().lo_apply_epilogue(_p(y), m, n, int(kind), _p(b), _p(r))
    return y


def silu_mul(gu) -> np.ndarray:
    """silu(gate) * up for gu [m, 2N] (steel_gemm_fused.wgsl:541-555)."""
    gu = _c(gu, np.float32)
    m, n2 = gu.shape
    out = np.empty((m, n2 // 2), np.float32)
    lib().lo_silu_mul(_p(gu), _p(out), m, n2 // 2)
    return out


def rms_norm(x, gamma, eps=1e-6):
    """rms_norm.wgsl on x [rows, hidden] (float32); returns (y, rms per row)."""
    x = _c(x, np.float32)
    rows, hidden = x.shape
    g = _c(gamma, np.float32)
    y = np.empty_like(x)
    r = np.empty(rows, np.float32)
    lib().lo_rms_norm(_p(x), _p(g), _p(y), _p(r), rows, hidden, float(eps))
    return y, r


# --------------------------------------------------------------------------- ground truth
def qmatmul_f64(W, scale, X, gs, wbits, coding=NIBBLE_OFFSET_BINARY) -> np.ndarray:
    """Y[m, n] = sum_k (q*s)(n, k) * X[m, k] in double; token-major X and Y."""
    X = _c(X, np.float32)
    scale = _c(scale, np.float32)
    if wbits == 4:
        W = _c(W, np.uint32)
        n_out, K = W.shape[0], W.shape[1] * 8
    else:
        W = _c(W, np.int8)
        n_out, K = W.shape
    M = X.shape[0]
    Y = np.empty((M, n_out), np.float64)
    lib().lo_qmatmul_f64(_p(W), _p(scale), _p(X), _p(Y), n_out, K, M, gs, wbits, coding)
    return Y


def num_threads() -> int:
    return int(lib().lo_num_threads())
