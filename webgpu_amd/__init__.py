"""Python mirror of the Lux GPU plugin boundary for libluxgpu_backend_hip.so.

The product is the C-ABI shared library built from ``webgpu_amd/csrc`` (HIP for
gfx950).  This module only binds it with ctypes the way luxcpp/gpu's loader does
(dlopen + ``lux_gpu_backend_init`` + vtable, reference docs/architecture.md:89-107),
plus the quantized entry points of ``include/lux/gpu/hip_quant.h``.  It never
computes anything itself: if the library is missing the import of a context
raises instead of falling back.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import (CFUNCTYPE, POINTER, Structure, byref, c_bool, c_char_p, c_float, c_int,
                    c_int32, c_size_t, c_uint32, c_uint64, c_void_p)

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_NAME = "libluxgpu_backend_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")

# ---- LuxBackendError (include/lux/gpu/backend_plugin.h) ----
LUX_BACKEND_OK = 0
LUX_BACKEND_ERROR_INVALID_ARGUMENT = 1
LUX_BACKEND_ERROR_OUT_OF_MEMORY = 2
LUX_BACKEND_ERROR_NOT_SUPPORTED = 3
LUX_BACKEND_ERROR_DEVICE_LOST = 4
LUX_BACKEND_ERROR_INTERNAL = 5
ERROR_NAMES = {0: "OK", 1: "INVALID_ARGUMENT", 2: "OUT_OF_MEMORY", 3: "NOT_SUPPORTED",
               4: "DEVICE_LOST", 5: "INTERNAL"}

LUX_GPU_BACKEND_ABI_VERSION = 3
LUX_CAP_TENSOR_OPS = 1 << 0
LUX_CAP_MATMUL = 1 << 1

# ---- hip_quant.h enums ----
F32, F16, BF16, I32, I8, I4 = 0, 1, 2, 3, 32, 33
NIBBLE_OFFSET_BINARY, NIBBLE_TWOS_COMPLEMENT = 0, 1
SCALE_NONE, SCALE_F16, SCALE_F32, SCALE_GROUPSCALE = 0, 1, 2, 3
QFLAG_GROUP_PARTIALS = 1
QFLAG_QUANTIZE_X = 2
(EPI_NONE, EPI_RELU, EPI_GELU, EPI_SILU, EPI_TANH, EPI_SIGMOID, EPI_ADD_BIAS, EPI_ADD_RESIDUAL,
 EPI_SILU_MUL) = range(9)


class LuxError(RuntimeError):
    def __init__(self, code: int, where: str, msg: str = ""):
        self.code = code
        super().__init__(f"{where}: {ERROR_NAMES.get(code, code)}" + (f" ({msg})" if msg else ""))


class DeviceInfo(Structure):
    _fields_ = [("name", c_char_p), ("vendor", c_char_p), ("memory_total", c_uint64),
                ("memory_available", c_uint64), ("compute_units", c_int),
                ("max_workgroup_size", c_int), ("is_discrete", c_bool),
                ("is_unified_memory", c_bool)]


_FN = c_void_p  # every vtable slot is one function pointer
VTBL_SLOTS = [
    "create_context", "destroy_context", "get_device_count", "get_device_info", "sync",
    "buffer_alloc", "buffer_alloc_with_data", "buffer_free", "buffer_copy_to_host",
    "buffer_copy_from_host", "buffer_get_host_ptr",
    "op_add_f32", "op_sub_f32", "op_mul_f32", "op_div_f32", "op_matmul_f32", "op_transpose_f32",
    "op_reduce_sum_f32", "op_reduce_max_f32", "op_reduce_min_f32", "op_reduce_mean_f32",
    "op_reduce_sum_axis_f32", "op_reduce_max_axis_f32", "op_softmax_f32", "op_log_softmax_f32",
    "op_exp_f32", "op_log_f32", "op_sqrt_f32", "op_neg_f32", "op_abs_f32", "op_tanh_f32",
    "op_sigmoid_f32", "op_relu_f32", "op_gelu_f32", "op_copy_f32", "op_layer_norm_f32",
    "op_rms_norm_f32",
    "op_ntt_forward", "op_ntt_inverse", "op_poly_mul", "op_tfhe_bootstrap", "op_tfhe_keyswitch",
    "op_blind_rotate",
    "op_poseidon2_hash", "op_blake3_hash", "op_keccak256_hash", "op_bls12_381_add",
    "op_bls12_381_mul", "op_bls12_381_pairing", "op_bn254_add", "op_bn254_mul", "op_msm",
    "op_kzg_commit", "op_kzg_open", "op_kzg_verify",
    "op_ecrecover_batch", "op_mldsa_verify_batch", "op_mlkem_decapsulate_batch",
    "op_slhdsa_verify_batch", "op_ringtail_partial_sign_batch", "op_ringtail_combine_batch",
    "op_frost_partial_verify_batch", "op_cggmp21_partial_sign_batch",
    "op_ed25519_verify_batch", "op_sr25519_verify_batch",
]


class Vtbl(Structure):
    _fields_ = [(n, _FN) for n in VTBL_SLOTS]


class BackendDesc(Structure):
    _fields_ = [("abi_version", c_uint32), ("vtbl_size", c_uint32), ("backend_name", c_char_p),
                ("backend_version", c_char_p), ("capabilities", c_uint32),
                ("vtbl", POINTER(Vtbl))]


class QMatmulDesc(Structure):
    _fields_ = [("struct_size", c_uint32), ("n_out", c_int32), ("k", c_int32), ("m", c_int32),
                ("weight_bits", c_int32), ("group_size", c_int32), ("nibble_coding", c_int32),
                ("scale_format", c_int32), ("x_dtype", c_int32), ("y_dtype", c_int32),
                ("flags", c_int32)]


class QuantizeDesc(Structure):
    _fields_ = [("struct_size", c_uint32), ("rows", c_int32), ("k", c_int32),
                ("weight_bits", c_int32), ("group_size", c_int32), ("nibble_coding", c_int32),
                ("scale_format", c_int32), ("x_dtype", c_int32)]


class RmsNormParams(Structure):
    _fields_ = [("batch_size", c_uint32), ("hidden_size", c_uint32), ("eps", c_float),
                ("x_dtype", c_int32), ("y_dtype", c_int32)]


class GemvParams(Structure):
    _fields_ = [("M", c_uint32), ("N", c_uint32), ("alpha", c_float), ("beta", c_float),
                ("lda", c_uint32), ("trans", c_uint32), ("_pad0", c_uint32), ("_pad1", c_uint32)]


class DotParams(Structure):
    _fields_ = [("size", c_uint32), ("num_vectors", c_uint32), ("vector_stride", c_uint32),
                ("_pad", c_uint32)]


class GemvBatchedParams(Structure):
    _fields_ = [("M", c_uint32), ("N", c_uint32), ("alpha", c_float), ("beta", c_float),
                ("lda", c_uint32), ("batch_count", c_uint32), ("stride_a", c_uint32),
                ("stride_x", c_uint32), ("stride_y", c_uint32), ("_pad0", c_uint32),
                ("_pad1", c_uint32), ("_pad2", c_uint32)]


# Typed views of the vtable slots this plugin fills.
_T_CREATE = CFUNCTYPE(c_void_p, c_int)
_T_DESTROY = CFUNCTYPE(None, c_void_p)
_T_COUNT = CFUNCTYPE(c_int, POINTER(c_int))
_T_INFO = CFUNCTYPE(c_int, c_void_p, POINTER(DeviceInfo))
_T_SYNC = CFUNCTYPE(c_int, c_void_p)
_T_ALLOC = CFUNCTYPE(c_void_p, c_void_p, c_size_t)
_T_ALLOC_DATA = CFUNCTYPE(c_void_p, c_void_p, c_void_p, c_size_t)
_T_FREE = CFUNCTYPE(None, c_void_p, c_void_p)
_T_COPY = CFUNCTYPE(c_int, c_void_p, c_void_p, c_void_p, c_size_t)
_T_HOSTPTR = CFUNCTYPE(c_void_p, c_void_p, c_void_p)
_T_MATMUL = CFUNCTYPE(c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int)
_T_BINARY = CFUNCTYPE(c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t)

EXPORTS = {
    "lux_gpu_backend_init": (c_bool, [POINTER(BackendDesc)]),
    "lux_hip_qmatmul": (c_int, [c_void_p, POINTER(QMatmulDesc), c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p]),
    "lux_hip_qmatmul_ex": (c_int, [c_void_p, POINTER(QMatmulDesc), c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "lux_hip_qmatmul_noalloc": (c_int, [c_void_p, POINTER(QMatmulDesc), c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "lux_hip_rms_norm": (c_int, [c_void_p, POINTER(RmsNormParams), c_void_p, c_void_p, c_void_p,
                                 c_void_p]),
    "lux_hip_rms_norm_qmatmul": (c_int, [c_void_p, POINTER(RmsNormParams), c_void_p,
                                         POINTER(QMatmulDesc), c_void_p, c_void_p, c_void_p, c_int,
                                         c_void_p, c_void_p, c_void_p]),
    "lux_hip_quantize": (c_int, [c_void_p, POINTER(QuantizeDesc), c_void_p, c_void_p, c_void_p]),
    "lux_hip_dequantize": (c_int, [c_void_p, POINTER(QuantizeDesc), c_void_p, c_void_p, c_void_p]),
    "lux_hip_convert_nibbles": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_int, c_int]),
    "lux_hip_convert_scales": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int, c_size_t]),
    "lux_hip_requantize_i32": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_float, c_float,
                                       c_int32]),
    "lux_hip_quantize_int8_per_channel": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                                  c_uint32, c_uint32]),
    "lux_hip_dequantize_int8_per_channel": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                                    c_uint32, c_uint32]),
    "lux_hip_gemv_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, POINTER(GemvParams)]),
    "lux_hip_gemv_f32_batched": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                         POINTER(GemvBatchedParams)]),
    "lux_hip_dot_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, POINTER(DotParams)]),
    "lux_hip_pack_int4_host": (c_int, [c_void_p, c_size_t, c_int, c_void_p]),
    "lux_hip_unpack_int4_host": (c_int, [c_void_p, c_size_t, c_int, c_void_p]),
    "lux_hip_convert_scales_host": (c_int, [c_void_p, c_int, c_void_p, c_int, c_size_t]),
    "lux_hip_gemv_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                 c_uint32]),
    "lux_hip_buffer_wrap": (c_void_p, [c_void_p, c_void_p, c_size_t]),
    "lux_hip_buffer_device_ptr": (c_void_p, [c_void_p]),
    "lux_hip_buffer_size": (c_size_t, [c_void_p]),
    "lux_hip_context_set_stream": (c_int, [c_void_p, c_void_p]),
    "lux_hip_context_get_stream": (c_void_p, [c_void_p]),
    "lux_hip_context_set_synchronous": (c_int, [c_void_p, c_int]),
    "lux_hip_last_error": (c_char_p, []),
    "lux_hip_quant_api_version": (c_uint32, []),
}


def header_exports() -> list[str]:
    """Every function name declared in include/lux/gpu/*.h."""
    import re
    names = []
    inc = os.path.join(REPO_DIR, "include", "lux", "gpu")
    for fn in sorted(os.listdir(inc)):
        if fn.endswith(".h"):
            txt = open(os.path.join(inc, fn)).read()
            names += re.findall(r"^[A-Za-z_][\w \*]*?\b(lux_\w+)\s*\(", txt, re.M)
    return sorted(set(names))


def build(force: bool = True, jobs: int = 8) -> str:
    """Compile the HIP plugin for gfx950 with csrc/Makefile (in-tree)."""
    cmd = ["make", "-C", CSRC_DIR, f"-j{jobs}"] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


_lib = None


def load_library(path: str | None = None):
    """dlopen the plugin (no fallback: a missing library is an error)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise FileNotFoundError(f"{p} not built; run __graft_entry__.build() or make -C {CSRC_DIR}")
    L = ctypes.CDLL(p, mode=ctypes.RTLD_LOCAL)
    for name, (res, args) in EXPORTS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = L
    return L


class Buffer:
    """A LuxBackendBuffer handle (owned unless wrapped)."""

    def __init__(self, ctx: "Context", handle: int, nbytes: int, keepalive=None):
        self.ctx = ctx
        self.handle = handle
        self.nbytes = nbytes
        self._keep = keepalive

    @property
    def ptr(self) -> int:
        return self.ctx.plugin.lib.lux_hip_buffer_device_ptr(self.handle) or 0

    def free(self):
        if self.handle:
            self.ctx.plugin.vt_free(self.ctx.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            if self.handle and self.ctx.handle:
                self.free()
        except Exception:
            pass


class Plugin:
    """The loaded backend: descriptor + typed vtable slots."""

    def __init__(self, path: str | None = None):
        self.lib = load_library(path)
        self.desc = BackendDesc()
        if not self.lib.lux_gpu_backend_init(byref(self.desc)):
            raise LuxError(LUX_BACKEND_ERROR_INTERNAL, "lux_gpu_backend_init")
        if self.desc.vtbl_size != ctypes.sizeof(Vtbl):
            raise LuxError(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "vtbl_size",
                           f"{self.desc.vtbl_size} != {ctypes.sizeof(Vtbl)}")
        vt = self.desc.vtbl.contents
        self.vtbl = vt
        self.vt_create = _T_CREATE(vt.create_context)
        self.vt_destroy = _T_DESTROY(vt.destroy_context)
        self.vt_count = _T_COUNT(vt.get_device_count)
        self.vt_info = _T_INFO(vt.get_device_info)
        self.vt_sync = _T_SYNC(vt.sync)
        self.vt_alloc = _T_ALLOC(vt.buffer_alloc)
        self.vt_alloc_data = _T_ALLOC_DATA(vt.buffer_alloc_with_data)
        self.vt_free = _T_FREE(vt.buffer_free)
        self.vt_to_host = _T_COPY(vt.buffer_copy_to_host)
        self.vt_from_host = _T_COPY(vt.buffer_copy_from_host)
        self.vt_host_ptr = _T_HOSTPTR(vt.buffer_get_host_ptr)
        self.vt_matmul = _T_MATMUL(vt.op_matmul_f32)
        self.vt_binary = {op: _T_BINARY(getattr(vt, f"op_{op}_f32")) for op in ("add", "sub", "mul", "div")}

    def device_count(self) -> int:
        n = c_int(-1)
        self.check(self.vt_count(byref(n)), "get_device_count")
        return n.value

    def last_error(self) -> str:
        s = self.lib.lux_hip_last_error()
        return s.decode() if s else ""

    def check(self, code: int, where: str):
        if code != LUX_BACKEND_OK:
            raise LuxError(code, where, self.last_error())

    def create_context(self, device: int = 0) -> "Context":
        h = self.vt_create(device)
        if not h:
            raise LuxError(LUX_BACKEND_ERROR_NOT_SUPPORTED, "create_context", self.last_error())
        return Context(self, h)


class Context:
    def __init__(self, plugin: Plugin, handle: int):
        self.plugin = plugin
        self.handle = handle
        self.lib = plugin.lib

    def close(self):
        if self.handle:
            self.plugin.vt_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # -- device
    def info(self) -> DeviceInfo:
        inf = DeviceInfo()
        self.plugin.check(self.plugin.vt_info(self.handle, byref(inf)), "get_device_info")
        return inf

    def sync(self):
        self.plugin.check(self.plugin.vt_sync(self.handle), "sync")

    def set_stream(self, stream: int | None):
        self.plugin.check(self.lib.lux_hip_context_set_stream(self.handle, stream or None),
                          "set_stream")

    def set_synchronous(self, on: bool):
        self.plugin.check(self.lib.lux_hip_context_set_synchronous(self.handle, int(on)),
                          "set_synchronous")

    # -- buffers
    def alloc(self, nbytes: int) -> Buffer:
        h = self.plugin.vt_alloc(self.handle, nbytes)
        if not h:
            raise LuxError(LUX_BACKEND_ERROR_OUT_OF_MEMORY, "buffer_alloc", self.plugin.last_error())
        return Buffer(self, h, nbytes)

    def upload(self, arr: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(arr)
        h = self.plugin.vt_alloc_data(self.handle, a.ctypes.data_as(c_void_p), a.nbytes)
        if not h:
            raise LuxError(LUX_BACKEND_ERROR_OUT_OF_MEMORY, "buffer_alloc_with_data",
                           self.plugin.last_error())
        return Buffer(self, h, a.nbytes)

    def download(self, buf: Buffer, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        self.plugin.check(self.plugin.vt_to_host(self.handle, buf.handle,
                                                 out.ctypes.data_as(c_void_p), out.nbytes),
                          "buffer_copy_to_host")
        return out

    def wrap(self, tensor) -> Buffer:
        """Wrap a torch CUDA tensor's memory (the tensor is kept alive)."""
        nbytes = tensor.numel() * tensor.element_size()
        h = self.lib.lux_hip_buffer_wrap(self.handle, tensor.data_ptr(), nbytes)
        if not h:
            raise LuxError(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "buffer_wrap", self.plugin.last_error())
        return Buffer(self, h, nbytes, keepalive=tensor)

    # -- ops
    def binary_f32(self, op: str, a: Buffer, b: Buffer, out: Buffer, n: int):
        """op_add_f32 / op_sub_f32 / op_mul_f32 / op_div_f32 through the vtable."""
        self.plugin.check(self.plugin.vt_binary[op](self.handle, a.handle, b.handle, out.handle, n),
                          f"op_{op}_f32")

    def matmul_f32(self, a: Buffer, b: Buffer, out: Buffer, M: int, K: int, N: int):
        self.plugin.check(self.plugin.vt_matmul(self.handle, a.handle, b.handle, out.handle, M, K, N),
                          "op_matmul_f32")

    def gemv_f32(self, a: Buffer, x: Buffer, y: Buffer, M: int, N: int, alpha=1.0, beta=0.0,
                 lda=None, trans=False):
        p = GemvParams(M, N, alpha, beta, lda if lda is not None else N, int(trans), 0, 0)
        self.plugin.check(self.lib.lux_hip_gemv_f32(self.handle, a.handle, x.handle, y.handle,
                                                    byref(p)), "gemv_f32")

    def gemv_f32_batched(self, a: Buffer, x: Buffer, y: Buffer, M: int, N: int, batch: int,
                         stride_a: int, stride_x: int, stride_y: int, alpha=1.0, beta=0.0, lda=None):
        """gemv_batched (gemv.wgsl:297-354); strides and lda in elements."""
        p = GemvBatchedParams(M, N, alpha, beta, lda if lda is not None else N, batch, stride_a,
                              stride_x, stride_y, 0, 0, 0)
        self.plugin.check(self.lib.lux_hip_gemv_f32_batched(self.handle, a.handle, x.handle, y.handle,
                                                            byref(p)), "gemv_f32_batched")

    def dot_f16(self, a: Buffer, b: Buffer, result: Buffer, size: int, num_vectors: int,
                vector_stride: int):
        """dot_product_fp16_fp32 (fp_quantized.wgsl:418-469); stride in elements."""
        p = DotParams(size, num_vectors, vector_stride, 0)
        self.plugin.check(self.lib.lux_hip_dot_f16(self.handle, a.handle, b.handle, result.handle,
                                                   byref(p)), "dot_f16")

    def gemv_f16(self, a: Buffer, x: Buffer, y: Buffer, M: int, N: int, lda=None):
        self.plugin.check(self.lib.lux_hip_gemv_f16(self.handle, a.handle, x.handle, y.handle, M, N,
                                                    lda if lda is not None else N), "gemv_f16")

    def qmatmul(self, desc: QMatmulDesc, w: Buffer, scales: Buffer | None, x: Buffer,
                x_scales: Buffer | None, y: Buffer):
        self.plugin.check(self.lib.lux_hip_qmatmul(self.handle, byref(desc), w.handle,
                                                   scales.handle if scales else None, x.handle,
                                                   x_scales.handle if x_scales else None,
                                                   y.handle), "qmatmul")

    def qmatmul_ex(self, desc: QMatmulDesc, w: Buffer, scales: Buffer | None, x: Buffer,
                   x_scales: Buffer | None, epilogue: int, bias: Buffer | None,
                   residual: Buffer | None, y: Buffer):
        self.plugin.check(self.lib.lux_hip_qmatmul_ex(
            self.handle, byref(desc), w.handle, scales.handle if scales else None, x.handle,
            x_scales.handle if x_scales else None, epilogue, bias.handle if bias else None,
            residual.handle if residual else None, y.handle), "qmatmul_ex")

    def qmatmul_noalloc(self, desc: QMatmulDesc, w: Buffer, scales: Buffer | None, x: Buffer,
                        x_scales: Buffer | None, epilogue: int, bias: Buffer | None,
                        residual: Buffer | None, y: Buffer):
        """lux_hip_qmatmul_ex with the library's fixed per-device scratch (no allocation)."""
        self.plugin.check(self.lib.lux_hip_qmatmul_noalloc(
            self.handle, byref(desc), w.handle, scales.handle if scales else None, x.handle,
            x_scales.handle if x_scales else None, epilogue, bias.handle if bias else None,
            residual.handle if residual else None, y.handle), "qmatmul_noalloc")

    def rms_norm(self, x: Buffer, gamma: Buffer, y: Buffer, rows: int, hidden: int,
                 eps: float = 1e-6, x_dtype: int = F32, y_dtype: int = F32,
                 rms_out: Buffer | None = None):
        p = RmsNormParams(rows, hidden, eps, x_dtype, y_dtype)
        self.plugin.check(self.lib.lux_hip_rms_norm(self.handle, byref(p), x.handle, gamma.handle,
                                                    y.handle, rms_out.handle if rms_out else None),
                          "rms_norm")

    def rms_norm_qmatmul(self, x: Buffer, gamma: Buffer, eps: float, x_dtype: int,
                         desc: QMatmulDesc, w: Buffer, scales: Buffer | None, epilogue: int,
                         bias: Buffer | None, residual: Buffer | None, y: Buffer):
        """lux_hip_rms_norm_qmatmul: rms_norm of x ([desc.m x desc.k], x_dtype) into
        desc.x_dtype, then lux_hip_qmatmul_ex on the normalised rows."""
        p = RmsNormParams(desc.m, desc.k, eps, x_dtype, desc.x_dtype)
        self.plugin.check(self.lib.lux_hip_rms_norm_qmatmul(
            self.handle, byref(p), gamma.handle, byref(desc), w.handle,
            scales.handle if scales else None, x.handle, epilogue, bias.handle if bias else None,
            residual.handle if residual else None, y.handle), "rms_norm_qmatmul")

    def quantize(self, desc: QuantizeDesc, x: Buffer, q: Buffer, scales: Buffer):
        self.plugin.check(self.lib.lux_hip_quantize(self.handle, byref(desc), x.handle, q.handle,
                                                    scales.handle), "quantize")

    def dequantize(self, desc: QuantizeDesc, q: Buffer, scales: Buffer, out: Buffer):
        """out = q * s; desc.x_dtype is the output type (lux_hip_dequantize)."""
        self.plugin.check(self.lib.lux_hip_dequantize(self.handle, byref(desc), q.handle,
                                                      scales.handle, out.handle), "dequantize")

    def convert_nibbles(self, src: Buffer, dst: Buffer, words: int, from_coding: int,
                        to_coding: int):
        self.plugin.check(self.lib.lux_hip_convert_nibbles(self.handle, src.handle, dst.handle,
                                                           words, from_coding, to_coding),
                          "convert_nibbles")

    def convert_scales(self, src: Buffer, in_format: int, dst: Buffer, out_format: int,
                       count: int):
        self.plugin.check(self.lib.lux_hip_convert_scales(self.handle, src.handle, in_format,
                                                          dst.handle, out_format, count),
                          "convert_scales")

    def quantize_int8_per_channel(self, src: Buffer, channel_scales: Buffer, dst: Buffer, size: int,
                                  channel_stride: int, quant_type: int = 0):
        """quantize_int8_per_channel (quantized.wgsl:264-280): f32 -> one i32 per element."""
        self.plugin.check(self.lib.lux_hip_quantize_int8_per_channel(
            self.handle, src.handle, channel_scales.handle, dst.handle, size, channel_stride, quant_type),
            "quantize_int8_per_channel")

    def dequantize_int8_per_channel(self, src: Buffer, channel_scales: Buffer, dst: Buffer, size: int,
                                    channel_stride: int, quant_type: int = 0):
        """dequantize_int8_per_channel (quantized.wgsl:282-297): i32 per element -> f32."""
        self.plugin.check(self.lib.lux_hip_dequantize_int8_per_channel(
            self.handle, src.handle, channel_scales.handle, dst.handle, size, channel_stride, quant_type),
            "dequantize_int8_per_channel")

    def requantize(self, src: Buffer, dst: Buffer, size: int, input_scale: float,
                   output_scale: float, output_zero_point: int = 0):
        self.plugin.check(self.lib.lux_hip_requantize_i32(self.handle, src.handle, dst.handle,
                                                          size, input_scale, output_scale,
                                                          output_zero_point), "requantize")


# --------------------------------------------------------------------------- host packers
def _host_check(L, code: int, where: str):
    if code != LUX_BACKEND_OK:
        raise LuxError(code, where, (L.lux_hip_last_error() or b"").decode())


def pack_int4_host(q, coding: int = 0) -> np.ndarray:
    """lux_hip_pack_int4_host: int4 values (any shape, size % 8 == 0) -> uint32 words."""
    L = load_library()
    qa = np.ascontiguousarray(q, dtype=np.int8).reshape(-1)
    out = np.empty(qa.size // 8, np.uint32)
    _host_check(L, L.lux_hip_pack_int4_host(qa.ctypes.data, qa.size, coding, out.ctypes.data), "pack_int4_host")
    return out


def unpack_int4_host(words, n: int, coding: int = 0) -> np.ndarray:
    """lux_hip_unpack_int4_host: n int4 values (int8) from n / 8 words."""
    L = load_library()
    wa = np.ascontiguousarray(words, dtype=np.uint32).reshape(-1)
    if wa.size * 8 < n:
        raise ValueError("unpack_int4_host: too few words")
    out = np.empty(n, np.int8)
    _host_check(L, L.lux_hip_unpack_int4_host(wa.ctypes.data, n, coding, out.ctypes.data), "unpack_int4_host")
    return out


_SCALE_NP = {SCALE_F16: (np.uint16, 1), SCALE_F32: (np.float32, 1), SCALE_GROUPSCALE: (np.uint32, 4)}


def convert_scales_host(scales, in_format: int, out_format: int) -> np.ndarray:
    """lux_hip_convert_scales_host.  F16 as uint16 bits, F32 as float32, GROUPSCALE as
    uint32 [count, 4] records (scale and min/max are float bit patterns)."""
    L = load_library()
    idt, iw = _SCALE_NP[in_format]
    odt, ow = _SCALE_NP[out_format]
    a = np.ascontiguousarray(scales, dtype=idt).reshape(-1)
    count = a.size // iw
    out = np.empty(count * ow, odt)
    _host_check(L, L.lux_hip_convert_scales_host(a.ctypes.data, in_format, out.ctypes.data, out_format, count),
                "convert_scales_host")
    return out.reshape(count, 4) if ow == 4 else out


def quant_desc(rows: int, k: int, weight_bits: int = 4, group_size: int = 32,
               nibble_coding: int = NIBBLE_OFFSET_BINARY, scale_format: int = SCALE_F16,
               x_dtype: int = F32) -> QuantizeDesc:
    return QuantizeDesc(ctypes.sizeof(QuantizeDesc), rows, k, weight_bits, group_size,
                        nibble_coding, scale_format, x_dtype)


def qdesc(n_out: int, k: int, m: int, weight_bits: int = 4, group_size: int = 32,
          nibble_coding: int = NIBBLE_OFFSET_BINARY, scale_format: int = SCALE_F16,
          x_dtype: int = F16, y_dtype: int = F16, flags: int = 0) -> QMatmulDesc:
    return QMatmulDesc(ctypes.sizeof(QMatmulDesc), n_out, k, m, weight_bits, group_size,
                       nibble_coding, scale_format, x_dtype, y_dtype, flags)
