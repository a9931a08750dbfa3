"""CPU checks of the drop-in boundary: the plugin loads, exports exactly what the
headers declare, and lux_gpu_backend_init fills the descriptor like the reference
(src/webgpu_plugin.cpp:4129-4152).  No compute call is made here."""
import ctypes
import os
import subprocess

import pytest

import webgpu_amd as W


def test_library_exists_and_loads():
    assert os.path.exists(W.LIB_PATH), "run __graft_entry__.build() first"
    W.load_library()


def test_exports_match_headers():
    declared = set(W.header_exports())
    out = subprocess.run(["nm", "-D", "--defined-only", W.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert declared, "no declarations found"
    assert declared <= exported, f"declared but not exported: {declared - exported}"
    extra = {s for s in exported - declared if s.startswith("lux_")}
    assert not extra, f"exported but not declared: {extra}"


def test_backend_init_descriptor():
    p = W.Plugin()
    d = p.desc
    assert d.abi_version == W.LUX_GPU_BACKEND_ABI_VERSION
    assert d.vtbl_size == ctypes.sizeof(W.Vtbl) == 65 * ctypes.sizeof(ctypes.c_void_p)
    assert d.backend_name == b"hip"
    assert d.capabilities == W.LUX_CAP_TENSOR_OPS | W.LUX_CAP_MATMUL
    vt = d.vtbl.contents
    filled = {n for n in W.VTBL_SLOTS if getattr(vt, n)}
    assert filled == {"create_context", "destroy_context", "get_device_count", "get_device_info",
                      "sync", "buffer_alloc", "buffer_alloc_with_data", "buffer_free",
                      "buffer_copy_to_host", "buffer_copy_from_host", "buffer_get_host_ptr",
                      "op_add_f32", "op_sub_f32", "op_mul_f32", "op_div_f32", "op_matmul_f32"}
    # init(NULL) must fail cleanly
    assert not p.lib.lux_gpu_backend_init(None)


def test_null_arguments_rejected():
    p = W.Plugin()
    L = p.lib
    d = W.qdesc(16, 64, 1)
    assert L.lux_hip_qmatmul(None, ctypes.byref(d), None, None, None, None, None) == \
        W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    assert L.lux_hip_gemv_f32(None, None, None, None, None) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    assert p.vt_matmul(None, None, None, None, 4, 4, 4) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    for op in ("add", "sub", "mul", "div"):
        assert p.vt_binary[op](None, None, None, None, 4) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    assert L.lux_hip_rms_norm(None, None, None, None, None, None) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    assert p.vt_count(None) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    assert p.vt_info(None, None) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    assert L.lux_hip_context_set_synchronous(None, 1) == W.LUX_BACKEND_ERROR_INVALID_ARGUMENT
    assert L.lux_hip_buffer_wrap(None, None, 0) is None
    assert L.lux_hip_buffer_device_ptr(None) is None
    assert L.lux_hip_quant_api_version() == 5
    assert "NULL" in p.last_error() or p.last_error() != ""


def test_no_device_behaviour():
    """Without a GPU: zero devices, create_context returns NULL (core falls back)."""
    p = W.Plugin()
    if p.device_count() > 0:
        pytest.skip("a HIP device is visible")
    assert p.vt_create(0) is None
    assert "device" in p.last_error()


def test_c_loader_compiles_as_c11():
    """The headers serve a plain C caller: tests/c_loader builds with gcc -std=c11 -pedantic
    -Werror against include/ alone (no HIP headers), and links only libdl."""
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_loader")
    subprocess.run(["make", "-B", "-C", here], check=True, capture_output=True)
    exe = os.path.join(here, "lux_loader_check")
    assert os.access(exe, os.X_OK)
    out = subprocess.run(["nm", "-D", "--undefined-only", exe], capture_output=True, text=True,
                         check=True).stdout
    assert "hip" not in out.lower()
    usage = subprocess.run([exe], capture_output=True, text=True)
    assert usage.returncode == 2 and "usage" in usage.stderr
