"""GPU parity through a compiled C caller of the boundary.

tests/c_loader/lux_loader_check.c is built with `gcc -std=c11 -I include` and binds the plugin
the way luxcpp/gpu's loader does (docs/architecture.md:89-107: dlopen, dlsym
"lux_gpu_backend_init", abi_version and vtbl_size checks, then the vtable) plus the lux_hip_*
extensions by dlsym.  It runs op_matmul_f32 as lux_tensor_matmul would (a GEMV with N = 1 and
a general GEMM, src/webgpu_plugin.cpp:1721-1771) and an int4 g32 GEMV through lux_hip_qmatmul
(matmul_nax_grouped, quantized_nax.wgsl:568-626), writes the results as raw arrays, and this
test checks them against the oracle.  The program runs in its own process, so no Python binding
is between the caller and the library.
"""
import os
import subprocess

import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import compare, int4_weights, rng, round_to

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
LOADER_DIR = os.path.join(HERE, "c_loader")
LOADER = os.path.join(LOADER_DIR, "lux_loader_check")

# Shapes fixed in lux_loader_check.c.
GM, GK = 1000, 4096
MM, MK, MN = 70, 300, 130
QN, QK, GS = 4096, 4096, 32


def _loader() -> str:
    if not os.path.exists(LOADER):
        subprocess.run(["make", "-C", LOADER_DIR], check=True, stdout=subprocess.DEVNULL)
    return LOADER


def test_c_loader_end_to_end(tmp_path, plugin):
    if plugin.device_count() < 1:
        pytest.skip("no HIP device")
    r = rng(2024)
    gA = (r.standard_normal((GM, GK)) * 0.02).astype(np.float32)
    gx = r.standard_normal(GK).astype(np.float32)
    mA = r.standard_normal((MM, MK)).astype(np.float32)
    mB = r.standard_normal((MK, MN)).astype(np.float32)
    _, qW, qS = int4_weights(r, QN, QK, GS)
    qx = r.standard_normal(QK).astype(np.float16)
    for name, arr in (("gemv_A.f32", gA), ("gemv_x.f32", gx), ("gemm_A.f32", mA),
                      ("gemm_B.f32", mB), ("q_W.u32", qW), ("q_S.f16", qS), ("q_x.f16", qx)):
        np.ascontiguousarray(arr).tofile(str(tmp_path / name))

    print(f"c_loader: {LOADER} {W.LIB_PATH}", flush=True)
    run = subprocess.run([_loader(), W.LIB_PATH, str(tmp_path)], capture_output=True, text=True,
                         timeout=120)
    print(run.stdout, run.stderr, flush=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "PASSED: 0 failed checks" in run.stdout

    y = np.fromfile(str(tmp_path / "gemv_y.f32"), np.float32)
    compare(y, oracle.matmul_f32(gA, gx[:, None])[:, 0], "C loader op_matmul_f32 N=1", rel_tol=1e-5)
    C = np.fromfile(str(tmp_path / "gemm_C.f32"), np.float32).reshape(MM, MN)
    compare(C, oracle.matmul_f32(mA, mB), "C loader op_matmul_f32 GEMM", rel_tol=1e-5)
    qy = np.fromfile(str(tmp_path / "q_y.f16"), np.float16).astype(np.float64)
    ref = oracle.matmul_nax_grouped(qW, qS.astype(np.float32).reshape(-1),
                                    qx.astype(np.float32).reshape(-1, 1), GS)[:, 0]
    compare(qy, round_to(ref, "f16"), "C loader lux_hip_qmatmul int4 GEMV")
