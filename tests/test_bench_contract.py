"""CPU: the parts of bench.py's contract that need no GPU.  More than one GPU is refused
with a message and a non-zero exit before anything touches a device; the algorithmic
byte counts the roofline divides by are the shapes' own arithmetic."""
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU only" in p.stderr and p.stdout == ""


def test_algorithmic_bytes():
    # config 2: nibbles + fp16 g32 scales + fp16 x + fp16 y
    assert bench.C2_BYTES == 14336 * 4096 // 2 + 14336 * 128 * 2 + 4096 * 2 + 14336 * 2 == 33_067_008
    assert bench.C1_BYTES == 67_141_632
    assert bench.c3_bytes(8) == 28672 * 8192 + 28672 * 2 + 8 * 8192 * 2 + 8 * 28672 * 2 == 235_528_192
    assert bench.C4_FLOPS == 240_518_168_576
    assert bench.GB_BYTES == 135_299_072 and bench.GT_BYTES == 67_141_632 and bench.GH_BYTES == 117_506_048
    assert bench.DQ_BYTES == bench.QW_BYTES == 267_911_168
