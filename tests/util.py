"""Shared generators and comparison helpers for the parity tests.

Inputs follow the distributions of BASELINE.json's configs and are produced with
numpy's seeded PCG64 so the HIP path, the oracle and the CPU baseline see the same
bytes.  Packing here is vectorised numpy; the oracle's own codecs are pinned
separately in test_oracle.py.
"""
from __future__ import annotations

import numpy as np

# Tolerances stated for fp paths with fp32 accumulation: rel-L2 <= 1e-3 and
# max-abs <= 1e-2 * ||ref||_inf, after rounding the reference to the output dtype.
REL_L2_TOL = 1e-3
MAX_ABS_FRAC = 1e-2


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def pack_nibbles(q: np.ndarray, coding: int = 0) -> np.ndarray:
    """q int in [-8, 7], shape [n, K] -> u32 [n, K/8]; value i of a word in bits 4i..4i+3.
    coding 0: offset-binary (q + 8); 1: two's complement (q & 0xF)."""
    q = np.asarray(q, np.int64)
    nib = (q + 8) if coding == 0 else (q & 0xF)
    nib = nib.astype(np.uint32).reshape(q.shape[:-1] + (q.shape[-1] // 8, 8))
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    return np.bitwise_or.reduce(nib << shifts, axis=-1).astype(np.uint32)


def unpack_nibbles(w: np.ndarray, coding: int = 0) -> np.ndarray:
    w = np.asarray(w, np.uint32)
    nib = (w[..., None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF
    nib = nib.astype(np.int64)
    q = nib - 8 if coding == 0 else np.where(nib >= 8, nib - 16, nib)
    return q.reshape(w.shape[:-1] + (w.shape[-1] * 8,))


def f16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round-nearest-even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to(y: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 results to the output dtype (RNE) and widen back to float64."""
    y = np.asarray(y, np.float32)
    if dtype == "f16":
        return y.astype(np.float16).astype(np.float64)
    if dtype == "bf16":
        return bf16_to_f32(bf16_bits(y)).astype(np.float64)
    return y.astype(np.float64)


def compare(got, ref, what: str = "", rel_tol: float = REL_L2_TOL,
            abs_frac: float = MAX_ABS_FRAC) -> dict:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    den = np.linalg.norm(ref)
    rel = float(np.linalg.norm(got - ref) / den) if den > 0 else float(np.linalg.norm(got))
    linf = float(np.abs(ref).max()) if ref.size else 0.0
    mabs = float(np.abs(got - ref).max()) if ref.size else 0.0
    assert rel <= rel_tol, f"{what}: rel-L2 {rel:.3e} > {rel_tol:.1e}"
    assert mabs <= abs_frac * max(linf, 1e-30) or ref.size == 0, \
        f"{what}: max-abs {mabs:.3e} > {abs_frac:.0e}*{linf:.3e}"
    return {"rel_l2": rel, "max_abs": mabs, "ref_inf": linf}


# ---------------------------------------------------------------- config inputs
def int4_weights(r: np.random.Generator, n_out: int, K: int, gs: int, coding: int = 0,
                 scale_lo: float = 0.005, scale_hi: float = 0.02):
    """q uniform in [-8, 7] (stored offset-binary or two's complement), fp16 scales."""
    q = r.integers(0, 16, size=(n_out, K), dtype=np.int64) - 8
    W = pack_nibbles(q, coding)
    s = r.uniform(scale_lo, scale_hi, size=(n_out, K // gs)).astype(np.float16)
    return q, W, s


def int8_weights(r: np.random.Generator, n_out: int, K: int):
    q = r.integers(-127, 128, size=(n_out, K), dtype=np.int64).astype(np.int8)
    s = r.uniform(0.001, 0.01, size=(n_out, 1)).astype(np.float16)
    return q, s


def quantize_rows_int8(a: np.ndarray):
    """Per-row symmetric int8: s = max|row|/127, q = clamp(rint(a/s), -128, 127)
    (compute_group_scales NAX_INT8_SYM + quantize_nax_int8_group with gs = K,
    quantized_nax.wgsl:204-212, 336-362)."""
    a = np.asarray(a, np.float32)
    s = (np.abs(a).max(axis=1) / np.float32(127.0)).astype(np.float32)
    s = np.where(s == 0, np.float32(1.0), s).astype(np.float32)
    q = np.clip(np.rint(a / s[:, None]), -128, 127).astype(np.int8)
    return q, s
