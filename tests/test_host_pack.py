"""CPU: the host packers of the C-ABI library (lux_hip_pack_int4_host,
lux_hip_unpack_int4_host, lux_hip_convert_scales_host).  Host code, no device: they run
in the CPU suite.  Checked exhaustively against the oracle's nibble codec
(pack_nax_int4_sym_x8 / unpack_int4x8, quantized_nax.wgsl:94-112, quantized.wgsl:148-156)
and against numpy's IEEE binary16 conversion (round to nearest even).
"""
import itertools

import numpy as np
import pytest

import oracle
import webgpu_amd as W
from util import rng


def test_int4_pack_exhaustive_against_oracle():
    """Every value at every position, both codings, word for word equal to the oracle."""
    vals = np.arange(-8, 8, dtype=np.int8)
    q = np.zeros((16 * 8, 8), np.int8)
    for i, (v, pos) in enumerate(itertools.product(range(16), range(8))):
        q[i] = vals[(v + np.arange(8) * 5) % 16]  # a different value in every slot
        q[i, pos] = vals[v]
    for coding in (W.NIBBLE_OFFSET_BINARY, W.NIBBLE_TWOS_COMPLEMENT):
        got = W.pack_int4_host(q, coding)
        fn = oracle.lib().lo_pack_int4_ob if coding == W.NIBBLE_OFFSET_BINARY else oracle.lib().lo_pack_int4_tc
        want = np.array([fn(np.ascontiguousarray(row, np.int32).ctypes.data) for row in q], np.uint32)
        assert np.array_equal(got, want)
        assert np.array_equal(W.unpack_int4_host(got, q.size, coding), q.reshape(-1))
    ob = W.pack_int4_host(q, W.NIBBLE_OFFSET_BINARY)
    assert np.array_equal(ob, W.pack_int4_host(q, W.NIBBLE_TWOS_COMPLEMENT) ^ np.uint32(0x88888888))


def test_int4_pack_refusals():
    with pytest.raises(W.LuxError, match="outside"):
        W.pack_int4_host(np.array([0, 1, 2, 3, 8, 0, 0, 0], np.int8))
    with pytest.raises(W.LuxError, match="multiple of 8"):
        W.pack_int4_host(np.zeros(12, np.int8))
    with pytest.raises(W.LuxError, match="coding"):
        W.pack_int4_host(np.zeros(8, np.int8), 5)


def test_scales_f16_exhaustive_and_rne():
    """All 65,536 binary16 patterns widen exactly; binary32 -> binary16 matches numpy's
    RNE for random, subnormal-range, tie, overflow and special values."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    wide = W.convert_scales_host(h, W.SCALE_F16, W.SCALE_F32)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(wide), nan)
    assert np.array_equal(wide[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    r = rng(17)
    f = np.concatenate([
        r.standard_normal(20000).astype(np.float32),
        (r.standard_normal(20000) * 1e-6).astype(np.float32),           # binary16 subnormals
        (r.standard_normal(5000) * 1e-8).astype(np.float32),            # below the least subnormal
        (r.uniform(6e4, 7e4, 5000)).astype(np.float32),                 # around the largest finite
        ((np.arange(4096, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24)),  # ties of subnormals
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, np.inf, -np.inf, 2.0 ** -25,
                  2.0 ** -25 * 1.0000001, 2.0 ** -14, 2.0 ** -14 * (1 - 2 ** -12)], np.float32),
    ])
    got = W.convert_scales_host(f, W.SCALE_F32, W.SCALE_F16)
    with np.errstate(over="ignore"):  # the overflow cases are meant to become inf
        assert np.array_equal(got, f.astype(np.float16).view(np.uint16))
    assert np.isnan(W.convert_scales_host(np.array([np.nan], np.float32), W.SCALE_F32, W.SCALE_F16)
                    .view(np.float16)).all()


def test_scales_groupscale_round_trips():
    """GroupScale records keep all four fields when copied, carry {s, 0, 0, 0} when made
    from F16/F32, and give back their scale."""
    r = rng(18)
    s = r.uniform(0.001, 0.1, 100).astype(np.float32)
    gs = W.convert_scales_host(s, W.SCALE_F32, W.SCALE_GROUPSCALE)
    assert np.array_equal(gs[:, 0].view(np.float32), s) and not gs[:, 1:].any()
    full = np.stack([s.view(np.uint32), np.arange(100, dtype=np.uint32),
                     (-s).view(np.uint32), (2 * s).view(np.uint32)], axis=1)
    assert np.array_equal(W.convert_scales_host(full, W.SCALE_GROUPSCALE, W.SCALE_GROUPSCALE), full)
    assert np.array_equal(W.convert_scales_host(full, W.SCALE_GROUPSCALE, W.SCALE_F32), s)
    assert np.array_equal(W.convert_scales_host(full, W.SCALE_GROUPSCALE, W.SCALE_F16),
                          s.astype(np.float16).view(np.uint16))
