"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

- Weight quantizer: bit-exact against golden vectors written by the reference's
  own src/quantization.cpp (tests/golden/make_golden.py), plus the reference
  unit-test invariants (tests/quantization_test.cpp:117-132).
- fp16 rounding: against numpy's IEEE binary16 conversion.
- Activation quantizers: closed forms (zero group, exact extremes, ties to even,
  nibble order).
- Integer GEMM and epilogue: brute force with Python integers / exact rationals.
"""
from __future__ import annotations

import fractions
import os

import numpy as np
import pytest

from conftest import golden

FORMATS = [(1, "w2"), (2, "w3"), (3, "w4")]
CASES = ["planted_3x256", "normal_32x256", "baseline_16x512", "edges_16x128"]


@pytest.mark.parametrize("fmt,name", FORMATS)
@pytest.mark.parametrize("case", CASES)
def test_quantizer_matches_reference_golden(orc, fmt, name, case):
    g = golden(f"quant_{name}.npz")
    w = g[f"{case}__input"]
    status, codes, scales = orc.quantize_group128(w, fmt)
    assert status == 0
    assert np.array_equal(codes, g[f"{case}__codes"])
    assert np.array_equal(scales.view(np.uint32), g[f"{case}__scales"].view(np.uint32))
    # dequantized_weight (quantization.cpp:222-235) == reference dequantize_group128
    wq = orc.unpack_weights(codes, w.shape[0], w.shape[1], fmt).astype(np.float32)
    deq = wq * np.repeat(scales, 128, axis=1)
    assert np.array_equal(deq.view(np.uint32), g[f"{case}__dequant"].view(np.uint32))


@pytest.mark.parametrize("fmt,name", FORMATS)
def test_quantizer_rejections_match_reference(orc, fmt, name):
    g = golden(f"quant_{name}.npz")
    assert orc.quantize_group128(np.zeros((1, 127), np.float32), fmt)[0] == int(g["reject_k127__status"][0]) == 1
    nan = np.zeros((1, 128), np.float32)
    nan[0, 3] = np.nan
    assert orc.quantize_group128(nan, fmt)[0] == int(g["reject_nan__status"][0]) == 1


@pytest.mark.parametrize("fmt,bound", [(1, 0.8), (2, 0.4), (3, 0.2)])
def test_quantizer_rmse_bounds(orc, fmt, bound):
    """tests/quantization_test.cpp:12-47 relative RMSE bounds."""
    rng = np.random.default_rng(1200)
    w = (rng.standard_normal((3, 256)) * 0.25).astype(np.float32)
    w[0, 0], w[1, 17], w[2, 93] = 0.0, 2.0, -2.0
    _, codes, scales = orc.quantize_group128(w, fmt)
    wq = orc.unpack_weights(codes, 3, 256, fmt).astype(np.float64) * np.repeat(scales, 128, axis=1)
    rmse = np.sqrt(((w - wq) ** 2).sum() / (w.astype(np.float64) ** 2).sum())
    assert rmse <= bound


def test_quantizer_full_shape_matches_reference(orc):
    """[17408, 5120] N(0, 0.02) W3 -- the BASELINE shape -- against the compiled reference."""
    if orc.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(0x5EED0001)
    w = (rng.standard_normal((17408, 5120), dtype=np.float32) * np.float32(0.02))
    a = orc.quantize_group128(w, 2)
    b = orc.ref_quantize_group128(w, 2)
    assert a[0] == b[0] == 0
    assert np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2])


def test_fp16_all_half_patterns_round_trip(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    as_f32 = bits.view(np.float16).astype(np.float32)
    ours = np.array([orc.lib().orc_f16_to_f32(int(b)) for b in bits[::97]], dtype=np.float32)
    assert np.array_equal(ours.view(np.uint32), as_f32[::97].view(np.uint32)) or np.isnan(as_f32[::97]).any()
    finite = ~np.isnan(as_f32)
    back = orc.f32_to_f16_bits(as_f32)
    assert np.array_equal(back[finite], bits[finite])


def test_fp16_rounding_matches_ieee(orc):
    """Every exponent with mantissas at and around each rounding boundary."""
    hi = (np.arange(1 << 19, dtype=np.uint32) << np.uint32(13))
    low = np.array([0x0000, 0x0001, 0x0FFF, 0x1000, 0x1001, 0x1FFF, 0x0800, 0x1800], dtype=np.uint32)
    x = (hi[:, None] | low[None, :]).ravel().view(np.float32)
    x = x[~np.isnan(x)]
    ours = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def _half(values):
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def test_activation_i4_closed_forms(orc):
    K = 256
    x = np.zeros((3, K), dtype=np.float32)
    # row 0: all zero -> scale exactly 1.0, codes 0 (lowbit_gemv.hip:386-388)
    # row 1: group max 7 -> scale 1.0 exactly, codes = round-half-even(x), clamp +-7
    x[1, :128] = np.arange(-64, 64) / 8.0 * 1.75  # multiples of 0.21875 in [-14, 14)
    x[1, :128] = np.clip(x[1, :128], -7.0, 7.0)
    x[1, 128:] = np.clip(np.arange(-32, 32).repeat(2) / 4.0, -7.0, 7.0)  # quarters: ties at .5, 1.5 ...
    x[1, 128] = 7.0
    # row 2: extremes of a random group map to exactly +-7
    rng = np.random.default_rng(7)
    x[2] = rng.standard_normal(K)
    packed, scales = orc.quantize_activation_i4(_half(x))
    q = orc.unpack_a4(packed, K).astype(np.int32)
    assert np.all(q[0] == 0) and np.all(scales[0] == 0x3C00)
    assert scales[1, 0] == 0x3C00 and scales[1, 1] == 0x3C00
    xs = _half(x[1]).view(np.float16).astype(np.float64)
    assert np.array_equal(q[1], np.clip(np.round(xs), -7, 7).astype(np.int32))  # np.round = half-even
    for grp in range(2):
        seg = x[2, grp * 128:(grp + 1) * 128]
        i = np.argmax(np.abs(seg))
        assert q[2, grp * 128 + i] == (7 if seg[i] > 0 else -7)
    # nibble order: even column in the low nibble (lowbit_gemv.hip:404-405)
    assert (packed[1, 64] & 0xF) == (q[1, 128] & 0xF) and (packed[1, 64] >> 4) == (q[1, 129] & 0xF)


def test_activation_i8_closed_forms(orc):
    K = 128
    x = np.zeros((2, K), dtype=np.float32)
    x[1] = np.linspace(-127, 127, K)
    codes, scales = orc.quantize_activation_i8(_half(x))
    assert np.all(codes[0] == 0) and scales[0, 0] == 0x3C00
    assert scales[1, 0] == 0x3C00
    xs = _half(x[1]).view(np.float16).astype(np.float64)
    assert np.array_equal(codes[1].astype(np.int32), np.round(xs).astype(np.int32))


def test_activation_scale_rounds_to_fp16(orc):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((4, 512)) * 3).astype(np.float32)
    _, scales = orc.quantize_activation_i4(_half(x))
    xs = _half(x).view(np.float16).astype(np.float32).reshape(4, 4, 128)
    expected = (np.abs(xs).max(axis=2) / np.float32(7.0)).astype(np.float16).view(np.uint16)
    assert np.array_equal(scales, expected)


def test_gemm_partials_brute_force(orc):
    rng = np.random.default_rng(3)
    w = rng.integers(-8, 8, size=(16, 384), dtype=np.int8)
    a = rng.integers(-127, 128, size=(3, 384), dtype=np.int8)
    P = orc.gemm_partials(w, a)
    for b in range(3):
        for n in range(0, 16, 5):
            for g in range(3):
                s = sum(int(w[n, k]) * int(a[b, k]) for k in range(g * 128, g * 128 + 128))
                assert P[b, n, g] == s


def test_gemm_epilogue_is_one_rounding_per_group(orc):
    """acc = fmaf(float(P), ws*as, acc): checked with exact rationals."""
    rng = np.random.default_rng(4)
    B, N, G = 2, 16, 5
    P = rng.integers(-3584, 3585, size=(B, N, G), dtype=np.int32)
    ws16 = (rng.uniform(0.002, 0.08, size=(N, G))).astype(np.float16).view(np.uint16)
    as16 = (rng.uniform(0.01, 0.5, size=(B, G))).astype(np.float16).view(np.uint16)
    y = orc.gemm_epilogue(P, ws16, as16)
    ws = ws16.view(np.float16).astype(np.float32)
    as_ = as16.view(np.float16).astype(np.float32)
    for b in range(B):
        for n in range(0, N, 3):
            acc = np.float32(0)
            for g in range(G):
                scale = np.float32(ws[n, g] * as_[b, g])
                exact = fractions.Fraction(int(P[b, n, g])) * fractions.Fraction(float(scale)) + fractions.Fraction(float(acc))
                acc = np.float32(float(exact))  # float(Fraction) is correctly rounded to double...
                # ...and double->float32 can double-round; the magnitudes here keep it exact
            assert y[b, n] == acc


def _fma32(p, scale, acc):
    exact = fractions.Fraction(int(p)) * fractions.Fraction(float(scale)) + fractions.Fraction(float(acc))
    return np.float32(float(exact))


@pytest.mark.parametrize("groups,splits", [(1, 1), (7, 1), (10, 1), (11, 1), (40, 1), (136, 1), (200, 1),
                                           (40, 4), (136, 4), (48, 3), (5, 5), (23, 2)])
def test_gemm_epilogue_ranges_brute_force(orc, groups, splits):
    """The library's K order, from its definition: split s = groups [G s/S, G(s+1)/S),
    R = clamp(ceil(n/10), 1, 16) ranges [b + n r/R, b + n(r+1)/R), each a sequential
    epilogue from 0, added in range order; one range is the reference epilogue itself."""
    rng = np.random.default_rng(groups * 10 + splits)
    B, N = 2, 3
    P = rng.integers(-3584, 3585, size=(B, N, groups), dtype=np.int32)
    ws16 = (rng.uniform(0.002, 0.08, size=(N, groups))).astype(np.float16).view(np.uint16)
    as16 = (rng.uniform(0.01, 0.5, size=(B, groups))).astype(np.float16).view(np.uint16)
    got = orc.gemm_epilogue_ranges(P, ws16, as16, splits)
    assert got.shape == (splits, B, N)
    ws = ws16.view(np.float16).astype(np.float32)
    as_ = as16.view(np.float16).astype(np.float32)
    for b in range(B):
        for n in range(N):
            for s in range(splits):
                lo, hi = groups * s // splits, groups * (s + 1) // splits
                count = hi - lo
                ranges = min(16, max(1, -(-count // 10)))
                plane = np.float32(0)
                for r in range(ranges):
                    value = np.float32(0)
                    for g in range(lo + count * r // ranges, lo + count * (r + 1) // ranges):
                        value = _fma32(P[b, n, g], np.float32(ws[n, g] * as_[b, g]), value)
                    plane = value if r == 0 else np.float32(plane + value)
                assert got[s, b, n] == plane, (s, b, n)
    if splits == 1 and groups <= 10:
        assert np.array_equal(got[0], orc.gemm_epilogue(P, ws16, as16))
    total = got.sum(axis=0, dtype=np.float64)
    assert np.allclose(total, orc.gemm_epilogue(P, ws16, as16), rtol=1e-5, atol=1e-6)


def test_dequant_dot_gemv_close_to_exact(orc):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((32, 512)) * 0.02).astype(np.float32)
    _, codes, scales = orc.quantize_group128(w, 2)
    x = rng.standard_normal((2, 512)).astype(np.float32)
    a, as16 = orc.quantize_activation_i8(_half(x))
    y = orc.dequant_dot_gemv_packed(codes, 2, scales, a, as16, 32, 512)
    wq = orc.unpack_weights(codes, 32, 512, 2).astype(np.float64) * np.repeat(scales, 128, axis=1)
    aq = a.astype(np.float64) * np.repeat(as16.view(np.float16).astype(np.float64), 128, axis=1)
    exact = aq @ wq.T
    assert np.allclose(y, exact, rtol=1e-4, atol=1e-6)


def test_ptr_keeps_temporaries_alive(orc):
    """orc.ptr() of a temporary (np.empty(...) inline, or a dtype conversion that copies)
    keeps the array alive through the call: the oracle writes into it and the result is
    readable afterwards through the pointer's own reference."""
    import ctypes
    import gc
    x = np.arange(256, dtype=np.float64)  # converted (copied) to fp32 inline below
    p_in = orc.ptr(np.ascontiguousarray(x, dtype=np.float32))
    p_out = orc.ptr(np.empty(256, np.uint16))
    gc.collect()
    orc.lib().orc_f32_to_f16_array(p_in, p_out, 256)
    back = np.ctypeslib.as_array(ctypes.cast(p_out, ctypes.POINTER(ctypes.c_uint16)), shape=(256,))
    assert np.array_equal(back.view(np.float16).astype(np.float64), x)
    assert orc.ptr(None) is None
