"""CPU tests of the C ABI library: symbols, argument validation, the gfx950 tile
layout and the kernel's operand bit tricks (through tests/kernel_model.py)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import kernel_model as KM


def test_library_exports_every_header_function(gx):
    names = gx.header_functions()
    assert len(names) >= 10
    L = gx.lib()
    for name in names:
        assert hasattr(L, name), name
    assert set(names) <= set(gx.SIGNATURES), set(names) - set(gx.SIGNATURES)


def test_packed_row_bytes_matches_reference(gx, orc):
    for fmt in (1, 2, 3):
        for k in (128, 5120, 17408):
            assert gx.packed_row_bytes(fmt, k) == orc.packed_row_bytes(fmt, k)


@pytest.mark.parametrize("fmt", [1, 2, 3])
@pytest.mark.parametrize("shape", [(16, 128), (32, 256), (48, 640)])
def test_tile_untile_round_trip(gx, orc, fmt, shape):
    rows, cols = shape
    rng = np.random.default_rng(rows * cols + fmt)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    _, codes, scales = orc.quantize_group128(w, fmt)
    tiled, tscales = gx.tile_group128(fmt, codes, scales, rows, cols)
    assert tiled.nbytes == rows * cols * {1: 2, 2: 3, 3: 4}[fmt] // 8
    wq, s16 = gx.untile_group128(fmt, tiled, tscales, rows, cols)
    assert np.array_equal(wq, orc.unpack_weights(codes, rows, cols, fmt))
    assert np.array_equal(s16, orc.f32_to_f16_bits(scales))


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_operand_expansion_bit_tricks(gx, orc, fmt):
    """Every lane chunk expands to 16*w (W4) / 32*w (W2, W3) in the documented slot order."""
    rows, cols = 32, 256
    rng = np.random.default_rng(9)
    if fmt == 1:
        wint = rng.choice(np.array([-3, -1, 1, 3], np.int8), size=(rows, cols))
        hi = 4
    else:
        lo, hi = (-4, 4) if fmt == 2 else (-8, 8)
        wint = rng.integers(lo, hi, size=(rows, cols)).astype(np.int8)
    # build reference-packed codes from integers via the oracle's storage order
    scales = np.ones((rows, cols // 128), np.float32)
    w = wint.astype(np.float32)
    w[:, ::128] = np.float32(hi - 1 if fmt == 3 else 3)  # pin max so scale fits the codebook
    _, codes, sc = orc.quantize_group128(w, fmt)
    wq = orc.unpack_weights(codes, rows, cols, fmt)
    tiled, ts = gx.tile_group128(fmt, codes, sc, rows, cols)
    LB = KM.lane_bytes(fmt)
    chunks = tiled.reshape(rows // 16, cols // 128, 64, LB)
    factor = 16 if fmt == 3 else 32
    for t in range(rows // 16):
        for g in range(cols // 128):
            d = chunks[t, g].copy().view(np.uint32).reshape(64, LB // 4)
            if fmt == 1:
                h0, h1 = KM.expand_w2(d[:, 0]), KM.expand_w2(d[:, 1])
            elif fmt == 2:
                h0, h1 = KM.expand_w3(d[:, 0], d[:, 1], d[:, 2])
            else:
                h0, h1 = KM.expand_nibbles(d[:, 0], d[:, 1]), KM.expand_nibbles(d[:, 2], d[:, 3])
            for h, regs in enumerate((h0, h1)):
                b = KM.regs_to_bytes(regs).astype(np.int32)  # [64 lanes, 16]
                for lane in range(64):
                    m, kb = lane % 16, lane // 16
                    for j in range(16):
                        reg, byte = j // 4, j % 4
                        col = g * 128 + kb * 32 + 16 * h + 8 * (reg >> 1) + 2 * byte + (reg & 1)
                        assert b[lane, j] == factor * int(wq[t * 16 + m, col])


@pytest.mark.parametrize("fmt,abits,batch", [(2, 4, 1), (2, 4, 5), (3, 4, 8), (2, 8, 3), (3, 8, 12), (2, 4, 20),
                                              (1, 4, 5), (1, 8, 3), (1, 4, 17)])
def test_kernel_lane_mapping_model(gx, orc, fmt, abits, batch):
    """The kernel's packing of groups/tokens into MFMA columns reproduces the exact
    per-group integer dot products (oracle) under the symmetric-operand MFMA model."""
    rows, cols = 32, 640  # G = 5: exercises partial packs for GP = 2 and 4
    rng = np.random.default_rng(fmt * 100 + abits * 10 + batch)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    _, codes, scales = orc.quantize_group128(w, fmt)
    tiled, _ = gx.tile_group128(fmt, codes, scales, rows, cols)
    x16 = rng.standard_normal((batch, cols)).astype(np.float32).astype(np.float16).view(np.uint16)
    if abits == 4:
        acts, _ = orc.quantize_activation_i4(x16)
        aint = orc.unpack_a4(acts, cols)
    else:
        acts, _ = orc.quantize_activation_i8(x16)
        aint = acts
        acts = acts.view(np.uint8)
    P = KM.simulate_partials(fmt, tiled, abits, acts, rows, cols, batch)
    expected = orc.gemm_partials(orc.unpack_weights(codes, rows, cols, fmt), aint)
    assert np.array_equal(P, expected)


def test_launchers_validate_before_launching(gx):
    """Argument errors return invalid_argument/unsupported without touching HIP
    (lowbit_gemv.hip:1123-1130 style)."""
    L = gx.lib()
    st = L.gfxinfer_launch_gfx950_i4_gemm(2, None, None, None, None, None, 16, 128, 1, 1, None)
    assert st == gx.INVALID_ARGUMENT and "batch" in gx.last_error()
    st = L.gfxinfer_launch_gfx950_i4_gemm(4, None, None, None, None, None, 16, 128, 1, 1, None)
    assert st == gx.UNSUPPORTED  # W8G128: declared, not implemented (as in the reference)
    fake = 1 << 20  # aligned non-null addresses; validation fails before any use
    st = L.gfxinfer_launch_gfx950_i4_gemm(2, fake, fake, fake, fake, fake, 17, 128, 1, 1, None)
    assert st == gx.INVALID_ARGUMENT
    st = L.gfxinfer_launch_gfx950_i4_gemm(2, fake, fake, fake, fake, fake, 16, 127, 1, 1, None)
    assert st == gx.INVALID_ARGUMENT
    st = L.gfxinfer_launch_gfx950_i4_gemm(2, fake, fake, fake, fake, fake, 16, 128, 33, 1, None)
    assert st == gx.INVALID_ARGUMENT
    st = L.gfxinfer_launch_gfx950_i4_gemm(2, fake, fake, fake + 4, fake, fake, 16, 128, 1, 1, None)
    assert st == gx.INVALID_ARGUMENT and "aligned" in gx.last_error()
    st = L.gfxinfer_launch_quantize_activation_i4(fake, fake, fake, 130, 1, None)
    assert st == gx.INVALID_ARGUMENT
    st = L.gfxinfer_launch_quantize_activation_i8(fake, fake, fake, 128, 0, None)
    assert st == gx.INVALID_ARGUMENT
    st = L.gfxinfer_launch_gfx950_i4_gemm_fused(2, None, 1, fake, fake, 128, 1, 1, None)
    assert st == gx.INVALID_ARGUMENT
    st = L.gfxinfer_launch_lowbit_row_gather_tiled(2, fake, fake, fake, 16, 16, 128, None)
    assert st == gx.INVALID_ARGUMENT  # row >= rows
    st = L.gfxinfer_launch_quantize_group128_gfx950(4, fake, 16, 128, fake, fake, None, None)
    assert st == gx.UNSUPPORTED
    with pytest.raises(gx.GfxinferError) as err:
        gx.check(gx.INVALID_ARGUMENT)
    assert err.value.code == gx.INVALID_ARGUMENT
