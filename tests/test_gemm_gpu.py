"""GPU parity of the packed low-bit path against the CPU oracle, through the C ABI.

Bars: integer codes, scales and per-group int32 partial sums bit-exact; fp32
GEMM outputs bit-exact against the oracle's epilogue cut into the library's K ranges
(orc_gemm_epilogue_ranges; one range is the reference's sequential epilogue itself),
and within 2e-5 of max|y| of the uncut sequential epilogue (the reference harness
accepts 0.008*max(1,|y|), src/cli/main.cpp:1499).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from gpu_util import dev, empty, host, say

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def _half(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def test_mfma_operand_layout(device):
    """v_mfma_i32_16x16x64_i8: A and B share the K-slot order; lane l of C holds
    rows 4*(l//16)..+3 of column l%16 (the assumption of tests/kernel_model.py)."""
    path = os.path.join(HERE, "hip", "libmfma_probe.so")
    L = ctypes.CDLL(path)
    rng = np.random.default_rng(17)
    a = rng.integers(-128, 128, size=(64, 16), dtype=np.int8)
    b = rng.integers(-128, 128, size=(64, 16), dtype=np.int8)
    da, db, dc = dev(a), dev(b), empty((64, 4), np.int32)
    say("mfma probe")
    assert L.mfma_probe(ctypes.c_void_p(da.data_ptr()), ctypes.c_void_p(db.data_ptr()),
                        ctypes.c_void_p(dc.data_ptr())) == 0
    c = host(dc)
    A = a.astype(np.int64).reshape(4, 16, 16)  # [kb][row][j]
    B = b.astype(np.int64).reshape(4, 16, 16)  # [kb][col][j]
    C = np.einsum("krj,kcj->rc", A, B)
    expected = np.empty((64, 4), dtype=np.int64)
    for lane in range(64):
        for r in range(4):
            expected[lane, r] = C[4 * (lane // 16) + r, lane % 16]
    assert np.array_equal(c.astype(np.int64), expected)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("batch,columns", [(1, 5120), (5, 5120), (5, 17408), (32, 5120)])
def test_activation_quantizer_bit_exact(device, gx, orc, bits, batch, columns):
    rng = np.random.default_rng(batch * columns + bits)
    x = rng.standard_normal((batch, columns)).astype(np.float32)
    x[0, :128] = 0.0                              # all-zero group -> scale 1
    x[-1, 128:256] = np.float32(3.5)              # constant group
    x[-1, 256:384] = rng.standard_normal(128) * 1e-4  # tiny values
    x16 = _half(x)
    if bits == 4:
        want_codes, want_scales = orc.quantize_activation_i4(x16)
        codes = empty((batch, columns // 2), np.uint8)
    else:
        want_codes, want_scales = orc.quantize_activation_i8(x16)
        codes = empty((batch, columns), np.int8)
    scales = empty((batch, columns // 128), np.uint16)
    say("quantize_activation", bits, batch, columns)
    fn = gx.launch_quantize_activation_i4 if bits == 4 else gx.launch_quantize_activation_i8
    fn(dev(x16), codes, scales, columns, batch)
    assert np.array_equal(host(codes).view(want_codes.dtype), want_codes)
    assert np.array_equal(host(scales, np.uint16), want_scales)


def _pad16(w):
    rows = (w.shape[0] + 15) // 16 * 16
    out = np.zeros((rows, w.shape[1]), dtype=np.float32)
    out[: w.shape[0]] = w
    return out


@pytest.mark.parametrize("fmt,name", [(1, "w2"), (2, "w3"), (3, "w4")])
def test_device_quantizer_matches_reference_golden(device, gx, orc, fmt, name):
    from conftest import golden
    g = golden(f"quant_{name}.npz")
    for case in ["planted_3x256", "normal_32x256", "baseline_16x512", "edges_16x128"]:
        w = g[f"{case}__input"]
        rows0, cols = w.shape
        wp = _pad16(w)
        rows = wp.shape[0]
        codes = empty((gx.tile_bytes(fmt, rows, cols),), np.uint8)
        scales = empty((rows * cols // 128,), np.uint16)
        flag = empty((1,), np.int32)
        say("device quantizer golden", name, case)
        gx.launch_quantize_group128(fmt, dev(wp), rows, cols, codes, scales, flag)
        wq, s16 = gx.untile_group128(fmt, host(codes), host(scales, np.uint16), rows, cols)
        want_w = orc.unpack_weights(g[f"{case}__codes"], rows0, cols, fmt)
        assert np.array_equal(wq[:rows0], want_w), case
        assert np.array_equal(s16[:rows0], orc.f32_to_f16_bits(g[f"{case}__scales"])), case
        assert int(host(flag)[0]) == 0


def test_device_quantizer_flags_non_finite(device, gx):
    w = np.zeros((16, 128), np.float32)
    w[3, 5] = np.inf
    codes = empty((gx.tile_bytes(2, 16, 128),), np.uint8)
    scales = empty((16,), np.uint16)
    flag = empty((1,), np.int32)
    say("device quantizer non-finite")
    gx.launch_quantize_group128(2, dev(w), 16, 128, codes, scales, flag)
    assert int(host(flag)[0]) == 1


@pytest.mark.parametrize("fmt", [2, 3])
def test_device_quantizer_full_shape(device, gx, orc, fmt):
    rows, cols = 17408, 5120
    rng = np.random.default_rng(0x5EED0001)
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    codes = empty((gx.tile_bytes(fmt, rows, cols),), np.uint8)
    scales = empty((rows * cols // 128,), np.uint16)
    say("device quantizer full shape", fmt)
    gx.launch_quantize_group128(fmt, dev(w), rows, cols, codes, scales)
    _, ocodes, oscales = orc.quantize_group128(w, fmt)
    tiled, tscales = gx.tile_group128(fmt, ocodes, oscales, rows, cols)
    assert np.array_equal(host(codes), tiled)
    assert np.array_equal(host(scales, np.uint16), tscales)


def _problem(orc, gx, fmt, abits, rows, cols, batch, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    _, codes, scales = orc.quantize_group128(w, fmt)
    tiled, tscales = gx.tile_group128(fmt, codes, scales, rows, cols)
    wint = orc.unpack_weights(codes, rows, cols, fmt)
    x16 = _half(rng.standard_normal((batch, cols)))
    if abits == 4:
        acts, as16 = orc.quantize_activation_i4(x16)
        aint = orc.unpack_a4(acts, cols)
    else:
        acts, as16 = orc.quantize_activation_i8(x16)
        aint = acts
    return dict(tiled=tiled, tscales=tscales, wint=wint, ws16=orc.f32_to_f16_bits(scales),
                acts=acts, as16=as16, aint=aint, x16=x16)


CASES = [
    # (fmt, abits, rows, cols, batch)
    (2, 4, 64, 640, 1), (2, 4, 64, 640, 2), (2, 4, 64, 640, 3), (2, 4, 64, 640, 4),
    (2, 4, 64, 640, 5), (2, 4, 64, 640, 7), (2, 4, 64, 640, 8), (2, 4, 64, 640, 9),
    (2, 4, 64, 640, 16), (2, 4, 64, 640, 17), (2, 4, 64, 640, 31), (2, 4, 64, 640, 32),
    (3, 4, 64, 640, 1), (3, 4, 64, 640, 5), (3, 4, 64, 640, 12), (3, 4, 64, 640, 32),
    (2, 8, 64, 640, 1), (2, 8, 64, 640, 5), (2, 8, 64, 640, 32),
    (3, 8, 64, 640, 3), (3, 8, 64, 640, 16),
    (2, 4, 17408, 5120, 5), (2, 4, 5120, 17408, 5), (3, 4, 17408, 5120, 5),
    (2, 4, 17408, 5120, 1), (2, 4, 17408, 5120, 32), (2, 8, 17408, 5120, 1),
    # the remaining timed GEMV shapes: W4A4 up at batch 1, plain
    # W3A4 / W4A4 down at batch 1 and 5
    (3, 4, 17408, 5120, 1), (2, 4, 5120, 17408, 1), (3, 4, 5120, 17408, 1), (3, 4, 5120, 17408, 5),
    # down projection at verify batches: K = 17408 needs the LDS wave cap at 32 tokens
    (2, 4, 5120, 17408, 32), (3, 4, 5120, 17408, 16), (2, 8, 5120, 17408, 32),
    # 9-32 tokens (LDS-ring kernel): workgroups of 4 or 8 tiles with a short last one
    (2, 4, 48, 256, 13), (3, 4, 112, 384, 32), (3, 4, 16480, 5120, 32), (2, 4, 34816, 5120, 24),
    # each direct-kernel shape class (row tiles x chunk groups by grid size) at 9-16 and
    # 17-32 tokens, with a short last workgroup where the tiles do not divide by three
    (2, 4, 34816, 5120, 16), (2, 4, 17408, 5120, 12), (3, 4, 12288, 5120, 32), (3, 4, 12352, 5120, 9),
    # W2 (reference formats W2/W3/W4; no BASELINE config uses it)
    (1, 4, 64, 640, 1), (1, 4, 64, 640, 5), (1, 4, 64, 640, 17), (1, 4, 64, 640, 32),
    (1, 8, 64, 640, 3), (1, 8, 64, 640, 16), (1, 4, 17408, 5120, 5), (1, 4, 5120, 17408, 32),
]


@pytest.mark.parametrize("fmt,abits,rows,cols,batch", CASES)
def test_gemm_partials_bit_exact_and_output(device, gx, orc, fmt, abits, rows, cols, batch):
    p = _problem(orc, gx, fmt, abits, rows, cols, batch, seed=rows + cols + batch + fmt * 7 + abits)
    want_P = orc.gemm_partials(p["wint"], p["aint"])
    want_y = orc.gemm_epilogue(want_P, p["ws16"], p["as16"])
    dw, dws = dev(p["tiled"]), dev(p["tscales"])
    da, das = dev(p["acts"]), dev(p["as16"])
    P = empty((batch, rows, cols // 128), np.int32)
    say("gemm partials", fmt, abits, rows, cols, batch)
    gx.debug_gemm_partials(fmt, dw, abits, da, rows, cols, batch, P)
    assert np.array_equal(host(P), want_P)
    y = empty((batch, rows), np.float32)
    say("gemm output", fmt, abits, rows, cols, batch)
    if abits == 4:
        gx.launch_i4_gemm(fmt, dw, dws, da, das, y, rows, cols, batch)
    else:
        gx.launch_i8_gemm(fmt, dw, dws, da, das, y, rows, cols, batch)
    got = host(y)
    assert np.array_equal(got, orc.gemm_epilogue_ranges(want_P, p["ws16"], p["as16"])[0])
    scale = max(1e-30, float(np.abs(want_y).max()))
    assert np.abs(got - want_y).max() <= 2e-5 * scale


@pytest.mark.parametrize("fmt,rows,cols,batch,splits", [
    (2, 5120, 17408, 5, 4), (2, 5120, 17408, 32, 4), (3, 5120, 17408, 5, 8), (3, 5120, 6144, 5, 4),
    (3, 5120, 6144, 16, 3), (2, 5120, 5120, 9, 5), (2, 64, 640, 1, 5), (3, 64, 640, 32, 2),
    (2, 48, 1024, 7, 8), (1, 5120, 17408, 5, 4), (1, 64, 640, 32, 2),
    # split grids in each direct-kernel shape class: 1280 and 2560 row tiles x splits
    (2, 5120, 17408, 12, 4), (2, 5120, 17408, 32, 8), (3, 5120, 17408, 20, 8),
])
def test_gemm_split_planes_sum_to_product(device, gx, orc, fmt, rows, cols, batch, splits):
    """Split-K planes: plane s = the epilogue over the s-th of `splits` equal pack ranges
    of K; their sum in plane order is the product (same 2e-5 bar as the plain GEMM)."""
    p = _problem(orc, gx, fmt, 4, rows, cols, batch, seed=rows * 3 + cols + batch + splits)
    P = orc.gemm_partials(p["wint"], p["aint"])
    want = orc.gemm_epilogue(P, p["ws16"], p["as16"])
    planes = empty((splits, batch, rows), np.float32)
    say("gemm split", fmt, rows, cols, batch, splits)
    gx.launch_i4_gemm_split(fmt, dev(p["tiled"]), dev(p["tscales"]), dev(p["acts"]), dev(p["as16"]),
                            planes, rows, cols, batch, splits)
    got = host(planes)
    assert np.array_equal(got, orc.gemm_epilogue_ranges(P, p["ws16"], p["as16"], splits))
    total = got[0].copy()
    for s in range(1, splits):
        total += got[s]
    scale = float(np.abs(want).max())
    assert np.abs(total - want).max() <= 2e-5 * scale
    # each plane is exactly its own K range: planes of disjoint ranges are not all alike
    groups = cols // 128
    if splits <= groups:
        assert not np.array_equal(got[0], got[-1])


@pytest.mark.parametrize("fmt,rows,cols", [(2, 640, 5120), (3, 512, 17408), (2, 48, 640), (3, 96, 1280)])
def test_gemm_is_batch_invariant(device, gx, orc, fmt, rows, cols):
    """Every kernel variant sums K in one canonical order, so token i of a batch of B
    gets bit for bit what it gets alone (what makes a verify block equal one-token
    steps), for the plain product and for split-K planes."""
    p = _problem(orc, gx, fmt, 4, rows, cols, 32, seed=rows + cols + fmt)
    acts, as16 = p["acts"], p["as16"]
    dw, dws = dev(p["tiled"]), dev(p["tscales"])
    splits = gx.gemm_split_count(rows, cols, 1)
    for b in (2, 5, 32):
        assert gx.gemm_split_count(rows, cols, b) == splits
    ref = ref_planes = None
    for batch in (32, 1, 2, 3, 4, 5, 7, 8, 9, 13, 16, 17, 24, 31):
        da, das = dev(np.ascontiguousarray(acts[:batch])), dev(np.ascontiguousarray(as16[:batch]))
        y = empty((batch, rows), np.float32)
        say("gemm batch invariance", fmt, rows, cols, batch)
        gx.launch_i4_gemm(fmt, dw, dws, da, das, y, rows, cols, batch)
        planes = empty((splits, batch, rows), np.float32)
        gx.launch_i4_gemm_split(fmt, dw, dws, da, das, planes, rows, cols, batch, splits)
        if ref is None:
            ref, ref_planes = host(y), host(planes)
            want = orc.gemm_epilogue(orc.gemm_partials(p["wint"], p["aint"]), p["ws16"], p["as16"])
            assert np.abs(ref - want).max() <= 2e-5 * float(np.abs(want).max())
            continue
        assert np.array_equal(host(y), ref[:batch]), batch
        assert np.array_equal(host(planes), ref_planes[:, :batch]), batch


def test_gemm_split_rejects_bad_counts(device, gx):
    z = empty((8,), np.uint8)
    L = gx.lib()
    for splits in (0, 9, 6):  # 6 > K/128 = 5
        rc = L.gfxinfer_launch_gfx950_i4_gemm_split(2, z.data_ptr(), z.data_ptr(), z.data_ptr(), z.data_ptr(),
                                                     z.data_ptr(), 16, 640, 1, splits, None)
        assert rc == gx.INVALID_ARGUMENT
    assert 1 <= gx.gemm_split_count(5120, 17408, 5) <= 8
    assert gx.gemm_split_count(34816, 5120, 5) == 1


def test_gemm_half_output(device, gx, orc):
    fmt, rows, cols, batch = 2, 5120, 10240, 1  # mtp.fc shape
    p = _problem(orc, gx, fmt, 4, rows, cols, batch, seed=21)
    P = orc.gemm_partials(p["wint"], p["aint"])
    want = orc.gemm_epilogue(P, p["ws16"], p["as16"])
    y = empty((batch, rows), np.uint16)
    say("gemm half", rows, cols)
    gx.launch_i4_gemm_half(fmt, dev(p["tiled"]), dev(p["tscales"]), dev(p["acts"]), dev(p["as16"]), y, rows, cols, batch)
    got = host(y, np.uint16).view(np.float16).astype(np.float32)
    exact = orc.gemm_epilogue_ranges(P, p["ws16"], p["as16"])[0]
    assert np.array_equal(got, exact.astype(np.float16).astype(np.float32))
    ref16 = want.astype(np.float16).astype(np.float32)
    assert np.abs(got - ref16).max() <= 2e-5 * np.abs(want).max() + np.abs(ref16).max() * 2 ** -10


def test_gemm_fused_four_matrices(device, gx, orc):
    """GDN input projection set: qkv/z/a/b (8192, 4096, 32, 32 rows) from K=5120."""
    fmt, cols, batch = 3, 5120, 5
    rng = np.random.default_rng(33)
    x16 = _half(rng.standard_normal((batch, cols)))
    acts, as16 = orc.quantize_activation_i4(x16)
    aint = orc.unpack_a4(acts, cols)
    mats, wants, outs = [], [], []
    for i, rows in enumerate((8192, 4096, 32, 32)):
        w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
        _, codes, scales = orc.quantize_group128(w, fmt)
        tiled, ts = gx.tile_group128(fmt, codes, scales, rows, cols)
        P = orc.gemm_partials(orc.unpack_weights(codes, rows, cols, fmt), aint)
        wants.append(orc.gemm_epilogue_ranges(P, orc.f32_to_f16_bits(scales), as16)[0])
        out = empty((batch, rows), np.float32)
        outs.append(out)
        mats.append((dev(tiled), dev(ts), out, rows))
    say("gemm fused")
    gx.launch_i4_gemm_fused(fmt, mats, dev(acts), dev(as16), cols, batch)
    for out, want in zip(outs, wants):
        assert np.array_equal(host(out), want)


def test_quantize_then_gemm_matches_float_reference(device, gx, orc):
    """fp16 x -> A4 on GPU -> W3A4 GEMM on GPU vs the dequant-dot reference of
    src/cli/main.cpp:1468-1495 at the BASELINE tolerance (1e-2 relative)."""
    fmt, rows, cols, batch = 2, 17408, 5120, 5
    p = _problem(orc, gx, fmt, 4, rows, cols, batch, seed=44)
    codes = empty((batch, cols // 2), np.uint8)
    scales = empty((batch, cols // 128), np.uint16)
    y = empty((batch, rows), np.float32)
    say("quant+gemm")
    gx.launch_quantize_activation_i4(dev(p["x16"]), codes, scales, cols, batch)
    gx.launch_i4_gemm(fmt, dev(p["tiled"]), dev(p["tscales"]), codes, scales, y, rows, cols, batch)
    got = host(y)
    ws = p["ws16"].view(np.float16).astype(np.float32)
    ref = orc.lib()
    out = np.empty((batch, rows), np.float32)
    ref.orc_dequant_dot_gemv(orc.ptr(np.ascontiguousarray(p["wint"])), orc.ptr(np.ascontiguousarray(ws)),
                             orc.ptr(p["aint"]), orc.ptr(p["as16"]), rows, cols, batch, orc.ptr(out))
    assert np.all(np.abs(got - out) <= 1e-2 * np.maximum(1.0, np.abs(out)))
    assert np.abs(got - out).max() <= 1e-4 * np.abs(out).max()


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_row_gather(device, gx, orc, fmt):
    rows, cols = 64, 5120
    p = _problem(orc, gx, fmt, 4, rows, cols, 1, seed=55)
    ws = p["ws16"].view(np.float16).astype(np.float32)
    dw, dws = dev(p["tiled"]), dev(p["tscales"])
    out = empty((cols,), np.uint16)
    for row in (0, 17, 63):
        say("row gather", fmt, row)
        gx.launch_row_gather_tiled(fmt, dw, dws, out, row, rows, cols)
        want = _half(p["wint"][row].astype(np.float32) * np.repeat(ws[row], 128))
        assert np.array_equal(host(out, np.uint16), want)
    idx = dev(np.array([41], np.uint32))
    gx.launch_row_gather_tiled_indirect(fmt, dw, dws, out, idx, rows, cols)
    want = _half(p["wint"][41].astype(np.float32) * np.repeat(ws[41], 128))
    assert np.array_equal(host(out, np.uint16), want)
    idx = dev(np.array([rows + 5], np.uint32))  # out of range -> zeros (lowbit_gemv.hip:202-205)
    gx.launch_row_gather_tiled_indirect(fmt, dw, dws, out, idx, rows, cols)
    assert np.all(host(out, np.uint16) == 0)

    # Batched gather: every row equals the one-row launch; host rows, a device first row
    # with device rest rows (the verifier's seed + drafts), out-of-range rows are zeros.
    def want_rows(ids):
        return np.stack([_half(p["wint"][r].astype(np.float32) * np.repeat(ws[r], 128)) if r < rows
                         else np.zeros(cols, np.uint16) for r in ids])
    ids = [5, 63, 0, rows + 1, 17, 17, 40, 2]
    many = empty((len(ids), cols), np.uint16)
    say("batched row gather", fmt, len(ids))
    gx.launch_row_gather_tiled_batch(fmt, dw, dws, many, ids, None, None, len(ids), rows, cols)
    assert np.array_equal(host(many, np.uint16), want_rows(ids))
    first, rest = dev(np.array([33], np.uint32)), dev(np.array(ids[1:], np.uint32))
    gx.launch_row_gather_tiled_batch(fmt, dw, dws, many, [0] * len(ids), first, rest, len(ids), rows, cols)
    assert np.array_equal(host(many, np.uint16), want_rows([33] + ids[1:]))
    full = empty((32, cols), np.uint16)
    ids32 = [(7 * j) % rows for j in range(32)]
    gx.launch_row_gather_tiled_batch(fmt, dw, dws, full, ids32, None, None, 32, rows, cols)
    assert np.array_equal(host(full, np.uint16), want_rows(ids32))
    for count in (0, 33):
        with pytest.raises(gx.GfxinferError):
            gx.launch_row_gather_tiled_batch(fmt, dw, dws, full, None, first, rest, count, rows, cols)


def _gemm_argmax(gx, fmt, p, rows, cols, batch, argmax_rows, ids=None, logits=True):
    ws_bytes = gx.lib().gfxinfer_gemm_argmax_workspace_bytes(rows, batch)
    work = empty((ws_bytes // 8,), np.uint64)
    tokens = empty((batch,), np.uint32)
    y = empty((batch, rows), np.float32) if logits else None
    dids = dev(ids) if ids is not None else None
    dw, dws, da, das = dev(p["tiled"]), dev(p["tscales"]), dev(p["acts"]), dev(p["as16"])
    say("gemm argmax", fmt, rows, cols, batch, argmax_rows)
    gx.check(gx.lib().gfxinfer_launch_gfx950_i4_gemm_argmax(
        fmt, dw.data_ptr(), dws.data_ptr(), da.data_ptr(), das.data_ptr(),
        None if y is None else y.data_ptr(), rows, cols, batch, argmax_rows,
        None if dids is None else dids.data_ptr(), work.data_ptr(), ws_bytes, tokens.data_ptr(), None))
    return host(tokens, np.uint32), (host(y) if y is not None else None)


@pytest.mark.parametrize("fmt,rows,cols,batch,limit", [
    (3, 1024, 256, 1, 1024), (3, 1024, 256, 5, 1000), (3, 4096, 640, 32, 4000), (2, 2048, 512, 17, 2048),
    (3, 151936, 5120, 5, 151936), (3, 151936, 5120, 16, 151936), (3, 151936, 5120, 32, 151936),
    # 17000 tiles: more keys per row than one pass of the reduction's loads holds
    (3, 272000, 128, 2, 271990)])
def test_gemm_argmax_matches_logits_argmax(device, gx, orc, fmt, rows, cols, batch, limit):
    """LM head + fused greedy argmax == argmax (ties to the lowest index) of the same
    GEMM's logits, and the logits match the oracle epilogue."""
    p = _problem(orc, gx, fmt, 4, rows, cols, batch, seed=rows + batch)
    tokens, y = _gemm_argmax(gx, fmt, p, rows, cols, batch, limit)
    want = np.empty(batch, np.uint32)
    orc.lib().orc_argmax(orc.ptr(np.ascontiguousarray(y)), limit, rows, batch, None, orc.ptr(want))
    assert np.array_equal(tokens, want)
    P = orc.gemm_partials(p["wint"], p["aint"])
    assert np.array_equal(y, orc.gemm_epilogue_ranges(P, p["ws16"], p["as16"])[0])
    want_y = orc.gemm_epilogue(P, p["ws16"], p["as16"])
    del P
    assert np.abs(y - want_y).max() <= 2e-5 * max(1e-30, float(np.abs(want_y).max()))
    tokens_only, _ = _gemm_argmax(gx, fmt, p, rows, cols, batch, limit, logits=False)
    assert np.array_equal(tokens_only, tokens)


def test_gemm_argmax_ties_limit_and_mapping(device, gx, orc):
    """Every row a copy of one row: all logits tie, so the lowest row wins; the
    shortlist limit and the token-id map (argmax_mapped) apply."""
    fmt, rows, cols, batch = 3, 512, 256, 3
    p = _problem(orc, gx, fmt, 4, 16, cols, batch, seed=9)  # activations only
    w = np.repeat(orc.synthetic_values(3, "tie", cols, 0.02, 0.0)[None, :], rows, axis=0)
    _, codes, scales = orc.quantize_group128(w, fmt)
    tiled, tscales = gx.tile_group128(fmt, codes, scales, rows, cols)
    q = dict(p, tiled=tiled, tscales=tscales)
    tokens, y = _gemm_argmax(gx, fmt, q, rows, cols, batch, rows)
    assert (y == y[:, :1]).all() and (tokens == 0).all()
    ids = (np.arange(rows, dtype=np.uint32) * 7 + 3) % 100000
    tokens, _ = _gemm_argmax(gx, fmt, q, rows, cols, batch, 100, ids=ids)
    assert (tokens == ids[0]).all()


def test_stream_read_floor_entry(gx, device):
    """The calibration read runs over in-bounds sizes (a tail shorter than one stride
    included), leaves the sink untouched for data whose XOR is not the marker, and
    rejects misaligned or empty requests."""
    import torch
    data = torch.zeros(3 * 256 * 16 + 7 * 16, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4 * 256, dtype=torch.int32, device="cuda")
    for width in (1, 3, 4):
        gx.debug_stream_read(data, data.numel(), sink, width)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    for nbytes, width in ((0, 1), (24, 1), (16, 0)):
        with pytest.raises(gx.GfxinferError):
            gx.debug_stream_read(data, nbytes, sink, width)


def test_stream_read_oneshot_entry(gx, device):
    """The one-shot calibration read covers sizes that leave a partial last workgroup
    (lanes past the end re-read the last piece), never writes a sink that is exactly
    bytes / 16 entries long for data whose XOR is not the marker, and rejects
    misaligned, empty and unsupported requests."""
    import torch
    data = torch.zeros(3 * 256 * 16 + 7 * 16, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(data.numel() // 16, dtype=torch.int32, device="cuda")
    for loads in (1, 2, 4, 8):
        gx.debug_stream_read_oneshot(data, data.numel(), sink, loads)
        gx.debug_stream_read_oneshot(data, 16, sink, loads)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    for nbytes, loads in ((0, 1), (24, 1), (16, 0), (16, 3), (16, 16)):
        with pytest.raises(gx.GfxinferError):
            gx.debug_stream_read_oneshot(data, nbytes, sink, loads)

