"""GPU parity of the v_dot8 GEMM kernel family (W3/W4 x A4, 1-8 tokens).

The dot kernel must give what the MFMA kernels give, bit for bit, for every output
form the launchers have: int32 partials (against the CPU oracle), fp32 outputs in the
canonical K order (against the oracle's range epilogue), fp16 outputs, split-K planes
and the fused argmax keys.  Quads of four 16-row tiles cut short by the matrix end and
K ranges of 1..10 groups are included.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import dev, empty, host, say
from test_gemm_gpu import _problem

pytestmark = pytest.mark.gpu

DOT_CASES = [
    # (fmt, rows, cols, batch): every token count on a small W3 matrix, W4 at four counts
    *[(2, 64, 1280, b) for b in range(1, 9)],
    (3, 64, 1280, 1), (3, 64, 1280, 3), (3, 64, 1280, 5), (3, 64, 1280, 8),
    # quads cut short by the matrix end; one-group and two-group K
    (2, 48, 1280, 5), (3, 112, 2560, 2), (2, 16, 256, 1), (3, 80, 256, 7),
    # many ranges per split (K = 17408: 14 ranges of 9-10 groups, 8 waves)
    (2, 128, 17408, 5), (3, 64, 17408, 1),
    # the timed GEMV shapes
    (2, 17408, 5120, 5), (2, 17408, 5120, 1), (3, 17408, 5120, 5), (3, 17408, 5120, 1),
    (2, 5120, 17408, 5), (3, 5120, 17408, 1),
]


def _keys_rows(rows):
    return rows - 3 if rows > 16 else rows


@pytest.mark.parametrize("fmt,rows,cols,batch", DOT_CASES)
def test_dot_kernel_equals_mfma_and_oracle(device, gx, orc, fmt, rows, cols, batch):
    p = _problem(orc, gx, fmt, 4, rows, cols, batch, seed=rows * 5 + cols + batch * 3 + fmt)
    want_P = orc.gemm_partials(p["wint"], p["aint"])
    dw, dws, da, das = dev(p["tiled"]), dev(p["tscales"]), dev(p["acts"]), dev(p["as16"])
    # int32 partials
    P = empty((batch, rows, cols // 128), np.int32)
    say("dot partials", fmt, rows, cols, batch)
    assert gx.debug_gemm_family(gx.GEMM_DOT, fmt, dw, dws, da, das, rows, cols, batch, partials=P) == gx.OK
    assert np.array_equal(host(P), want_P)
    # fp32 output: the canonical K order, and the MFMA kernels' result
    outs = {}
    for family in (gx.GEMM_MFMA, gx.GEMM_DOT):
        y = empty((batch, rows), np.float32)
        say("gemm family", family, fmt, rows, cols, batch)
        assert gx.debug_gemm_family(family, fmt, dw, dws, da, das, rows, cols, batch, out=y) == gx.OK
        outs[family] = host(y)
    assert np.array_equal(outs[gx.GEMM_DOT], orc.gemm_epilogue_ranges(want_P, p["ws16"], p["as16"])[0])
    assert np.array_equal(outs[gx.GEMM_DOT], outs[gx.GEMM_MFMA])
    # fp16 output and fused argmax keys
    halves, keys = {}, {}
    limit = _keys_rows(rows)
    for family in (gx.GEMM_MFMA, gx.GEMM_DOT):
        h = empty((batch, rows), np.uint16)
        say("gemm family half", family, fmt, rows, cols, batch)
        assert gx.debug_gemm_family(family, fmt, dw, dws, da, das, rows, cols, batch, out=h,
                                    half_output=True) == gx.OK
        halves[family] = host(h, np.uint16)
        k = empty((batch, rows // 16), np.uint64)
        say("gemm family keys", family, fmt, rows, cols, batch)
        assert gx.debug_gemm_family(family, fmt, dw, dws, da, das, rows, cols, batch, argmax_keys=k,
                                    argmax_rows=limit) == gx.OK
        keys[family] = host(k, np.uint64)
    assert np.array_equal(halves[gx.GEMM_DOT], halves[gx.GEMM_MFMA])
    assert np.array_equal(keys[gx.GEMM_DOT], keys[gx.GEMM_MFMA])
    # the keys name the best row below the limit (value order, lowest row on ties)
    y = outs[gx.GEMM_DOT]
    best = (0xFFFFFFFF - (keys[gx.GEMM_DOT].max(axis=1) & 0xFFFFFFFF)).astype(np.int64)
    assert np.array_equal(best, np.argmax(y[:, :limit], axis=1))


@pytest.mark.parametrize("fmt,rows,cols,batch,splits", [
    (2, 5120, 17408, 5, 4), (3, 5120, 17408, 1, 8), (2, 64, 1280, 3, 5), (3, 48, 2560, 8, 2),
])
def test_dot_kernel_split_planes(device, gx, orc, fmt, rows, cols, batch, splits):
    p = _problem(orc, gx, fmt, 4, rows, cols, batch, seed=rows + cols * 3 + batch + splits)
    P = orc.gemm_partials(p["wint"], p["aint"])
    dw, dws, da, das = dev(p["tiled"]), dev(p["tscales"]), dev(p["acts"]), dev(p["as16"])
    got = {}
    for family in (gx.GEMM_MFMA, gx.GEMM_DOT):
        planes = empty((splits, batch, rows), np.float32)
        say("gemm family split", family, fmt, rows, cols, batch, splits)
        assert gx.debug_gemm_family(family, fmt, dw, dws, da, das, rows, cols, batch, out=planes,
                                    splits=splits) == gx.OK
        got[family] = host(planes)
    assert np.array_equal(got[gx.GEMM_DOT], orc.gemm_epilogue_ranges(P, p["ws16"], p["as16"], splits))
    assert np.array_equal(got[gx.GEMM_DOT], got[gx.GEMM_MFMA])


def test_dot_kernel_rejections(device, gx, orc):
    """Shapes the dot kernel does not run are refused without a launch: W2, 9+ tokens,
    an odd group count (activation scales read as pairs)."""
    p = _problem(orc, gx, 2, 4, 64, 640, 9, seed=11)
    dw, dws, da, das = dev(p["tiled"]), dev(p["tscales"]), dev(p["acts"]), dev(p["as16"])
    y = empty((9, 64), np.float32)
    assert gx.debug_gemm_family(gx.GEMM_DOT, 2, dw, dws, da, das, 64, 1280, 9, out=y) == gx.UNSUPPORTED
    assert gx.debug_gemm_family(gx.GEMM_DOT, 1, dw, dws, da, das, 64, 1280, 1, out=y) == gx.UNSUPPORTED
    assert gx.debug_gemm_family(gx.GEMM_DOT, 2, dw, dws, da, das, 64, 640, 1, out=y) == gx.UNSUPPORTED
    assert gx.debug_gemm_family(3, 2, dw, dws, da, das, 64, 640, 1, out=y) == gx.INVALID_ARGUMENT
    # partials need no scales, so an odd group count runs there
    P = empty((1, 64, 5), np.int32)
    say("dot partials odd groups")
    assert gx.debug_gemm_family(gx.GEMM_DOT, 2, dw, dws, da, das, 64, 640, 1, partials=P) == gx.OK
    assert np.array_equal(host(P), orc.gemm_partials(p["wint"], p["aint"][:1]))
