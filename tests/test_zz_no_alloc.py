"""The allocation-free fused head (gfxinfer_launch_gfx950_i4_gemm_argmax_no_alloc)
against the workspace entry point it varies, through the C ABI: tokens and logits bit
for bit on two calls in a row, the second one smaller (the shared device array keeps the
first call's keys, which the second must not read), and oversize shapes rejected before
any launch."""
import numpy as np
import pytest

from gpu_util import dev, empty, host, say

pytestmark = pytest.mark.gpu


def _problem(orc, gx, fmt, rows, cols, batch, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    _, codes, scales = orc.quantize_group128(w, fmt)
    tiled, tscales = gx.tile_group128(fmt, codes, scales, rows, cols)
    x16 = rng.standard_normal((batch, cols)).astype(np.float16).view(np.uint16)
    acts, as16 = orc.quantize_activation_i4(x16)
    return [dev(a) for a in (tiled, tscales, acts, as16)]


def _both(gx, fmt, p, rows, cols, batch, limit):
    L = gx.lib()
    w, ws, a, sa = p
    work_bytes = L.gfxinfer_gemm_argmax_workspace_bytes(rows, batch)
    work = empty((work_bytes // 8,), np.uint64)
    want_t, want_y = empty((batch,), np.uint32), empty((batch, rows), np.float32)
    got_t, got_y = empty((batch,), np.uint32), empty((batch, rows), np.float32)
    say("gemm argmax with workspace", rows, cols, batch)
    gx.check(L.gfxinfer_launch_gfx950_i4_gemm_argmax(
        fmt, w.data_ptr(), ws.data_ptr(), a.data_ptr(), sa.data_ptr(), want_y.data_ptr(), rows, cols, batch,
        limit, None, work.data_ptr(), work_bytes, want_t.data_ptr(), None))
    say("gemm argmax without allocation", rows, cols, batch)
    gx.check(L.gfxinfer_launch_gfx950_i4_gemm_argmax_no_alloc(
        fmt, w.data_ptr(), ws.data_ptr(), a.data_ptr(), sa.data_ptr(), got_y.data_ptr(), rows, cols, batch,
        limit, None, got_t.data_ptr(), None))
    return (host(want_t, np.uint32), host(want_y)), (host(got_t, np.uint32), host(got_y))


def test_no_alloc_head_equals_workspace_entry(device, gx, orc):
    fmt = gx.W4G128
    first = (151936, 5120, 5, 151936)   # the W4 LM head at the verifier's 5 rows
    second = (4096, 640, 3, 4000)       # smaller: fewer tiles and tokens than the first call
    for rows, cols, batch, limit in (first, second):
        p = _problem(orc, gx, fmt, rows, cols, batch, rows + batch)
        (want_t, want_y), (got_t, got_y) = _both(gx, fmt, p, rows, cols, batch, limit)
        assert np.array_equal(got_t, want_t)
        assert np.array_equal(got_y, want_y)
        expect = np.empty(batch, np.uint32)
        orc.lib().orc_argmax(orc.ptr(np.ascontiguousarray(want_y)), limit, rows, batch, None, orc.ptr(expect))
        assert np.array_equal(got_t, expect)


def test_no_alloc_head_rejects_oversize(device, gx):
    """Every caller buffer is real and sized for the shape (no made-up address reaches
    the library); the key-count check rejects the shape before any launch."""
    L = gx.lib()
    rows, cols, batch = 272000, 128, 32  # 17000 tiles x 32 tokens > 524288 keys
    w = empty((rows * cols // 2,), np.uint8)          # W4 codes, 17.4 MB
    ws = empty((rows * cols // 128,), np.uint16)      # fp16 weight scales
    a = empty((batch, cols // 2), np.uint8)           # A4 codes
    sa = empty((batch, cols // 128), np.uint16)       # fp16 activation scales
    tokens = empty((batch,), np.uint32)
    say("no-alloc head rejects an oversize shape")
    rc = L.gfxinfer_launch_gfx950_i4_gemm_argmax_no_alloc(gx.W4G128, w.data_ptr(), ws.data_ptr(), a.data_ptr(),
                                                          sa.data_ptr(), None, rows, cols, batch, rows, None,
                                                          tokens.data_ptr(), None)
    assert rc == gx.INVALID_ARGUMENT
    assert "524288" in gx.last_error()
