"""GPU parity of the decoder operators (gfxinfer_amd/csrc/qwen_ops.hip,
attention.hip) against the CPU oracle, through the C ABI.

Bars: copies and integer codes bit-exact; fp16 outputs within a few fp16 ulps;
GDN state within fp32 1e-5 (relative to the state's magnitude); attention
within 1e-2; rollback bit-exact against running only the accepted prefix.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import dev, empty, host, say

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _half(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def _f(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def _bf16(x):
    x = np.asarray(x, dtype=np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)  # truncation: exact for test values


_KEEP: list = []


def D_(arr):
    """Device copy whose tensor stays alive for the rest of the test (an inline
    D_(x) would free the tensor before the kernel reads it)."""
    t = dev(arr)
    _KEEP.append(t)
    return t.data_ptr()


@pytest.fixture(autouse=True)
def _release_kept():
    yield
    _KEEP.clear()


def _close16(got, want, rel=2.0 ** -9, atol=1e-6):
    g, w = _f(got), _f(want)
    return np.all(np.abs(g - w) <= rel * np.abs(w) + atol)


# ---- norms --------------------------------------------------------------------

@pytest.mark.parametrize("batch", [1, 5, 32])
def test_rms_norm_batch_and_fused_quantize(device, gx, orc, batch):
    n = 5120
    rng = np.random.default_rng(batch)
    x = _half(rng.standard_normal((batch, n)) * 2)
    w = _bf16(np.round(rng.standard_normal(n) * 64) / 1024)
    want = np.empty_like(x)
    orc.lib().orc_rms_norm(orc.ptr(x), orc.ptr(w), orc.ptr(want), n, batch, EPS, 1)
    out = empty((batch, n), np.uint16)
    say("rms_norm_batch", batch)
    L = gx.lib()
    dx, dw = dev(x), dev(w)
    gx.check(L.gfxinfer_launch_rms_norm_batch(dx.data_ptr(), dw.data_ptr(), out.data_ptr(), n, batch, EPS, 1, None))
    got = host(out, np.uint16)
    assert np.array_equal(got, want)  # the reference's summation order on both sides
    # fused RMSNorm -> A4: the codes are exactly the A4 quantization of its own fp16 output
    normed = empty((batch, n), np.uint16)
    codes = empty((batch, n // 2), np.uint8)
    scales = empty((batch, n // 128), np.uint16)
    say("rms_norm_quantize_i4", batch)
    gx.check(L.gfxinfer_launch_rms_norm_quantize_i4(dx.data_ptr(), dw.data_ptr(), normed.data_ptr(), codes.data_ptr(),
                                                    scales.data_ptr(), n, batch, EPS, 1, None))
    g_norm = host(normed, np.uint16)
    assert np.array_equal(g_norm, got)
    c, s = orc.quantize_activation_i4(g_norm)
    assert np.array_equal(host(codes), c) and np.array_equal(host(scales, np.uint16), s)


@pytest.mark.parametrize("batch", [1, 5])
def test_residual_add_rms_norm_and_fused_quantize(device, gx, orc, batch):
    n = 5120
    rng = np.random.default_rng(10 + batch)
    res = _half(rng.standard_normal((batch, n)))
    upd = rng.standard_normal((batch, n)).astype(np.float32)
    w = _bf16(np.round(rng.standard_normal(n) * 64) / 1024)
    want_r = np.empty_like(res)
    want_n = np.empty_like(res)
    orc.lib().orc_residual_add_rms_norm(orc.ptr(res), orc.ptr(upd), orc.ptr(want_r), orc.ptr(w), orc.ptr(want_n),
                                        n, batch, EPS, 1)
    L = gx.lib()
    dr, du, dw = dev(res), dev(upd), dev(w)
    ro, no = empty((batch, n), np.uint16), empty((batch, n), np.uint16)
    say("residual_add_rms_norm", batch)
    gx.check(L.gfxinfer_launch_residual_add_rms_norm_batch(dr.data_ptr(), du.data_ptr(), ro.data_ptr(), dw.data_ptr(),
                                                           no.data_ptr(), n, batch, EPS, 1, None))
    assert np.array_equal(host(ro, np.uint16), want_r)  # one add, one rounding: exact
    assert np.array_equal(host(no, np.uint16), want_n)
    codes, scales = empty((batch, n // 2), np.uint8), empty((batch, n // 128), np.uint16)
    ro2, no2 = empty((batch, n), np.uint16), empty((batch, n), np.uint16)
    gx.check(L.gfxinfer_launch_residual_add_rms_norm_quantize_i4(dr.data_ptr(), du.data_ptr(), ro2.data_ptr(), dw.data_ptr(),
                                                                 no2.data_ptr(), codes.data_ptr(), scales.data_ptr(),
                                                                 n, batch, EPS, 1, None))
    assert np.array_equal(host(ro2, np.uint16), want_r)
    c, s = orc.quantize_activation_i4(host(no2, np.uint16))
    assert np.array_equal(host(codes), c) and np.array_equal(host(scales, np.uint16), s)


@pytest.mark.parametrize("n,batch,planes", [(5120, 5, 4), (5120, 32, 8), (5120, 1, 2), (6144, 3, 3),
                                            (10240, 2, 4), (640, 7, 5), (5120, 4, 1), (5120, 13, 4),
                                            (5120, 40, 4), (256, 6, 4)])
def test_residual_norm_sums_update_planes(device, gx, orc, n, batch, planes):
    """Planes entry == the plain fused entry on the fp32 sum of the planes taken in
    plane order (bit-exact: same additions, same kernel arithmetic); the residual is
    the oracle's one-rounding add of that sum."""
    rng = np.random.default_rng(n + batch * 7 + planes)
    res = _half(rng.standard_normal((batch, n)))
    upd = (rng.standard_normal((planes, batch, n)) * 0.5).astype(np.float32)
    total = upd[0].copy()
    for p in range(1, planes):
        total += upd[p]
    w = _bf16(np.round(rng.standard_normal(n) * 64) / 1024)
    want_r = np.empty_like(res)
    want_n = np.empty_like(res)
    orc.lib().orc_residual_add_rms_norm(orc.ptr(res), orc.ptr(total), orc.ptr(want_r), orc.ptr(w), orc.ptr(want_n),
                                        n, batch, EPS, 1)
    L = gx.lib()
    dr, dw = dev(res), dev(w)
    outs = []
    for update, count, fn in ((dev(upd), planes, "planes"), (dev(total), 1, "plain")):
        ro, no = empty((batch, n), np.uint16), empty((batch, n), np.uint16)
        codes, scales = empty((batch, n // 2), np.uint8), empty((batch, n // 128), np.uint16)
        say("residual norm", fn, n, batch, planes)
        if fn == "planes":
            gx.check(L.gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes(
                dr.data_ptr(), update.data_ptr(), count, ro.data_ptr(), dw.data_ptr(), no.data_ptr(),
                codes.data_ptr(), scales.data_ptr(), n, batch, EPS, 1, None))
        else:
            gx.check(L.gfxinfer_launch_residual_add_rms_norm_quantize_i4(
                dr.data_ptr(), update.data_ptr(), ro.data_ptr(), dw.data_ptr(), no.data_ptr(),
                codes.data_ptr(), scales.data_ptr(), n, batch, EPS, 1, None))
        outs.append([host(ro, np.uint16), host(no, np.uint16), host(codes), host(scales, np.uint16)])
    assert np.array_equal(outs[0][0], want_r)
    assert np.array_equal(outs[0][1], want_n)
    # register-resident (<= 6144 elements) and generic kernels alike sum in the
    # reference's order, so both entries agree bit for bit
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)
    bad = L.gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes(
        dr.data_ptr(), dr.data_ptr(), 9, dr.data_ptr(), dw.data_ptr(), dr.data_ptr(), dr.data_ptr(),
        dr.data_ptr(), n, batch, EPS, 1, None)
    assert bad == gx.INVALID_ARGUMENT


@pytest.mark.parametrize("batch", [1, 5, 32])
def test_residual_norm_in_place_equals_out_of_place(device, gx, orc, batch):
    """The residual written over its own input (one workgroup per row, every load before
    any store) equals the out-of-place call, which shares each row among several
    workgroups."""
    n, planes = 5120, 4
    rng = np.random.default_rng(500 + batch)
    res = _half(rng.standard_normal((batch, n)))
    upd = (rng.standard_normal((planes, batch, n)) * 0.5).astype(np.float32)
    w = _bf16(np.round(rng.standard_normal(n) * 64) / 1024)
    L = gx.lib()
    du, dw = dev(upd), dev(w)
    outs = []
    for in_place in (False, True):
        dr = dev(res)
        ro = dr if in_place else empty((batch, n), np.uint16)
        no = empty((batch, n), np.uint16)
        codes, scales = empty((batch, n // 2), np.uint8), empty((batch, n // 128), np.uint16)
        say("residual norm in place", in_place, batch)
        gx.check(L.gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes(
            dr.data_ptr(), du.data_ptr(), planes, ro.data_ptr(), dw.data_ptr(), no.data_ptr(),
            codes.data_ptr(), scales.data_ptr(), n, batch, EPS, 1, None))
        outs.append([host(ro, np.uint16), host(no, np.uint16), host(codes), host(scales, np.uint16)])
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("n", [5120, 130, 129, 7168])  # register-resident rows; odd / long: strided
def test_dual_rms_norm_concat(device, gx, orc, n):
    rng = np.random.default_rng(3 + n)
    left, right = _half(rng.standard_normal(n)), _half(rng.standard_normal(n) * 3)
    lw, rw = _bf16(rng.standard_normal(n) * 0.05), _bf16(rng.standard_normal(n) * 0.05)
    want = np.empty(2 * n, np.uint16)
    orc.lib().orc_dual_rms_norm_concat(orc.ptr(left), orc.ptr(lw), orc.ptr(right), orc.ptr(rw), orc.ptr(want), n, EPS, 1)
    out = empty((2 * n,), np.uint16)
    say("dual_rms_norm_concat")
    gx.check(gx.lib().gfxinfer_launch_dual_rms_norm_concat(D_(left), D_(lw), D_(right),
                                                           D_(rw), out.data_ptr(), n, EPS, 1, None))
    assert np.array_equal(host(out, np.uint16), want)


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_mtp_input_equals_gather_dual_norm_quantizer(device, gx, orc, fmt):
    """Embedding gather + dual RMSNorm/concat + A4 quantizer in one launch == the three
    launches: codes, scales and the fp16 concat bit for bit, for a direct and a device
    token id, and zeros for a token past the table."""
    n, rows = 5120, 64
    rng = np.random.default_rng(60 + fmt)
    w = (rng.standard_normal((rows, n)) * 0.05).astype(np.float32)
    _, codes, sc = orc.quantize_group128(w, fmt)
    tcodes, tscales = gx.tile_group128(fmt, codes, sc, rows, n)
    cond = _half(rng.standard_normal(n) * 3)
    ew, cw = _bf16(rng.standard_normal(n) * 0.05), _bf16(rng.standard_normal(n) * 0.05)
    dtc, dts, dcond, dew, dcw = D_(tcodes), D_(tscales), D_(cond), D_(ew), D_(cw)
    L = gx.lib()
    for token, indirect in ((37, False), (5, True), (rows + 3, False)):
        gathered = empty((n,), np.uint16)
        concat = empty((2 * n,), np.uint16)
        a4, s4 = empty((n,), np.uint8), empty((2 * n // 128,), np.uint16)
        say("mtp input pair", fmt, token)
        if token < rows:
            gx.check(L.gfxinfer_launch_lowbit_row_gather_tiled(fmt, dtc, dts, gathered.data_ptr(), token, rows, n, None))
        else:
            gathered.zero_()
        gx.check(L.gfxinfer_launch_dual_rms_norm_concat(gathered.data_ptr(), dew, dcond, dcw, concat.data_ptr(), n,
                                                        EPS, 1, None))
        gx.check(L.gfxinfer_launch_quantize_activation_i4(concat.data_ptr(), a4.data_ptr(), s4.data_ptr(), 2 * n, 1,
                                                          None))
        want = [host(concat, np.uint16), host(a4), host(s4, np.uint16)]
        concat2 = empty((2 * n,), np.uint16)
        a42, s42 = empty((n,), np.uint8), empty((2 * n // 128,), np.uint16)
        ind = dev(np.array([token], np.uint32)) if indirect else None
        say("mtp input fused", fmt, token, indirect)
        gx.check(L.gfxinfer_launch_mtp_input_quantize_i4(
            fmt, dtc, dts, rows, 0 if indirect else token, ind.data_ptr() if indirect else None, dew, dcond, dcw,
            concat2.data_ptr(), a42.data_ptr(), s42.data_ptr(), n, EPS, 1, None))
        assert np.array_equal(host(concat2, np.uint16), want[0])
        assert np.array_equal(host(a42), want[1])
        assert np.array_equal(host(s42, np.uint16), want[2])
    assert L.gfxinfer_launch_mtp_input_quantize_i4(fmt, dtc, dts, rows, 1, None, dew, dcond, dcw, None,
                                                   a42.data_ptr(), s42.data_ptr(), 130, EPS, 1,
                                                   None) == gx.INVALID_ARGUMENT


@pytest.mark.parametrize("mapped", [False, True])
def test_mtp_input_from_keys_equals_reduction_then_input(device, gx, orc, mapped):
    """A draft head run keys-only (fused GEMM argmax with tokens NULL), then the MTP input
    launch that reduces those keys itself, gives the token the fused head's own reduction
    gives (through token_ids or not), writes it, and produces the same codes, scales and
    concat as the MTP input launch given that token."""
    fmt, n, rows, head_rows, limit = 3, 5120, 64, 4096, 4000
    rng = np.random.default_rng(71 + mapped)
    w = (rng.standard_normal((rows, n)) * 0.05).astype(np.float32)
    _, codes, sc = orc.quantize_group128(w, fmt)
    tcodes, tscales = gx.tile_group128(fmt, codes, sc, rows, n)
    hw = (rng.standard_normal((head_rows, n)) * 0.02).astype(np.float32)
    _, hcodes, hsc = orc.quantize_group128(hw, fmt)
    htc, hts = gx.tile_group128(fmt, hcodes, hsc, head_rows, n)
    x16 = _half(rng.standard_normal((1, n)))
    a4, as16 = orc.quantize_activation_i4(x16)
    cond = _half(rng.standard_normal(n) * 3)
    ew, cw = _bf16(rng.standard_normal(n) * 0.05), _bf16(rng.standard_normal(n) * 0.05)
    ids = (np.arange(head_rows, dtype=np.uint32) * 7 + 3) % rows
    dtc, dts, dhtc, dhts, da, das, dcond, dew, dcw, dids = (
        D_(v) for v in (tcodes, tscales, htc, hts, a4, as16, cond, ew, cw, ids))
    ids_ptr = dids if mapped else None
    L = gx.lib()
    work_bytes = L.gfxinfer_gemm_argmax_workspace_bytes(head_rows, 1)
    work = empty((work_bytes // 8,), np.uint64)
    token = empty((1,), np.uint32)
    say("fused head with its reduction, mapped" if mapped else "fused head with its reduction")
    gx.check(L.gfxinfer_launch_gfx950_i4_gemm_argmax(fmt, dhtc, dhts, da, das, None, head_rows, n, 1, limit,
                                                     ids_ptr, work.data_ptr(), work_bytes, token.data_ptr(), None))
    want_token = int(host(token, np.uint32)[0])
    concat, c4, s4 = empty((2 * n,), np.uint16), empty((n,), np.uint8), empty((2 * n // 128,), np.uint16)
    gx.check(L.gfxinfer_launch_mtp_input_quantize_i4(fmt, dtc, dts, rows, want_token, None, dew, dcond, dcw,
                                                     concat.data_ptr(), c4.data_ptr(), s4.data_ptr(), n, EPS, 1,
                                                     None))
    work.zero_()
    say("keys-only head, then MTP input from the keys")
    gx.check(L.gfxinfer_launch_gfx950_i4_gemm_argmax(fmt, dhtc, dhts, da, das, None, head_rows, n, 1, limit,
                                                     ids_ptr, work.data_ptr(), work_bytes, None, None))
    got_token = empty((1,), np.uint32)
    concat2, c42, s42 = empty((2 * n,), np.uint16), empty((n,), np.uint8), empty((2 * n // 128,), np.uint16)
    gx.check(L.gfxinfer_launch_mtp_input_quantize_i4_from_keys(
        fmt, dtc, dts, rows, work.data_ptr(), head_rows // 16, ids_ptr, got_token.data_ptr(), dew, dcond, dcw,
        concat2.data_ptr(), c42.data_ptr(), s42.data_ptr(), n, EPS, 1, None))
    assert int(host(got_token, np.uint32)[0]) == want_token
    assert np.array_equal(host(concat2, np.uint16), host(concat, np.uint16))
    assert np.array_equal(host(c42), host(c4))
    assert np.array_equal(host(s42, np.uint16), host(s4, np.uint16))
    # the oracle's argmax of the same logits picks the same row
    logits = empty((1, head_rows), np.float32)
    gx.check(L.gfxinfer_launch_gfx950_i4_gemm_argmax(fmt, dhtc, dhts, da, das, logits.data_ptr(), head_rows, n, 1,
                                                     limit, None, work.data_ptr(), work_bytes, None, None))
    row = int(np.argmax(host(logits)[0, :limit]))
    assert want_token == (int(ids[row]) if mapped else row)
    assert L.gfxinfer_launch_mtp_input_quantize_i4_from_keys(
        fmt, dtc, dts, rows, work.data_ptr(), head_rows // 16, ids_ptr, None, dew, dcond, dcw, None,
        c42.data_ptr(), s42.data_ptr(), n, EPS, 1, None) == gx.INVALID_ARGUMENT


@pytest.mark.parametrize("batch", [1, 7, 32])
def test_dual_rms_norm_concat_batch_rows_equal_single(device, gx, orc, batch):
    """Each row of the batched launcher is bit-identical to the single-row launcher on
    that row (the batched MTP cache update of a chunked prefill relies on it)."""
    n = 5120
    rng = np.random.default_rng(30 + batch)
    left, right = _half(rng.standard_normal((batch, n))), _half(rng.standard_normal((batch, n)) * 3)
    lw, rw = _bf16(rng.standard_normal(n) * 0.05), _bf16(rng.standard_normal(n) * 0.05)
    dl, dr, dlw, drw = D_(left), D_(right), D_(lw), D_(rw)
    out = empty((batch, 2 * n), np.uint16)
    say("dual_rms_norm_concat_batch", batch)
    gx.check(gx.lib().gfxinfer_launch_dual_rms_norm_concat_batch(dl, dlw, dr, drw, out.data_ptr(), n, batch,
                                                                 EPS, 1, None))
    got = host(out, np.uint16)
    one = empty((2 * n,), np.uint16)
    for r in (0, batch // 2, batch - 1):
        gx.check(gx.lib().gfxinfer_launch_dual_rms_norm_concat(
            dl + r * n * 2, dlw, dr + r * n * 2, drw, one.data_ptr(), n, EPS, 1, None))
        assert np.array_equal(got[r], host(one, np.uint16))
        want = np.empty(2 * n, np.uint16)
        orc.lib().orc_dual_rms_norm_concat(orc.ptr(np.ascontiguousarray(left[r])), orc.ptr(lw),
                                           orc.ptr(np.ascontiguousarray(right[r])), orc.ptr(rw),
                                           orc.ptr(want), n, EPS, 1)
        assert np.array_equal(got[r], want)


@pytest.mark.parametrize("batch", [1, 5, 32])
def test_silu_multiply_quantize(device, gx, orc, batch):
    n = 17408
    rng = np.random.default_rng(20 + batch)
    g = (rng.standard_normal((batch, n)) * 2).astype(np.float32)
    u = rng.standard_normal((batch, n)).astype(np.float32)
    want = np.empty((batch, n), np.uint16)
    orc.lib().orc_silu_multiply(orc.ptr(g), orc.ptr(u), orc.ptr(want), batch * n)
    L = gx.lib()
    dg, du = dev(g), dev(u)
    prod = empty((batch, n), np.uint16)
    say("silu_multiply", batch)
    gx.check(L.gfxinfer_launch_silu_multiply(dg.data_ptr(), du.data_ptr(), prod.data_ptr(), batch * n, None))
    got = host(prod, np.uint16)
    assert _close16(got, want, rel=2.0 ** -10)
    codes, scales = empty((batch, n // 2), np.uint8), empty((batch, n // 128), np.uint16)
    gx.check(L.gfxinfer_launch_silu_multiply_quantize_i4(dg.data_ptr(), du.data_ptr(), codes.data_ptr(), scales.data_ptr(),
                                                         n, batch, None))
    c, s = orc.quantize_activation_i4(got)  # fused kernel == quantizer of the same fp16 products
    gs = host(scales, np.uint16)
    assert np.array_equal(host(codes), c)
    assert np.array_equal(gs, s), np.argwhere(gs != s)[:8]


# ---- GDN ------------------------------------------------------------------------

HK, HV, D = 16, 32, 128
C = 2 * HK * D + HV * D
# BASELINE config 4 (32 value heads) and the reference model's 48 value / 16 key heads
# (qwen38_spec.h:26-29: 10240 conv channels, three value heads per key head).
GDN_SHAPES = [(16, 32), (16, 48)]


def _gdn_inputs(seed, T, hk=HK, hv=HV):
    HK, HV = hk, hv
    C = 2 * HK * D + HV * D
    rng = np.random.default_rng(seed)
    qkv = _half(rng.standard_normal((T, C)))
    z = rng.standard_normal((T, HV * D)).astype(np.float32)
    a = rng.standard_normal((T, HV)).astype(np.float32)
    b = rng.standard_normal((T, HV)).astype(np.float32)
    a_log = _bf16(np.zeros(HV))
    dt_bias = _bf16(np.zeros(HV))
    norm_w = _bf16(np.ones(D))
    s0 = (rng.standard_normal((HV, D, D)) * 0.1).astype(np.float32)
    return qkv, z, a, b, a_log, dt_bias, norm_w, s0


def _gpu_window(gx, d, T, s0, logs=True, hk=HK, hv=HV):
    HK, HV = hk, hv
    L = gx.lib()
    fin = empty((HV, D, D), np.float32)
    out = empty((T, HV * D), np.uint16)
    work = empty((T, HV * D), np.float32)
    kl, dl, yl = (empty((T, HK * D), np.float32), empty((T, HV * D), np.float32), empty((T, HV), np.float32)) if logs else (None, None, None)
    gx.check(L.gfxinfer_launch_gdn_recurrent_decode_block(
        d["qkv"].data_ptr(), d["z"].data_ptr(), d["a"].data_ptr(), d["b"].data_ptr(), d["a_log"].data_ptr(),
        d["dt"].data_ptr(), d["nw"].data_ptr(), s0.data_ptr(), fin.data_ptr(), out.data_ptr(),
        kl.data_ptr() if logs else None, dl.data_ptr() if logs else None, yl.data_ptr() if logs else None,
        T, HK, HV, D, work.data_ptr(), None))
    return fin, out, kl, dl, yl


@pytest.mark.parametrize("HK,HV", GDN_SHAPES)
def test_gdn_window_matches_oracle(device, gx, orc, HK, HV):
    """Hv=32, Hk=16, d=128, T=32 tokens; and the reference model's
    Hv=48 (ratio 3)."""
    T = 32
    qkv, z, a, b, a_log, dt, nw, s0 = _gdn_inputs(41, T, HK, HV)
    want_s = np.empty_like(s0)
    want_o = np.empty((T, HV * D), np.uint16)
    wk, wd, wy = np.empty((T, HK * D), np.float32), np.empty((T, HV * D), np.float32), np.empty((T, HV), np.float32)
    orc.lib().orc_gdn_recurrent(orc.ptr(qkv), orc.ptr(z), orc.ptr(a), orc.ptr(b), orc.ptr(a_log), orc.ptr(dt),
                                orc.ptr(nw), orc.ptr(s0), orc.ptr(want_s), orc.ptr(want_o), orc.ptr(wk), orc.ptr(wd),
                                orc.ptr(wy), T, HK, HV, D)
    d = dict(qkv=dev(qkv), z=dev(z), a=dev(a), b=dev(b), a_log=dev(a_log), dt=dev(dt), nw=dev(nw))
    say("gdn window T=32", HK, HV)
    fin, out, kl, dl, yl = _gpu_window(gx, d, T, dev(s0), hk=HK, hv=HV)
    got_s = host(fin)
    assert np.abs(got_s - want_s).max() <= 1e-5 * max(1.0, np.abs(want_s).max())
    assert np.abs(host(kl) - wk).max() <= 1e-6
    assert np.abs(host(dl) - wd).max() <= 1e-5 * max(1.0, np.abs(wd).max())
    assert np.abs(host(yl) - wy).max() <= 1e-6
    go, wo = _f(host(out, np.uint16)), _f(want_o)
    assert np.abs(go - wo).max() <= 1e-2 * max(1.0, np.abs(wo).max())


def test_gdn_closed_forms(device, gx, orc):
    """beta = 0 (b -> -inf) with decay 1 (a -> -inf): state unchanged; zero state and
    one token: S = k_hat (outer) beta * v."""
    T = 1
    qkv, z, a, b, a_log, dt, nw, s0 = _gdn_inputs(42, T)
    d = dict(qkv=dev(qkv), z=dev(z), a=dev(np.full((T, HV), -1e4, np.float32)), b=dev(np.full((T, HV), -1e4, np.float32)),
             a_log=dev(a_log), dt=dev(dt), nw=dev(nw))
    say("gdn closed form: identity")
    fin, *_ = _gpu_window(gx, d, T, dev(s0))
    assert np.array_equal(host(fin), s0)
    zero = np.zeros_like(s0)
    d["a"], d["b"] = dev(a), dev(b)
    say("gdn closed form: outer product")
    fin, *_ = _gpu_window(gx, d, T, dev(zero))
    q = _f(qkv[0])
    beta = 1 / (1 + np.exp(-b[0].astype(np.float64)))
    for h in (0, 7, 31):
        kh = h // (HV // HK)
        k = q[HK * D + kh * D: HK * D + kh * D + D].astype(np.float64)
        khat = k / np.sqrt((k * k).sum() + 1e-6)
        v = q[2 * HK * D + h * D: 2 * HK * D + h * D + D].astype(np.float64)
        want = np.outer(khat, beta[h] * v)
        assert np.abs(host(fin)[h] - want).max() <= 1e-5


@pytest.mark.parametrize("accepted,HK,HV", [(1, 16, 32), (5, 16, 32), (17, 16, 32), (32, 16, 32),
                                           (3, 16, 48), (29, 16, 48)])
def test_gdn_rollback_equals_prefix_run(device, gx, orc, accepted, HK, HV):
    """restore(A) on the pre-window state == running only the first A tokens, bit for
    bit (same fp32 operations in the same order); also against the oracle replay."""
    T, layers = 32, 2
    C = 2 * HK * D + HV * D
    L = gx.lib()
    conv_states, conv_logs, states = [], [], []
    key_logs, delta_logs, decay_logs, prefix_states, pre = [], [], [], [], []
    for layer in range(layers):
        qkv, z, a, b, a_log, dt, nw, s0 = _gdn_inputs(100 + layer, T, HK, HV)
        d = dict(qkv=dev(qkv), z=dev(z), a=dev(a), b=dev(b), a_log=dev(a_log), dt=dev(dt), nw=dev(nw))
        say("gdn rollback window", accepted, layer, HK, HV)
        _, _, kl, dl, yl = _gpu_window(gx, d, T, dev(s0), hk=HK, hv=HV)
        key_logs.append(host(kl)); delta_logs.append(host(dl)); decay_logs.append(host(yl))
        dp = dict(qkv=dev(qkv[:accepted]), z=dev(z[:accepted]), a=dev(a[:accepted]), b=dev(b[:accepted]),
                  a_log=d["a_log"], dt=d["dt"], nw=d["nw"])
        fin, *_ = _gpu_window(gx, dp, accepted, dev(s0), logs=False, hk=HK, hv=HV)
        prefix_states.append(host(fin))
        pre.append(s0)
        rng = np.random.default_rng(200 + layer)
        conv_states.append(_half(rng.standard_normal((C, 4))))
        conv_logs.append(_half(rng.standard_normal((T, C))))
    st = dev(np.stack(pre))
    cs = dev(np.stack(conv_states))
    say("gdn restore all layers", accepted)
    gx.check(L.gfxinfer_launch_gdn_restore_prefix_all(cs.data_ptr(), st.data_ptr(), D_(np.stack(conv_logs)),
                                                      D_(np.stack(key_logs)), D_(np.stack(delta_logs)),
                                                      D_(np.stack(decay_logs)), C, layers, T, accepted,
                                                      HK, HV, D, None))
    got = host(st)
    for layer in range(layers):
        assert np.array_equal(got[layer], prefix_states[layer])
        want = pre[layer].copy()
        orc.lib().orc_gdn_restore_recurrent(orc.ptr(want), orc.ptr(key_logs[layer]), orc.ptr(delta_logs[layer]),
                                            orc.ptr(decay_logs[layer]), accepted, HK, HV, D)
        assert np.array_equal(got[layer], want)  # same operations, same order
        wc = conv_states[layer].copy()
        orc.lib().orc_gdn_restore_conv(orc.ptr(wc), orc.ptr(conv_logs[layer]), C, accepted)
        assert np.array_equal(host(cs, np.uint16)[layer], wc)


def test_gdn_restore_rejects_bad_accept(device, gx):
    """Accepted counts of 0 or above the logged tokens, and more than 32 logged tokens,
    are rejected before any launch (real buffers, sized for 64 logged tokens)."""
    L = gx.lib()
    layers, logged = 2, 64
    bufs = [empty((layers, C, 4), np.uint16), empty((layers, HV, D, D), np.float32),
            empty((layers, logged, C), np.uint16), empty((layers, logged, HK * D), np.float32),
            empty((layers, logged, HV * D), np.float32), empty((layers, logged, HV), np.float32)]
    ptrs = [b.data_ptr() for b in bufs]
    say("gdn restore rejects bad accepted counts")
    assert L.gfxinfer_launch_gdn_restore_prefix_all(*ptrs, C, layers, 32, 33, HK, HV, D, None) == gx.INVALID_ARGUMENT
    assert L.gfxinfer_launch_gdn_restore_prefix_all(*ptrs, C, layers, 32, 0, HK, HV, D, None) == gx.INVALID_ARGUMENT
    assert L.gfxinfer_launch_gdn_restore_prefix_all(*ptrs, C, layers, 64, 33, HK, HV, D, None) == gx.INVALID_ARGUMENT


@pytest.mark.parametrize("T,in_place", [(32, False), (5, True), (1, True)])
def test_gdn_conv(device, gx, orc, T, in_place):
    rng = np.random.default_rng(5 + T)
    proj = rng.standard_normal((T, C)).astype(np.float32)
    w = _bf16(rng.standard_normal((C, 4)) * 0.5)
    s0 = _half(rng.standard_normal((C, 4)))
    want_f, want_o, want_l = np.empty_like(s0), np.empty((T, C), np.uint16), np.empty((T, C), np.uint16)
    orc.lib().orc_gdn_conv_update(orc.ptr(proj), orc.ptr(w), orc.ptr(s0), orc.ptr(want_f), orc.ptr(want_o),
                                  orc.ptr(want_l), C, T)
    out, log = empty((T, C), np.uint16), empty((T, C), np.uint16)
    state = dev(s0)
    fin = state if in_place else empty((C, 4), np.uint16)
    say("gdn conv", T, "in place" if in_place else "")
    gx.check(gx.lib().gfxinfer_launch_gdn_conv_update_block(D_(proj), D_(w), state.data_ptr(),
                                                            fin.data_ptr(), out.data_ptr(), log.data_ptr(), C, T, None))
    assert np.array_equal(host(fin, np.uint16), want_f)
    assert np.array_equal(host(log, np.uint16), want_l)
    assert _close16(host(out, np.uint16), want_o, rel=2.0 ** -9, atol=1e-4)


def test_gdn_output_quantize(device, gx, orc):
    T = 5
    rng = np.random.default_rng(6)
    mixed = rng.standard_normal((T, HV * D)).astype(np.float32)
    z = rng.standard_normal((T, HV * D)).astype(np.float32)
    w = _bf16(np.ones(D))
    out, codes, scales = empty((T, HV * D), np.uint16), empty((T, HV * D // 2), np.uint8), empty((T, HV), np.uint16)
    say("gdn output quantize")
    gx.check(gx.lib().gfxinfer_launch_gdn_output_quantize_i4(D_(mixed), D_(z), D_(w),
                                                             out.data_ptr(), codes.data_ptr(), scales.data_ptr(), T, HV, D, None))
    o = host(out, np.uint16)
    m = mixed.reshape(T, HV, D).astype(np.float64)
    inv = 1 / np.sqrt((m * m).mean(axis=2, keepdims=True) + 1e-6)
    zz = z.reshape(T, HV, D).astype(np.float64)
    want = (m * inv * (zz / (1 + np.exp(-zz)))).reshape(T, HV * D)
    assert np.abs(_f(o) - want).max() <= 2e-3 * np.abs(want).max()
    c, s = orc.quantize_activation_i4(o)
    assert np.array_equal(host(codes), c) and np.array_equal(host(scales, np.uint16), s)


# ---- attention ---------------------------------------------------------------------

HQ, HKV, AD = 40, 8, 128
# BASELINE config 3 (40/8 x 128) and the reference model's 24/4 x 256 (qwen38_spec.h:22-25).
ATTN_SHAPES = [(40, 8, 128), (24, 4, 256)]


@pytest.mark.parametrize("HQ,HKV,AD", ATTN_SHAPES)
@pytest.mark.parametrize("T,base", [(5, 200), (32, 1000), (1, 64), (32, 4065), (5, 1), (32, 1), (3, 63), (8, 60),
                                    (1, 1), (5, 4065)])
def test_attention_matches_oracle(device, gx, orc, T, base, HQ, HKV, AD):
    capacity = 4096 + 32
    rng = np.random.default_rng(T * 7 + base)
    q = _half(rng.standard_normal((T, HQ, AD)))
    gate = rng.standard_normal((T, HQ, 2 * AD)).astype(np.float32)
    kc = np.zeros((capacity, HKV, AD), np.uint16)
    vc = np.zeros((capacity, HKV, AD), np.uint16)
    n = base + T - 1
    kc[:n] = _half(rng.standard_normal((n, HKV, AD)))
    vc[:n] = _half(rng.standard_normal((n, HKV, AD)))
    want = np.empty((T, HQ, AD), np.uint16)
    orc.lib().orc_gated_attention(orc.ptr(q), orc.ptr(gate), orc.ptr(kc), orc.ptr(vc), orc.ptr(want), base, T, HQ, HKV, AD,
                                  np.float32(1 / np.sqrt(AD)))
    L = gx.lib()
    wb = L.gfxinfer_attention_workspace_bytes(T, HQ, AD, capacity)
    work = empty((wb // 4,), np.float32)
    out = empty((T, HQ, AD), np.uint16)
    say("attention", T, base, HQ, HKV, AD)
    gx.check(L.gfxinfer_launch_gated_attention_decode_block(D_(q), D_(gate), D_(kc),
                                                            D_(vc), out.data_ptr(), base, capacity, T, HQ, HKV,
                                                            AD, work.data_ptr(), wb, None))
    got, w = _f(host(out, np.uint16)), _f(want)
    assert np.abs(got - w).max() <= 1e-2 * max(1.0, np.abs(w).max())
    pos = dev(np.array([base - 1], np.uint64))
    out2 = empty((T, HQ, AD), np.uint16)
    gx.check(L.gfxinfer_launch_gated_attention_decode_block_indirect_position(
        D_(q), D_(gate), D_(kc), D_(vc), out2.data_ptr(), pos.data_ptr(),
        capacity, T, HQ, HKV, AD, work.data_ptr(), wb, None))
    assert np.array_equal(host(out2, np.uint16), host(out, np.uint16))


@pytest.mark.parametrize("HQ,HKV,AD", ATTN_SHAPES)
@pytest.mark.parametrize("T,base", [(5, 200), (32, 1000), (1, 1)])
def test_attention_quantize_equals_attention_then_quantizer(device, gx, T, base, HQ, HKV, AD):
    """Attention with the A4 quantizer in its combine launch == attention followed by
    gfxinfer_launch_quantize_activation_i4 on its fp16 output: same output, codes and
    scales bit for bit (direct and device position)."""
    capacity = 2048
    rng = np.random.default_rng(T + base)
    q = _half(rng.standard_normal((T, HQ, AD)))
    gate = rng.standard_normal((T, HQ, 2 * AD)).astype(np.float32)
    kc = np.zeros((capacity, HKV, AD), np.uint16)
    vc = np.zeros((capacity, HKV, AD), np.uint16)
    n = base + T - 1
    kc[:n] = _half(rng.standard_normal((n, HKV, AD)))
    vc[:n] = _half(rng.standard_normal((n, HKV, AD)))
    L = gx.lib()
    wb = L.gfxinfer_attention_workspace_bytes(T, HQ, AD, capacity)
    work = empty((wb // 4,), np.float32)
    out = empty((T, HQ, AD), np.uint16)
    codes, scales = empty((T, HQ * AD // 2), np.uint8), empty((T, HQ * AD // 128), np.uint16)
    dq, dg, dk, dv = D_(q), D_(gate), D_(kc), D_(vc)
    say("attention then quantizer", T, base, HQ, HKV, AD)
    gx.check(L.gfxinfer_launch_gated_attention_decode_block(dq, dg, dk, dv, out.data_ptr(), base, capacity, T, HQ,
                                                            HKV, AD, work.data_ptr(), wb, None))
    gx.check(L.gfxinfer_launch_quantize_activation_i4(out.data_ptr(), codes.data_ptr(), scales.data_ptr(),
                                                      HQ * AD, T, None))
    want = [host(out, np.uint16), host(codes), host(scales, np.uint16)]
    pos = dev(np.array([base - 1], np.uint64))
    for indirect in (False, True):
        out2 = empty((T, HQ, AD), np.uint16)
        codes2, scales2 = empty((T, HQ * AD // 2), np.uint8), empty((T, HQ * AD // 128), np.uint16)
        say("attention + quantizer", T, base, indirect)
        if indirect:
            gx.check(L.gfxinfer_launch_gated_attention_decode_block_quantize_i4_indirect_position(
                dq, dg, dk, dv, out2.data_ptr(), codes2.data_ptr(), scales2.data_ptr(), pos.data_ptr(), capacity,
                T, HQ, HKV, AD, work.data_ptr(), wb, None))
        else:
            gx.check(L.gfxinfer_launch_gated_attention_decode_block_quantize_i4(
                dq, dg, dk, dv, out2.data_ptr(), codes2.data_ptr(), scales2.data_ptr(), base, capacity,
                T, HQ, HKV, AD, work.data_ptr(), wb, None))
        assert np.array_equal(host(out2, np.uint16), want[0])
        assert np.array_equal(host(codes2), want[1])
        assert np.array_equal(host(scales2, np.uint16), want[2])
    assert L.gfxinfer_launch_gated_attention_decode_block_quantize_i4(
        dq, dg, dk, dv, out.data_ptr(), codes.data_ptr(), None, base, capacity, T, HQ, HKV, AD, work.data_ptr(), wb,
        None) == gx.INVALID_ARGUMENT


@pytest.mark.parametrize("HQ,HKV,AD,rot,T,base", [(40, 8, 128, 32, 5, 1234), (24, 4, 256, 64, 5, 1234),
                                                  (24, 4, 256, 64, 32, 4064), (24, 4, 256, 64, 1, 0)])
def test_qk_norm_rope_and_kv_append(device, gx, orc, HQ, HKV, AD, rot, T, base):
    theta = np.float32(1e7)
    rng = np.random.default_rng(8)
    qin = rng.standard_normal((T, HQ, 2 * AD)).astype(np.float32)
    kin = rng.standard_normal((T, HKV, AD)).astype(np.float32)
    qw, kw = _bf16(rng.standard_normal(AD) * 0.1), _bf16(rng.standard_normal(AD) * 0.1)
    wq, wk = np.empty((T, HQ, AD), np.uint16), np.empty((T, HKV, AD), np.uint16)
    orc.lib().orc_head_norm_rope(orc.ptr(qin), 2 * AD, orc.ptr(qw), orc.ptr(wq), HQ, AD, rot, base, T, theta)
    orc.lib().orc_head_norm_rope(orc.ptr(kin), AD, orc.ptr(kw), orc.ptr(wk), HKV, AD, rot, base, T, theta)
    L = gx.lib()
    qo, ko = empty((T, HQ, AD), np.uint16), empty((T, HKV, AD), np.uint16)
    say("qk norm rope", HQ, HKV, AD, rot, T, base)
    gx.check(L.gfxinfer_launch_qk_rms_norm_rope_block(D_(qin), D_(qw), qo.data_ptr(), HQ, 2 * AD,
                                                      D_(kin), D_(kw), ko.data_ptr(), HKV, AD, AD,
                                                      rot, base, T, theta, None))
    assert _close16(host(qo, np.uint16), wq, rel=2.0 ** -8, atol=2e-3)
    assert _close16(host(ko, np.uint16), wk, rel=2.0 ** -8, atol=2e-3)
    pos = dev(np.array([base], np.uint64))
    qo2, ko2 = empty((T, HQ, AD), np.uint16), empty((T, HKV, AD), np.uint16)
    gx.check(L.gfxinfer_launch_qk_rms_norm_rope_block_indirect_position(
        D_(qin), D_(qw), qo2.data_ptr(), HQ, 2 * AD, D_(kin), D_(kw),
        ko2.data_ptr(), HKV, AD, AD, rot, pos.data_ptr(), T, theta, None))
    assert np.array_equal(host(qo2, np.uint16), host(qo, np.uint16))
    # KV append
    cap = 4096 + 32
    kc, vc = empty((cap, HKV * AD), np.uint16), empty((cap, HKV * AD), np.uint16)
    val = rng.standard_normal((T, HKV * AD)).astype(np.float32)
    gx.check(L.gfxinfer_launch_kv_append_block(ko.data_ptr(), D_(val), kc.data_ptr(), vc.data_ptr(), base, cap,
                                               T, HKV * AD, None))
    assert np.array_equal(host(kc, np.uint16)[base:base + T], host(ko, np.uint16).reshape(T, -1))
    assert np.array_equal(host(vc, np.uint16)[base:base + T], _half(val))
    assert L.gfxinfer_launch_kv_append_block(ko.data_ptr(), D_(val), kc.data_ptr(), vc.data_ptr(), cap - T + 1, cap,
                                             T, HKV * AD, None) == gx.INVALID_ARGUMENT


@pytest.mark.parametrize("HQ,HKV,AD,rot", [(40, 8, 128, 32), (24, 4, 256, 64)])
@pytest.mark.parametrize("T,base", [(5, 1234), (32, 7), (1, 2047)])
def test_fused_rope_kv_append_equals_the_pair(device, gx, T, base, HQ, HKV, AD, rot):
    """Q/K norm + RoPE with the K/V cache append in one launch == the two launches: the
    same q/k outputs and the same cache rows, bit for bit (direct and device position);
    the cache outside the block is untouched."""
    theta, cap = np.float32(1e7), 2048
    rng = np.random.default_rng(80 + T)
    qin = rng.standard_normal((T, HQ, 2 * AD)).astype(np.float32)
    kin = rng.standard_normal((T, HKV, AD)).astype(np.float32)
    qw, kw = _bf16(rng.standard_normal(AD) * 0.1), _bf16(rng.standard_normal(AD) * 0.1)
    val = rng.standard_normal((T, HKV * AD)).astype(np.float32)
    fill = rng.integers(0, 65536, (cap, HKV * AD), dtype=np.uint16)
    L = gx.lib()
    qo, ko = empty((T, HQ, AD), np.uint16), empty((T, HKV, AD), np.uint16)
    kc, vc = dev(fill), dev(fill)
    say("rope + kv append pair", T, base, HQ, HKV, AD)
    gx.check(L.gfxinfer_launch_qk_rms_norm_rope_block(D_(qin), D_(qw), qo.data_ptr(), HQ, 2 * AD,
                                                      D_(kin), D_(kw), ko.data_ptr(), HKV, AD, AD,
                                                      rot, base, T, theta, None))
    gx.check(L.gfxinfer_launch_kv_append_block(ko.data_ptr(), D_(val), kc.data_ptr(), vc.data_ptr(), base, cap,
                                               T, HKV * AD, None))
    want = [host(x, np.uint16) for x in (qo, ko, kc, vc)]
    pos = dev(np.array([base], np.uint64))
    for indirect in (False, True):
        qo2, ko2 = empty((T, HQ, AD), np.uint16), empty((T, HKV, AD), np.uint16)
        kc2, vc2 = dev(fill), dev(fill)
        say("fused rope + kv append", T, base, indirect)
        if indirect:
            gx.check(L.gfxinfer_launch_qk_rms_norm_rope_kv_append_block_indirect_position(
                D_(qin), D_(qw), qo2.data_ptr(), HQ, 2 * AD, D_(kin), D_(kw), ko2.data_ptr(), HKV, AD, AD, rot,
                D_(val), kc2.data_ptr(), vc2.data_ptr(), cap, pos.data_ptr(), T, theta, None))
        else:
            gx.check(L.gfxinfer_launch_qk_rms_norm_rope_kv_append_block(
                D_(qin), D_(qw), qo2.data_ptr(), HQ, 2 * AD, D_(kin), D_(kw), ko2.data_ptr(), HKV, AD, AD, rot,
                D_(val), kc2.data_ptr(), vc2.data_ptr(), cap, base, T, theta, None))
        for got, exp in zip((qo2, ko2, kc2, vc2), want):
            assert np.array_equal(host(got, np.uint16), exp)
    assert L.gfxinfer_launch_qk_rms_norm_rope_kv_append_block(
        D_(qin), D_(qw), qo.data_ptr(), HQ, 2 * AD, D_(kin), D_(kw), ko.data_ptr(), HKV, AD, AD, rot,
        D_(val), kc.data_ptr(), vc.data_ptr(), cap, cap - T + 1, T, theta, None) == gx.INVALID_ARGUMENT
    assert L.gfxinfer_launch_qk_rms_norm_rope_kv_append_block(
        D_(qin), D_(qw), qo.data_ptr(), HQ, 2 * AD, D_(kin), D_(kw), ko.data_ptr(), HKV, AD, AD, rot,
        None, kc.data_ptr(), vc.data_ptr(), cap, base, T, theta, None) == gx.INVALID_ARGUMENT


def test_argmax_ties_and_mapping(device, gx, orc):
    V, T = 151936, 6
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((T, V)).astype(np.float32)
    logits[1, 500] = logits[1, 90000] = 50.0       # tie -> lowest index
    logits[2, V - 1] = 60.0                         # last element
    logits[3, :] = -np.inf
    logits[4, 7] = np.nan
    logits[4, 8] = 70.0
    want = np.empty(T, np.uint32)
    orc.lib().orc_argmax(orc.ptr(logits), V, V, T, None, orc.ptr(want))
    out = empty((T,), np.uint32)
    L = gx.lib()
    say("argmax")
    gx.check(L.gfxinfer_launch_argmax_batch(D_(logits), out.data_ptr(), V, V, T, None))
    got = host(out).view(np.uint32)
    assert np.array_equal(got, want) and got[1] == 500 and got[3] == 0
    ids = (np.arange(98304, dtype=np.uint32) * 7 + 3).astype(np.uint32)
    one = empty((1,), np.uint32)
    gx.check(L.gfxinfer_launch_argmax_mapped(D_(logits[2]), D_(ids), one.data_ptr(), 98304, None))
    assert int(host(one).view(np.uint32)[0]) == int(ids[np.argmax(logits[2, :98304])])


@pytest.mark.parametrize("T,HK,HV", [(1, 16, 32), (3, 16, 32), (5, 16, 32), (32, 16, 32), (1, 16, 48),
                                     (5, 16, 48), (32, 16, 48), (32, 16, 64)])
def test_gdn_conv_window_equals_conv_then_window(device, gx, orc, T, HK, HV):
    """The fused conv + recurrence launch reproduces gdn_conv_update_block followed by
    gdn_recurrent_window bit for bit (states, logs, unnormalized output).  32 value
    heads run 16 state columns per workgroup, 48 and 64 run 32."""
    C = 2 * HK * D + HV * D
    rng = np.random.default_rng(70 + T)
    proj = rng.standard_normal((T, C)).astype(np.float32)
    w = _bf16(rng.standard_normal((C, 4)) * 0.5)
    c0 = _half(rng.standard_normal((C, 4)))
    a = rng.standard_normal((T, HV)).astype(np.float32)
    b = rng.standard_normal((T, HV)).astype(np.float32)
    a_log, dt = _bf16(rng.standard_normal(HV) * 0.5), _bf16(rng.standard_normal(HV) * 0.5)
    s0 = (rng.standard_normal((HV, D, D)) * 0.1).astype(np.float32)
    L = gx.lib()
    dp, dw, dc0, da, db, dal, ddt, ds0 = (D_(x) for x in (proj, w, c0, a, b, a_log, dt, s0))
    outs = []
    for fused in (False, True):
        cf = empty((C, 4), np.uint16)
        clog = empty((T, C), np.uint16)
        sf = empty((HV, D, D), np.float32)
        mixed = empty((T, HV * D), np.float32)
        kl, dl, yl = empty((T, HK * D), np.float32), empty((T, HV * D), np.float32), empty((T, HV), np.float32)
        say("gdn conv window", T, HK, HV, "fused" if fused else "two launches")
        if fused:
            gx.check(L.gfxinfer_launch_gdn_conv_window(dp, dw, dc0, cf.data_ptr(), clog.data_ptr(), da, db, dal, ddt,
                                                       ds0, sf.data_ptr(), mixed.data_ptr(), kl.data_ptr(),
                                                       dl.data_ptr(), yl.data_ptr(), T, HK, HV, D, None))
        else:
            conv = empty((T, C), np.uint16)
            gx.check(L.gfxinfer_launch_gdn_conv_update_block(dp, dw, dc0, cf.data_ptr(), conv.data_ptr(),
                                                             clog.data_ptr(), C, T, None))
            gx.check(L.gfxinfer_launch_gdn_recurrent_window(conv.data_ptr(), da, db, dal, ddt, ds0, sf.data_ptr(),
                                                            mixed.data_ptr(), kl.data_ptr(), dl.data_ptr(),
                                                            yl.data_ptr(), T, HK, HV, D, None))
        outs.append([host(x) for x in (cf, clog, sf, mixed, kl, dl, yl)])
    for got, want in zip(outs[1], outs[0]):
        assert np.array_equal(got, want)
    # the conv state cannot be updated in place
    assert L.gfxinfer_launch_gdn_conv_window(dp, dw, dc0, dc0, None, da, db, dal, ddt, ds0, ds0, ds0, None, None,
                                             None, T, HK, HV, D, None) == gx.INVALID_ARGUMENT


# ---- single-token launchers (qwen_ops.h:83,101,130,217,246,278) ------------------------

def test_single_token_launchers_equal_block_forms(device, gx, orc):
    """The one-token entry points of greedy_step / the MTP proposal give what their block
    launchers give at batch 1, bit for bit, with the states updated in place; the conv
    and recurrent steps also agree with the oracle."""
    L = gx.lib()
    rng = np.random.default_rng(77)
    # conv update, in place
    proj = rng.standard_normal((1, C)).astype(np.float32)
    w = _bf16(rng.standard_normal((C, 4)) * 0.5)
    s0 = _half(rng.standard_normal((C, 4)))
    block_fin, block_out = empty((C, 4), np.uint16), empty((1, C), np.uint16)
    say("single conv update vs block")
    gx.check(L.gfxinfer_launch_gdn_conv_update_block(D_(proj), D_(w), D_(s0), block_fin.data_ptr(),
                                                     block_out.data_ptr(), None, C, 1, None))
    state, out = dev(s0), empty((1, C), np.uint16)
    gx.check(L.gfxinfer_launch_gdn_conv_update(D_(proj), D_(w), state.data_ptr(), out.data_ptr(), C, None))
    assert np.array_equal(host(state, np.uint16), host(block_fin, np.uint16))
    assert np.array_equal(host(out, np.uint16), host(block_out, np.uint16))
    want_f, want_o = np.empty_like(s0), np.empty((1, C), np.uint16)
    orc.lib().orc_gdn_conv_update(orc.ptr(proj), orc.ptr(w), orc.ptr(s0), orc.ptr(want_f), orc.ptr(want_o),
                                  None, C, 1)
    assert np.array_equal(host(state, np.uint16), want_f)
    # recurrent decode, in place
    qkv, z, a, b, a_log, dt, nw, r0 = _gdn_inputs(78, 1)
    d = dict(qkv=dev(qkv), z=dev(z), a=dev(a), b=dev(b), a_log=dev(a_log), dt=dev(dt), nw=dev(nw))
    say("single recurrent decode vs block")
    fin, block_o, *_ = _gpu_window(gx, d, 1, dev(r0), logs=False)
    rs, o, work = dev(r0), empty((1, HV * D), np.uint16), empty((1, HV * D), np.float32)
    gx.check(L.gfxinfer_launch_gdn_recurrent_decode(
        d["qkv"].data_ptr(), d["z"].data_ptr(), d["a"].data_ptr(), d["b"].data_ptr(), d["a_log"].data_ptr(),
        d["dt"].data_ptr(), d["nw"].data_ptr(), rs.data_ptr(), o.data_ptr(), HK, HV, D, work.data_ptr(), None))
    assert np.array_equal(host(rs), host(fin))
    assert np.array_equal(host(o, np.uint16), host(block_o, np.uint16))
    want_s, want_out = np.empty_like(r0), np.empty((1, HV * D), np.uint16)
    orc.lib().orc_gdn_recurrent(orc.ptr(qkv), orc.ptr(z), orc.ptr(a), orc.ptr(b), orc.ptr(a_log), orc.ptr(dt),
                                orc.ptr(nw), orc.ptr(r0), orc.ptr(want_s), orc.ptr(want_out),
                                None, None, None, 1, HK, HV, D)
    assert np.abs(host(rs) - want_s).max() <= 1e-5 * max(1.0, np.abs(want_s).max())
    # restore of one layer == restore_prefix_all over one layer
    T, accepted = 8, 5
    qkv, z, a, b, a_log, dt, nw, r0 = _gdn_inputs(79, T)
    d = dict(qkv=dev(qkv), z=dev(z), a=dev(a), b=dev(b), a_log=dev(a_log), dt=dev(dt), nw=dev(nw))
    _, _, kl, dl, yl = _gpu_window(gx, d, T, dev(r0))
    clog = _half(rng.standard_normal((T, C)))
    cs0 = _half(rng.standard_normal((C, 4)))
    st_all, cs_all, st_one, cs_one = dev(r0), dev(cs0), dev(r0), dev(cs0)
    say("single restore vs all-layer restore")
    gx.check(L.gfxinfer_launch_gdn_restore_prefix_all(cs_all.data_ptr(), st_all.data_ptr(), D_(clog), kl.data_ptr(),
                                                      dl.data_ptr(), yl.data_ptr(), C, 1, T, accepted, HK, HV, D,
                                                      None))
    gx.check(L.gfxinfer_launch_gdn_restore_prefix(cs_one.data_ptr(), st_one.data_ptr(), D_(clog), kl.data_ptr(),
                                                  dl.data_ptr(), yl.data_ptr(), C, accepted, HK, HV, D, None))
    assert np.array_equal(host(st_one), host(st_all))
    assert np.array_equal(host(cs_one, np.uint16), host(cs_all, np.uint16))
    assert L.gfxinfer_launch_gdn_restore_prefix(cs_one.data_ptr(), st_one.data_ptr(), D_(clog), kl.data_ptr(),
                                                dl.data_ptr(), yl.data_ptr(), C, 0, HK, HV, D, None) == gx.INVALID_ARGUMENT
    # K/V append at one position
    capacity, pos, row = 64, 17, HKV * AD
    key = _half(rng.standard_normal((1, row)))
    value = rng.standard_normal((1, row)).astype(np.float32)
    kc1, vc1 = empty((capacity, row), np.uint16), empty((capacity, row), np.uint16)
    kc2, vc2 = empty((capacity, row), np.uint16), empty((capacity, row), np.uint16)
    say("single kv append vs block")
    gx.check(L.gfxinfer_launch_kv_append_block(D_(key), D_(value), kc1.data_ptr(), vc1.data_ptr(), pos, capacity, 1,
                                               row, None))
    gx.check(L.gfxinfer_launch_kv_append(D_(key), D_(value), kc2.data_ptr(), vc2.data_ptr(), pos, capacity, row, None))
    assert np.array_equal(host(kc1, np.uint16), host(kc2, np.uint16))
    assert np.array_equal(host(vc1, np.uint16), host(vc2, np.uint16))
    assert np.array_equal(host(kc2, np.uint16)[pos], key[0])
    assert L.gfxinfer_launch_kv_append(D_(key), D_(value), kc2.data_ptr(), vc2.data_ptr(), capacity, capacity, row,
                                       None) == gx.INVALID_ARGUMENT
    # attention of one token over token_count positions
    capacity, count = 4096 + 32, 1000
    q = _half(rng.standard_normal((1, HQ, AD)))
    gate = rng.standard_normal((1, HQ, 2 * AD)).astype(np.float32)
    kc = np.zeros((capacity, HKV, AD), np.uint16)
    vc = np.zeros((capacity, HKV, AD), np.uint16)
    kc[:count] = _half(rng.standard_normal((count, HKV, AD)))
    vc[:count] = _half(rng.standard_normal((count, HKV, AD)))
    wb = L.gfxinfer_attention_workspace_bytes(1, HQ, AD, capacity)
    work = empty((wb // 4,), np.float32)
    o1, o2 = empty((1, HQ, AD), np.uint16), empty((1, HQ, AD), np.uint16)
    say("single attention vs block")
    args = (D_(q), D_(gate), D_(kc), D_(vc))
    gx.check(L.gfxinfer_launch_gated_attention_decode_block(*args, o1.data_ptr(), count, capacity, 1, HQ, HKV, AD,
                                                            work.data_ptr(), wb, None))
    gx.check(L.gfxinfer_launch_gated_attention_decode(*args, o2.data_ptr(), count, capacity, HQ, HKV, AD,
                                                      work.data_ptr(), wb, None))
    assert np.array_equal(host(o1, np.uint16), host(o2, np.uint16))
    want = np.empty((1, HQ, AD), np.uint16)
    orc.lib().orc_gated_attention(orc.ptr(q), orc.ptr(gate), orc.ptr(kc), orc.ptr(vc), orc.ptr(want), count, 1, HQ,
                                  HKV, AD, np.float32(1 / np.sqrt(AD)))
    assert np.abs(_f(host(o2, np.uint16)) - _f(want)).max() <= 1e-2 * max(1.0, np.abs(_f(want)).max())
    # argmax of one row, ties to the lowest index
    V = 151936
    logits = rng.standard_normal(V).astype(np.float32)
    logits[[9000, 120000]] = 50.0
    token = empty((1,), np.uint32)
    say("single argmax")
    gx.check(L.gfxinfer_launch_argmax(D_(logits), token.data_ptr(), V, None))
    assert int(host(token, np.uint32)[0]) == 9000
