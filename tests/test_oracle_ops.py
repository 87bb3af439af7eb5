"""CPU pinning of the decoder-op half of the oracle (oracle/oracle.c: norms, SwiGLU,
GDN conv / gated delta rule / restore, Q/K norm + RoPE, KV append, gated attention,
argmax, acceptance).

The reference has no CPU implementation of these (they exist only as gfx1200 kernels),
so each oracle function is pinned by what the mathematics fixes: closed forms of
special parameter values, invariants between functions, and reductions to textbook
routines evaluated independently in float64 numpy.  Each case is chosen so that a
plausible slip (a dropped term, a sign, a transposed state, a wrong head mapping, an
off-by-one shift) fails it."""
import ctypes

import numpy as np
import pytest

P = ctypes.c_void_p


def _h(x):
    from oracle import oracle as O
    return O.f32_to_f16_bits(np.asarray(x, np.float32))


def _f(bits):
    from oracle import oracle as O
    return O.f16_bits_to_f32(bits).astype(np.float64)


def _bf(x):
    from oracle import oracle as O
    return O.f32_to_bf16_bits(np.asarray(x, np.float32))


def _bff(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float64)


def _ulps16(a_bits, want):
    """Distance in fp16 units (of the wanted value's binade) between a and want."""
    a = _f(a_bits)
    want = np.asarray(want, np.float64)
    ulp = np.maximum(np.abs(want), 2.0 ** -14) * 2.0 ** -10
    return np.abs(a - want) / ulp


def _silu(x):
    return x / (1.0 + np.exp(-x))


# ---- RMSNorm family (qwen_ops.hip:31-106, 176-217) ------------------------------

@pytest.mark.parametrize("unit", [1, 0])
def test_rms_norm_is_textbook(orc, unit):
    rng = np.random.default_rng(1)
    n, b = 512, 3
    x = _h(rng.standard_normal((b, n)) * 3)
    w = _bf(rng.standard_normal(n) * 0.3)
    out = np.empty((b, n), np.uint16)
    orc.lib().orc_rms_norm(orc.ptr(x), orc.ptr(w), orc.ptr(out), n, b, ctypes.c_float(1e-6), unit)
    xf = _f(x)
    scale = _bff(w) + (1.0 if unit else 0.0)
    want = xf / np.sqrt((xf ** 2).mean(1, keepdims=True) + 1e-6) * scale
    assert _ulps16(out, want).max() <= 1.0


def _reference_kernel_norm(x16, w16, eps, unit, sequential=False):
    """The reference's rms_norm kernel (qwen_ops.hip:31-63) simulated thread by thread:
    256 threads with per-thread fmaf chains, wave32 __shfl_down trees (a lane whose
    source is past its 32-lane segment keeps its own value), wave 0's tree over the eight
    wave sums, then 1/sqrt correctly rounded and fp16(x * inverse * (1 + w)).  fmaf is
    emulated in float64, exact for the magnitudes the caller uses (squares and partial
    sums within 2^29 of each other), then rounded once to float32."""
    x = x16.view(np.float16).astype(np.float32)
    n = x.size
    lanes = np.zeros(256, np.float32)
    for t in range(256):
        s = np.float32(0.0)
        for i in range(t, n, 256):
            s = np.float32(np.float64(x[i]) * np.float64(x[i]) + np.float64(s))
        lanes[t] = s

    def shfl_tree(v):  # v: 32 lanes; returns lane 0 after += shfl_down 16, 8, 4, 2, 1
        v = v.copy()
        for d in (16, 8, 4, 2, 1):
            src = np.array([v[l + d] if l + d < 32 else v[l] for l in range(32)], np.float32)
            v = (v + src).astype(np.float32)
        return v[0]

    waves = np.array([shfl_tree(lanes[32 * g:32 * g + 32]) for g in range(8)], np.float32)
    total = shfl_tree(np.concatenate([waves, np.zeros(24, np.float32)]))
    if sequential:  # a planted mistake: one fmaf chain over the whole row
        total = np.float32(0.0)
        for v in x:
            total = np.float32(np.float64(v) * np.float64(v) + np.float64(total))
    inverse = np.float32(1.0) / np.float32(np.sqrt(np.float32(total / np.float32(n) + np.float32(eps))))
    scale = (w16.astype(np.uint32) << 16).view(np.float32) + np.float32(1.0 if unit else 0.0)
    return ((x * inverse).astype(np.float32) * scale).astype(np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("n", [5120, 300, 7, 256])
def test_rms_norm_sums_in_the_reference_kernel_order(orc, n):
    """orc_rms_norm == the thread-level simulation of the reference kernel, bit for bit;
    a row whose sequential fmaf sum differs from the kernel's tree sum proves the
    comparison sees the order."""
    rng = np.random.default_rng(n)
    mags = rng.uniform(0.25, 4.0, n) * rng.choice([-1.0, 1.0], n)
    x = _h(mags)
    w = _bf(rng.standard_normal(n) * 0.05)
    out = np.empty(n, np.uint16)
    orc.lib().orc_rms_norm(orc.ptr(x), orc.ptr(w), orc.ptr(out), n, 1, ctypes.c_float(1e-6), 1)
    assert np.array_equal(out, _reference_kernel_norm(x, w, 1e-6, True))
    if n == 5120:  # the comparison distinguishes the summation orders
        assert not np.array_equal(out, _reference_kernel_norm(x, w, 1e-6, True, sequential=True))


def test_residual_add_norm_normalizes_the_rounded_sum(orc):
    rng = np.random.default_rng(2)
    n, b = 384, 2
    res = _h(rng.standard_normal((b, n)))
    upd = (rng.standard_normal((b, n)) * 5).astype(np.float32)
    w = _bf(rng.standard_normal(n) * 0.1)
    r_out, normed, direct = (np.empty((b, n), np.uint16) for _ in range(3))
    orc.lib().orc_residual_add_rms_norm(orc.ptr(res), orc.ptr(upd), orc.ptr(r_out), orc.ptr(w), orc.ptr(normed),
                                        n, b, ctypes.c_float(1e-6), 1)
    # r = fp16(fp16 res + fp32 upd): the sum is rounded once, from the exact sum
    assert np.array_equal(r_out, _h(_f(res) + upd.astype(np.float64)))
    orc.lib().orc_rms_norm(orc.ptr(r_out), orc.ptr(w), orc.ptr(direct), n, b, ctypes.c_float(1e-6), 1)
    assert np.array_equal(normed, direct)


def test_dual_norm_is_two_norms_side_by_side(orc):
    rng = np.random.default_rng(3)
    n = 256
    left, right = _h(rng.standard_normal(n)), _h(rng.standard_normal(n) * 4)
    wl, wr = _bf(rng.standard_normal(n) * 0.1), _bf(rng.standard_normal(n) * 0.1)
    out, a, b = np.empty(2 * n, np.uint16), np.empty(n, np.uint16), np.empty(n, np.uint16)
    orc.lib().orc_dual_rms_norm_concat(orc.ptr(left), orc.ptr(wl), orc.ptr(right), orc.ptr(wr), orc.ptr(out),
                                       n, ctypes.c_float(1e-6), 1)
    orc.lib().orc_rms_norm(orc.ptr(left), orc.ptr(wl), orc.ptr(a), n, 1, ctypes.c_float(1e-6), 1)
    orc.lib().orc_rms_norm(orc.ptr(right), orc.ptr(wr), orc.ptr(b), n, 1, ctypes.c_float(1e-6), 1)
    assert np.array_equal(out, np.concatenate([a, b]))


# ---- SwiGLU (qwen_ops.hip:108-163) ----------------------------------------------

def test_silu_multiply_is_textbook_and_feeds_the_quantizer(orc):
    rng = np.random.default_rng(4)
    b, n = 3, 512
    g = (rng.standard_normal((b, n)) * 4).astype(np.float32)
    u = rng.standard_normal((b, n)).astype(np.float32)
    g[0, :4] = [0.0, -80.0, 80.0, 1e-3]
    out = np.empty((b, n), np.uint16)
    orc.lib().orc_silu_multiply(orc.ptr(g), orc.ptr(u), orc.ptr(out), b * n)
    want = _silu(g.astype(np.float64)) * u
    assert _ulps16(out, want).max() <= 1.0
    assert _f(out)[0, 0] == 0.0 and abs(_f(out)[0, 1]) < 1e-30
    codes, scales = np.empty((b, n // 2), np.uint8), np.empty((b, n // 128), np.uint16)
    assert orc.lib().orc_silu_multiply_quantize_i4(orc.ptr(g), orc.ptr(u), orc.ptr(codes), orc.ptr(scales), n, b) == 0
    c2, s2 = orc.quantize_activation_i4(out)
    assert np.array_equal(codes, c2) and np.array_equal(scales, s2)


# ---- GDN causal conv (qwen_ops.hip:219-261) -------------------------------------

def _conv(orc, proj, w, s0, C, T):
    fin, out, log = np.empty((C, 4), np.uint16), np.empty((T, C), np.uint16), np.empty((T, C), np.uint16)
    orc.lib().orc_gdn_conv_update(orc.ptr(proj), orc.ptr(w), orc.ptr(s0), orc.ptr(fin), orc.ptr(out),
                                  orc.ptr(log), C, T)
    return fin, out, log


def test_gdn_conv_taps_shift_and_log(orc):
    rng = np.random.default_rng(5)
    C, T = 64, 6
    proj = rng.standard_normal((T, C)).astype(np.float32)
    s0 = _h(rng.standard_normal((C, 4)))
    x = np.concatenate([_f(s0).T, _f(_h(proj))], axis=0)  # x[-4..T-1] as rows 0..T+3
    for tap in range(4):
        w = np.zeros((C, 4), np.float32)
        w[:, tap] = 1.0
        fin, out, log = _conv(orc, proj, _bf(w), s0, C, T)
        # tap 3 multiplies the newest input; tap 0 the input three tokens back
        want = _silu(x[1 + tap:1 + tap + T])
        assert _ulps16(out, want).max() <= 1.0, tap
        assert np.array_equal(log, _h(proj))
        assert np.array_equal(fin, _h(x[T:T + 4].T))


def test_gdn_conv_matches_window_sum_and_restore(orc):
    rng = np.random.default_rng(6)
    C, T = 96, 9
    proj = rng.standard_normal((T, C)).astype(np.float32)
    w = _bf(rng.standard_normal((C, 4)) * 0.5)
    s0 = _h(rng.standard_normal((C, 4)))
    fin, out, log = _conv(orc, proj, w, s0, C, T)
    x = np.concatenate([_f(s0).T, _f(_h(proj))], axis=0)
    wf = _bff(w)
    conv = sum(x[1 + tap:1 + tap + T] * wf[:, tap] for tap in range(4))
    assert _ulps16(out, _silu(conv)).max() <= 2.0
    for A in (1, 4, T):
        state = s0.copy()
        orc.lib().orc_gdn_restore_conv(orc.ptr(state), orc.ptr(log), C, A)
        prefix_fin, _, _ = _conv(orc, np.ascontiguousarray(proj[:A]), w, s0, C, A)
        assert np.array_equal(state, prefix_fin), A


# ---- Gated delta rule (qwen_ops.hip:263-411, 413-539) ---------------------------

class _Gdn:
    def __init__(self, Hk, Hv, d, T, seed):
        rng = np.random.default_rng(seed)
        self.Hk, self.Hv, self.d, self.T = Hk, Hv, d, T
        C = 2 * Hk * d + Hv * d
        self.qkv = _h(rng.standard_normal((T, C)))
        self.z = rng.standard_normal((T, Hv * d)).astype(np.float32)
        self.a = rng.standard_normal((T, Hv)).astype(np.float32)
        self.b = rng.standard_normal((T, Hv)).astype(np.float32)
        self.a_log = _bf(rng.standard_normal(Hv) * 0.5)
        self.dt = _bf(rng.standard_normal(Hv) * 0.5)
        self.norm = _bf(1.0 + rng.standard_normal(d) * 0.1)
        self.S0 = (rng.standard_normal((Hv, d, d)) * 0.1).astype(np.float32)

    def q(self, t, kh):
        return _f(self.qkv[t, kh * self.d:(kh + 1) * self.d])

    def k(self, t, kh):
        o = self.Hk * self.d
        return _f(self.qkv[t, o + kh * self.d:o + (kh + 1) * self.d])

    def v(self, t, h):
        o = 2 * self.Hk * self.d
        return _f(self.qkv[t, o + h * self.d:o + (h + 1) * self.d])

    def run(self, orc, S0=None, T=None, logs=False):
        T = self.T if T is None else T
        S0 = self.S0 if S0 is None else S0
        Hv, d, Hk = self.Hv, self.d, self.Hk
        S = np.empty_like(S0)
        out = np.empty((T, Hv * d), np.uint16)
        kl = np.zeros((T, Hk * d), np.float32) if logs else None
        dl = np.zeros((T, Hv * d), np.float32) if logs else None
        gl = np.zeros((T, Hv), np.float32) if logs else None
        orc.lib().orc_gdn_recurrent(orc.ptr(np.ascontiguousarray(self.qkv[:T])), orc.ptr(np.ascontiguousarray(self.z[:T])),
                                    orc.ptr(np.ascontiguousarray(self.a[:T])), orc.ptr(np.ascontiguousarray(self.b[:T])),
                                    orc.ptr(self.a_log), orc.ptr(self.dt), orc.ptr(self.norm), orc.ptr(S0), orc.ptr(S),
                                    orc.ptr(out), orc.ptr(kl), orc.ptr(dl), orc.ptr(gl), T, Hk, Hv, d)
        return (S, out, kl, dl, gl) if logs else (S, out)


def test_gdn_no_write_when_beta_zero_and_no_decay(orc):
    g = _Gdn(2, 4, 8, 1, 7)
    g.b[:] = -1e4       # beta = sigmoid(b) = 0
    g.a[:] = -1e4       # softplus(a + dt) = 0  ->  decay = exp(-0) = 1
    S, out = g.run(orc)
    assert np.array_equal(S, g.S0)
    for h in range(g.Hv):
        kh = h // (g.Hv // g.Hk)
        q = g.q(0, kh)
        qn = q / np.sqrt((q ** 2).sum() + 1e-6) / np.sqrt(g.d)
        o = g.S0[h].astype(np.float64).T @ qn                      # S is [k][v]: o = S^T q
        gate = _silu(g.z[0, h * g.d:(h + 1) * g.d].astype(np.float64))
        want = o / np.sqrt((o ** 2).mean() + 1e-6) * _bff(g.norm) * gate
        assert _ulps16(out[0, h * g.d:(h + 1) * g.d], want).max() <= 2.0, h


@pytest.mark.parametrize("a_value", [-1.5, 0.3, 25.0])
def test_gdn_decay_is_exp_of_minus_exp_alog_softplus(orc, a_value):
    g = _Gdn(1, 2, 8, 1, 8)
    g.b[:] = -1e4
    g.a[:] = a_value
    S, _ = g.run(orc)
    for h in range(g.Hv):
        x = a_value + _bff(g.dt)[h]
        softplus = x if x > 20 else np.log1p(np.exp(x))           # threshold 20 as qwen_ops.hip
        decay = np.exp(-np.exp(_bff(g.a_log)[h]) * softplus)
        np.testing.assert_allclose(S[h], g.S0[h] * decay, rtol=2e-6, atol=1e-30)


def test_gdn_first_write_is_key_outer_beta_value(orc):
    g = _Gdn(2, 4, 8, 1, 9)          # key head of value head h is h // 2
    S, _ = g.run(orc, S0=np.zeros_like(g.S0))
    for h in range(g.Hv):
        k = g.k(0, h // 2)
        kn = k / np.sqrt((k ** 2).sum() + 1e-6)
        beta = 1.0 / (1.0 + np.exp(-g.b[0, h]))
        np.testing.assert_allclose(S[h], np.outer(kn, beta * g.v(0, h)), rtol=1e-5, atol=1e-6)


def test_gdn_unit_beta_recalls_value_exactly(orc):
    g = _Gdn(1, 2, 16, 1, 10)
    g.b[:] = 1e4    # beta = 1
    g.a[:] = -1e4   # decay = 1
    S, _ = g.run(orc)
    for h in range(g.Hv):
        k = g.k(0, 0)
        kn = k / np.sqrt((k ** 2).sum() + 1e-6)
        np.testing.assert_allclose(S[h].astype(np.float64).T @ kn, g.v(0, h), rtol=0, atol=2e-4)


def test_gdn_logs_replay_to_the_prefix_state(orc):
    g = _Gdn(2, 4, 16, 6, 11)
    S, out, kl, dl, gl = g.run(orc, logs=True)
    for A in (1, 3, 6):
        state = g.S0.copy()
        orc.lib().orc_gdn_restore_recurrent(orc.ptr(state), orc.ptr(kl), orc.ptr(dl), orc.ptr(gl), A,
                                            g.Hk, g.Hv, g.d)
        prefix, _ = g.run(orc, T=A)
        assert np.array_equal(state, prefix), A


# ---- Q/K norm + partial RoPE (qwen_ops.hip:599-676) -----------------------------

def _rope(orc, x, w, heads, hd, rotary, pos, tokens, theta=1e7):
    out = np.empty((tokens, heads, hd), np.uint16)
    orc.lib().orc_head_norm_rope(orc.ptr(x), 2 * hd, orc.ptr(w), orc.ptr(out), heads, hd, rotary,
                                 ctypes.c_uint64(pos), tokens, ctypes.c_float(theta))
    return out


def test_rope_is_textbook_rotate_half(orc):
    rng = np.random.default_rng(12)
    heads, hd, rotary, T, pos = 3, 128, 64, 4, 1000
    x = rng.standard_normal((T, heads, 2 * hd)).astype(np.float32)   # query half, then gate half
    w = _bf(rng.standard_normal(hd) * 0.1)
    out = _rope(orc, x, w, heads, hd, rotary, pos, T)
    xs = x[:, :, :hd].astype(np.float64)
    n = xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + 1e-6) * (1.0 + _bff(w))
    want = n.copy()
    half = rotary // 2
    for t in range(T):
        for i in range(half):
            angle = (pos + t) * 1e7 ** (-2.0 * i / rotary)
            c, s = np.cos(angle), np.sin(angle)
            want[t, :, i] = n[t, :, i] * c - n[t, :, i + half] * s
            want[t, :, i + half] = n[t, :, i + half] * c + n[t, :, i] * s
    err = np.abs(_f(out) - want)
    assert err.max() <= 2e-3 * np.abs(want).max()
    assert np.array_equal(out[..., rotary:], _h(n[..., rotary:]))   # past the rotary dims: norm only


def test_rope_position_zero_is_identity(orc):
    rng = np.random.default_rng(13)
    x = rng.standard_normal((1, 2, 256)).astype(np.float32)
    w = _bf(np.zeros(128))
    out = _rope(orc, x, w, 2, 128, 64, 0, 1)
    xs = x[:, :, :128].astype(np.float64)
    assert _ulps16(out, xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + 1e-6)).max() <= 1.0


# ---- KV append + gated attention (qwen_ops.hip:678-766) -------------------------

def test_kv_append_places_rows(orc):
    kv, T, cap, pos = 256, 3, 16, 5
    key = _h(np.arange(T * kv).reshape(T, kv) % 97)
    val = (np.arange(T * kv).reshape(T, kv) % 89).astype(np.float32)
    kc, vc = np.zeros((cap, kv), np.uint16), np.zeros((cap, kv), np.uint16)
    orc.lib().orc_kv_append(orc.ptr(key), orc.ptr(val), orc.ptr(kc), orc.ptr(vc), pos, kv, T)
    assert np.array_equal(kc[pos:pos + T], key) and np.array_equal(vc[pos:pos + T], _h(val))
    assert not kc[:pos].any() and not kc[pos + T:].any()


def test_gated_attention_is_textbook_causal_gqa_softmax(orc):
    rng = np.random.default_rng(14)
    T, Hq, Hkv, hd, base = 3, 4, 2, 128, 5
    ctx = base + T
    q = _h(rng.standard_normal((T, Hq, hd)))
    gate = rng.standard_normal((T, Hq, 2 * hd)).astype(np.float32)
    kc, vc = _h(rng.standard_normal((ctx, Hkv, hd))), _h(rng.standard_normal((ctx, Hkv, hd)))
    out = np.empty((T, Hq, hd), np.uint16)
    scale = 1.0 / np.sqrt(hd)
    orc.lib().orc_gated_attention(orc.ptr(q), orc.ptr(gate), orc.ptr(kc), orc.ptr(vc), orc.ptr(out), base, T, Hq,
                                  Hkv, hd, ctypes.c_float(scale))
    for t in range(T):
        n = base + t                                           # token t sees base + t positions
        for h in range(Hq):
            kvh = h // (Hq // Hkv)
            s = (_f(kc[:n, kvh]) @ _f(q[t, h])) * scale
            p = np.exp(s - s.max())
            o = (p / p.sum()) @ _f(vc[:n, kvh])
            want = o / (1.0 + np.exp(-gate[t, h, hd:].astype(np.float64)))
            assert np.abs(_f(out[t, h]) - want).max() <= 2e-3 * max(1.0, np.abs(want).max()), (t, h)


def test_gated_attention_single_position_returns_gated_value(orc):
    hd = 128
    rng = np.random.default_rng(15)
    q = _h(rng.standard_normal((1, 1, hd)) * 30)
    gate = rng.standard_normal((1, 1, 2 * hd)).astype(np.float32)
    kc, vc = _h(rng.standard_normal((1, 1, hd))), _h(rng.standard_normal((1, 1, hd)))
    out = np.empty((1, 1, hd), np.uint16)
    orc.lib().orc_gated_attention(orc.ptr(q), orc.ptr(gate), orc.ptr(kc), orc.ptr(vc), orc.ptr(out), 1, 1, 1, 1,
                                  hd, ctypes.c_float(1.0 / np.sqrt(hd)))
    want = _f(vc[0, 0]) / (1.0 + np.exp(-gate[0, 0, hd:].astype(np.float64)))
    assert _ulps16(out[0, 0], want).max() <= 1.0


# ---- argmax + acceptance (qwen_ops.hip:768-807, qwen_runtime.cpp:1497-1501) -----

def test_argmax_first_maximum_nan_skipped_and_mapped(orc):
    rng = np.random.default_rng(16)
    rows, V, stride = 5, 1000, 1024
    x = rng.standard_normal((rows, stride)).astype(np.float32)
    x[1, 10] = x[1, 700] = 50.0                          # tie -> lower index
    x[2, :] = np.nan
    x[2, 33] = 3.0                                       # NaN never wins
    x[3, :] = -np.inf                                    # nothing beats -inf -> index 0
    x[4, 999] = 99.0
    x[4, 1000] = 1000.0                                  # beyond the vocabulary
    out = np.empty(rows, np.uint32)
    orc.lib().orc_argmax(orc.ptr(x), V, stride, rows, None, orc.ptr(out))
    assert list(out) == [int(np.argmax(x[0, :V])), 10, 33, 0, 999]
    ids = (np.arange(stride, dtype=np.uint32) * 7 + 1)
    orc.lib().orc_argmax(orc.ptr(x), V, stride, rows, orc.ptr(ids), orc.ptr(out))
    assert out[1] == ids[10] and out[3] == ids[0]


def test_accept_is_first_mismatch(orc):
    def accept(d, t):
        d, t = np.asarray(d, np.uint32), np.asarray(t, np.uint32)
        return int(orc.lib().orc_accept(orc.ptr(d), orc.ptr(t), len(d)))
    assert accept([1, 2, 3], [1, 2, 3, 4]) == 3
    assert accept([1, 2, 3], [1, 9, 3, 4]) == 1
    assert accept([5], [4, 4]) == 0
    assert accept([1, 2, 3, 4], [1, 2, 3, 0, 7]) == 3


def test_gdn_decay_applies_before_the_delta_update(orc):
    """With beta = 1 the write recalls v exactly only if the state is decayed before
    the memory read-out (S <- S*decay; delta = v - S^T k; S += k delta^T)."""
    g = _Gdn(1, 2, 16, 1, 17)
    g.b[:] = 1e4
    g.a[:] = 0.7    # decay well below 1
    S, _ = g.run(orc)
    for h in range(g.Hv):
        k = g.k(0, 0)
        kn = k / np.sqrt((k ** 2).sum() + 1e-6)
        np.testing.assert_allclose(S[h].astype(np.float64).T @ kn, g.v(0, h), rtol=0, atol=2e-4)


def test_gdn_query_scale_shows_when_output_is_below_epsilon(orc):
    """The RMS norm of the head output hides the 1/sqrt(d) query scale unless mean(o^2)
    is far below its epsilon 1e-6; then out ~ o / 1e-3 and the scale is visible."""
    g = _Gdn(1, 1, 8, 1, 18)
    g.b[:] = -1e4
    g.a[:] = -1e4
    S0 = (g.S0 * 1e-4).astype(np.float32)
    _, out = g.run(orc, S0=S0)
    q = g.q(0, 0)
    qn = q / np.sqrt((q ** 2).sum() + 1e-6) / np.sqrt(g.d)
    o = S0[0].astype(np.float64).T @ qn
    gate = _silu(g.z[0].astype(np.float64))
    want = o / np.sqrt((o ** 2).mean() + 1e-6) * _bff(g.norm) * gate
    assert (o ** 2).mean() < 1e-8
    assert _ulps16(out[0], want).max() <= 2.0
