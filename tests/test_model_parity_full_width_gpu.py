"""Verify-step parity at the 27B widths against the model-level CPU oracle.

A reduced-depth model keeps every width of the 27B shape (hidden 5120, MLP 17408 in W3
then W4) with four layers (GDN, attention, GDN, attention) and an 8192-row W4 LM head,
at two head shapes: the BASELINE configs' (40 query / 8 KV heads x 128, GDN 16 key / 32
value heads x 128) and the reference's own model's (qwen38_spec.h:22-29: 24 / 4 x 256,
GDN 16 / 48, where the GDN window runs 32 state columns per workgroup).  So the composed
pass meets the oracle on the paths the small model never reaches: K = 5120 and 17408
cut into several canonical ranges, split-K planes summed by the residual norm, the
9-32-row direct GEMM, attention of either head size over a context.

The comparison is teacher-forced stage by stage: the session records every layer's
stage boundaries (gfxinfer_session_set_layer_trace) -- the rows entering the layer, the
A4 input of the o / out projection, the rows after the mixer's residual add, the A4
SwiGLU output, the rows leaving the layer -- and the oracle runs each stage from the
session's own inputs and pre-block state.  A free-running comparison of whole passes is
not meaningful at these widths: with A4 activations an ulp-level difference anywhere
(an expf, a reduction order) can move one activation across a rounding boundary, which
changes a projection by a whole quantization step, and over a few layers such steps
grow into O(1) logit differences -- between two correct implementations as much as
between a correct and a wrong one.  Per stage the bars are:

- stages of integer codes, GEMMs, norms and residual adds (the projections with their
  residual add, the logits): bit for bit against the oracle in the library's canonical
  K order (the one intended departure from the reference's arithmetic, pinned on its
  own by tests/test_oracle.py), and within 1e-3 of the largest value (logits: 2e-2
  absolute) against the oracle in the reference's own GEMM epilogue order;
- stages that end in an A4 quantizer after transcendental functions (the GDN or
  attention mixer, SwiGLU): the session's codes equal the oracle's except for at most
  1 % of them, each of which dequantizes within one quantization step;
- greedy tokens equal wherever the oracle's top-2 margin exceeds 4e-2;
- a planted speculative round (drafts = the session's own serial stream, the fourth
  one wrong) accepts exactly 3, and the rolled-back GDN state equals the oracle's replay
  (orc_gdn_restore_*) of the session's logs within fp32 1e-5.
"""
import numpy as np
import pytest

from gpu_util import empty, host, say

pytestmark = pytest.mark.gpu

SEED = 5120
CTX = 128
DEEP_CTX = 4096  # the BASELINE model's context
LOGIT_TOL = 2e-2
MARGIN = 2 * LOGIT_TOL


HEADS = {
    "baseline": dict(attention_head_count=40, kv_head_count=8, attention_head_size=128, gdn_value_head_count=32),
    "reference": dict(attention_head_count=24, kv_head_count=4, attention_head_size=256, gdn_value_head_count=48),
}


def _spec(heads):
    from gfxinfer_amd.runtime import tiny_spec
    return tiny_spec(hidden_size=5120, intermediate_size=17408, layer_count=4, full_attention_interval=2,
                     rotary_size=64, gdn_key_head_count=16, vocabulary_size=8192,
                     tokenizer_vocabulary_size=8000, mtp_draft_vocabulary=4096, w3_mlp_layers=2, **HEADS[heads])


@pytest.fixture(scope="module", params=sorted(HEADS))
def models(request, device, gx):
    from gfxinfer_amd.runtime import SyntheticModel
    from oracle.model import OracleModel
    spec = _spec(request.param)
    say("full-width 4-layer model on the GPU,", request.param, "heads")
    gpu = SyntheticModel(spec, SEED)
    say("full-width oracle models (reference and library K order)")
    reference = OracleModel(spec.as_dict(), SEED)
    library = OracleModel(spec.as_dict(), SEED,
                          k_order=lambda rows, cols: int(gx.lib().gfxinfer_gemm_split_count(rows, cols, 1)))
    yield spec, gpu, reference, library
    gpu.close()


def _prompt(spec, seed, n):
    return [int(t) for t in np.random.default_rng(seed).integers(0, spec.tokenizer_vocabulary_size, n)]


def _margins(logits, vocab):
    top2 = np.sort(logits[:, :vocab], axis=1)[:, -2:]
    return top2[:, 1] - top2[:, 0]


class Traced:
    """A session with its layer trace buffer, parsed into the trace's sections."""

    def __init__(self, gpu, spec, keep_logits=True, ctx=CTX):
        from gfxinfer_amd.runtime import QwenDecodeSession
        self.spec = spec
        self.session = QwenDecodeSession(gpu, ctx, 0, keep_logits=keep_logits)
        self.trace = empty((self.session.layer_trace_bytes(),), np.uint8)
        self.session.set_layer_trace(self.trace.data_ptr(), self.trace.numel())

    def sections(self, count):
        """residual [layers + 1][T][H], post [layers][T][H] (fp16 bits), and per layer the
        mixer and MLP (codes [T][w / 2], scales [T][w / 128])."""
        sp = self.spec
        L, B, H, I = sp.layer_count, 32, sp.hidden_size, sp.intermediate_size
        attn = sp.attention_head_count * sp.attention_head_size
        gdn = sp.gdn_value_head_count * sp.gdn_head_size
        W = max(attn, gdn)
        raw = host(self.trace)
        at = 0

        def take(n):
            nonlocal at
            piece = raw[at:at + n]
            at += n
            return piece
        residual = take((L + 1) * B * H * 2).view(np.uint16).reshape(L + 1, B, H)[:, :count].copy()
        post = take(L * B * H * 2).view(np.uint16).reshape(L, B, H)[:, :count].copy()
        mixer_codes = take(L * B * W // 2).reshape(L, -1)
        mixer_scales = take(L * B * (W // 128) * 2).view(np.uint16).reshape(L, -1)
        mlp_codes = take(L * B * I // 2).reshape(L, -1)
        mlp_scales = take(L * B * (I // 128) * 2).view(np.uint16).reshape(L, -1)
        mixer, mlp = [], []
        for i in range(L):
            w = attn if (i + 1) % sp.full_attention_interval == 0 else gdn
            mixer.append((mixer_codes[i, :count * w // 2].reshape(count, w // 2).copy(),
                          mixer_scales[i, :count * w // 128].reshape(count, w // 128).copy()))
            mlp.append((mlp_codes[i, :count * I // 2].reshape(count, I // 2).copy(),
                        mlp_scales[i, :count * I // 128].reshape(count, I // 128).copy()))
        return residual, post, mixer, mlp

    def close(self):
        self.session.close()


def _load_states(oracle, session, spec):
    """The oracle session takes the GPU session's recurrent states and K/V caches."""
    hv, d = spec.gdn_value_head_count, spec.gdn_head_size
    gdn = session.buffer("gdn_states", np.float32).reshape(len(oracle.state), hv, d, d)
    conv = session.buffer("conv_states", np.uint16).reshape(len(oracle.conv), -1, 4)
    keys = session.buffer("key_caches", np.uint16).reshape(len(oracle.kcache), oracle.capacity, -1)
    values = session.buffer("value_caches", np.uint16).reshape(len(oracle.vcache), oracle.capacity, -1)
    oracle.state = [gdn[i].copy() for i in range(len(oracle.state))]
    oracle.conv = [conv[i].copy() for i in range(len(oracle.conv))]
    oracle.kcache = [keys[i].copy() for i in range(len(oracle.kcache))]
    oracle.vcache = [values[i].copy() for i in range(len(oracle.vcache))]


def _codes_agree(got, want, label):
    """A4 codes and scales of one stage: at most 1 % of the codes differ, each within one
    quantization step once dequantized."""
    from oracle import oracle as O
    (gc, gs), (wc, ws) = got, want
    K = gc.shape[1] * 2
    gi, wi = O.unpack_a4(gc, K).astype(np.float64), O.unpack_a4(wc, K).astype(np.float64)
    gsc = np.repeat(gs.view(np.float16).astype(np.float64), 128, axis=1)
    wsc = np.repeat(ws.view(np.float16).astype(np.float64), 128, axis=1)
    differ = float(np.mean((gi != wi) | (gsc != wsc)))
    step = np.abs(gi * gsc - wi * wsc) / np.maximum(gsc, wsc)
    say(label, f"codes differing {differ:.2e}, largest step {step.max():.3f}")
    assert differ <= 0.01 and step.max() <= 1.0 + 1e-3, (label, differ, float(step.max()))


def _rows_agree(got, want, exact, label):
    g = got.view(np.float16).astype(np.float64)
    w = want.view(np.float16).astype(np.float64)
    err = float(np.abs(g - w).max() / np.abs(w).max())
    if exact:
        assert np.array_equal(got, want), (label, err)
    else:
        assert err <= 1e-3, (label, err)


def _teacher_forced(oracle, traced, count, position, exact, label):
    """Every stage of every layer from the session's own stage inputs."""
    residual, post, mixer, mlp = traced.sections(count)
    for i in range(len(oracle.m.layers)):
        _codes_agree(mixer[i], oracle.mixer_stage(i, residual[i], position), f"{label} layer {i} mixer")
        _rows_agree(post[i], oracle.post_stage(i, residual[i], *mixer[i]), exact, f"{label} layer {i} post")
        _codes_agree(mlp[i], oracle.mlp_codes_stage(i, post[i]), f"{label} layer {i} SwiGLU")
        _rows_agree(residual[i + 1], oracle.out_stage(i, post[i], *mlp[i]), exact, f"{label} layer {i} out")
    return residual[-1]


def _check_block(traced, oracles, block, position):
    spec = traced.spec
    V, Vt = spec.vocabulary_size, spec.tokenizer_vocabulary_size
    for oracle in oracles:
        _load_states(oracle, traced.session, spec)
    say("full-width block", len(block), "at", position)
    got = traced.session.block_step(block)
    logits = traced.session.buffer("logits", np.float32, len(block) * V).reshape(len(block), V)
    for oracle, label in zip(oracles, ("library order", "reference order")):
        last = _teacher_forced(oracle, traced, len(block), position, label == "library order", label)
        want_logits = oracle.final_logits(last)
        err = float(np.abs(logits - want_logits).max())
        say(label, "logit error", err)
        if label == "library order":
            assert np.array_equal(logits, want_logits)
        else:
            assert err <= LOGIT_TOL, err
        sure = _margins(want_logits, Vt) > MARGIN
        assert sure.sum() >= len(block) // 2
        want_tokens = np.argmax(want_logits[:, :Vt], axis=1)
        assert np.array_equal(np.asarray(got)[sure], want_tokens[sure])
    assert float(np.abs(logits).max()) > 1.0  # non-trivial logits
    return got


def test_full_width_verify_blocks_match_oracle(models):
    """A 5-token block from an empty context, then a 32-token block over it, layer by
    layer against the oracle; the GDN states the 32-token block leaves are within fp32
    1e-5 of the teacher-forced library-order oracle's (the recurrences sum in different
    orders, so the states, unlike the fp16 rows, differ in the last bits)."""
    from oracle.model import OracleSession
    spec, gpu, reference, library = models
    traced = Traced(gpu, spec)
    oracles = [OracleSession(library, CTX), OracleSession(reference, CTX)]
    try:
        _check_block(traced, oracles, _prompt(spec, SEED, 5), 0)
        _check_block(traced, oracles, _prompt(spec, SEED + 1, 32), 5)
        got = traced.session.buffer("gdn_states", np.float32).reshape(len(oracles[0].state),
                                                                      *oracles[0].state[0].shape)
        want = np.stack(oracles[0].state)
        assert np.abs(got - want).max() <= 1e-5 * max(1.0, float(np.abs(want).max()))
    finally:
        traced.close()


def test_full_width_block_deep_in_context(models):
    """A 32-token block at position 4000 of a 4096-position context, after a chunked
    prefill of 4000 tokens, layer by layer against the oracle run from the session's own
    caches and states: attention over 4032 positions inside the composed pass (the split
    kernels with their positions spread over many splits, the combine over all of them)."""
    from oracle.model import OracleSession
    spec, gpu, reference, library = models
    traced = Traced(gpu, spec, ctx=DEEP_CTX)
    oracles = [OracleSession(library, DEEP_CTX), OracleSession(reference, DEEP_CTX)]
    try:
        say("full-width prefill of 4000 tokens")
        traced.session.prefill(_prompt(spec, SEED + 2, 4000))
        assert traced.session.position() == 4000
        _check_block(traced, oracles, _prompt(spec, SEED + 3, 32), 4000)
    finally:
        traced.close()


def test_full_width_planted_round_and_rollback(models):
    """speculative == serial (cli/main.cpp:970-979) at full width: the session's own
    greedy stream after a 5-token prompt is planted as drafts with the fourth one wrong,
    so the verifier accepts exactly 3 (qwen_runtime.cpp:1497-1501); the verify block of
    the round matches the oracle layer by layer; the GDN states left by the partial
    acceptance equal the oracle replay (orc_gdn_restore_*) of seed + 3 accepted tokens
    from the session's own logs onto the pre-round states."""
    from gfxinfer_amd.runtime import QwenDecodeSession
    from oracle import oracle as O
    from oracle.model import OracleSession
    spec, gpu, _, library = models
    Vt = spec.tokenizer_vocabulary_size
    prompt = _prompt(spec, 2, 5)
    serial = QwenDecodeSession(gpu, CTX, 0)
    try:
        say("full-width serial stream")
        seed = serial.prefill(prompt)
        stream = [serial.greedy_step(seed)]
        while len(stream) < 4:
            stream.append(serial.greedy_step(stream[-1]))
    finally:
        serial.close()
    drafts = list(stream)
    drafts[3] = (drafts[3] + 1) % Vt
    traced = Traced(gpu, spec, keep_logits=False)
    session = traced.session
    oracle = OracleSession(library, CTX)
    try:
        say("full-width prefill + planted round")
        assert session.prefill(prompt) == seed
        pre_states = session.buffer("gdn_states", np.float32)
        pre_conv = session.buffer("conv_states", np.uint16)
        _load_states(oracle, session, spec)
        r = session.speculative_step_planted(seed, drafts)
        assert r.accepted_drafts == 3 and r.tokens == stream[:4], (r.accepted_drafts, r.tokens, stream)
        assert session.position() == len(prompt) + 4
        _teacher_forced(oracle, traced, len(drafts) + 1, len(prompt), True, "planted verify block")
        post_s = session.buffer("gdn_states", np.float32)
        post_c = session.buffer("conv_states", np.uint16)
        B = 32  # the session's log depth (one verifier block)
        hk, hv, d = spec.gdn_key_head_count, spec.gdn_value_head_count, spec.gdn_head_size
        channels = 2 * hk * d + hv * d
        layers = 2
        key_log = session.buffer("key_log", np.float32).reshape(layers, B, hk * d)
        delta_log = session.buffer("delta_log", np.float32).reshape(layers, B, hv * d)
        decay_log = session.buffer("decay_log", np.float32).reshape(layers, B, hv)
        conv_log = session.buffer("conv_log", np.uint16).reshape(layers, B, channels)
    finally:
        traced.close()
    states = pre_states.reshape(layers, hv, d, d)
    convs = pre_conv.reshape(layers, channels, 4)
    got_s = post_s.reshape(layers, hv, d, d)
    got_c = post_c.reshape(layers, channels, 4)
    for layer in range(layers):
        want = np.ascontiguousarray(states[layer]).copy()
        keys = np.ascontiguousarray(key_log[layer])
        deltas = np.ascontiguousarray(delta_log[layer])
        decays = np.ascontiguousarray(decay_log[layer])
        O.lib().orc_gdn_restore_recurrent(O.ptr(want), O.ptr(keys), O.ptr(deltas), O.ptr(decays), 4, hk, hv, d)
        scale = max(1.0, float(np.abs(want).max()))
        assert np.abs(got_s[layer] - want).max() <= 1e-5 * scale
        wc = np.ascontiguousarray(convs[layer]).copy()
        clog = np.ascontiguousarray(conv_log[layer])
        O.lib().orc_gdn_restore_conv(O.ptr(wc), O.ptr(clog), channels, 4)
        assert np.array_equal(got_c[layer], wc)
