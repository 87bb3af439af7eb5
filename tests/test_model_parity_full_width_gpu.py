"""Verify-step parity at the 27B widths against the model-level CPU oracle.

A reduced-depth model keeps every width of the 27B shape (hidden 5120, MLP 17408 in W3
then W4, 40 query / 8 KV heads x 128, GDN 16 key / 32 value heads x 128) with four
layers (GDN, attention, GDN, attention) and a 8192-row W4 LM head, so the composed pass
meets the oracle on the paths the small model never reaches: K = 5120 and 17408 cut
into several canonical ranges, split-K planes summed by the residual norm, the 9-32-row
direct GEMM, 40/8 x 128 attention over a context.

Bars: logits within 2e-2 absolute of oracle/model.py with the
reference's own GEMM epilogue order, greedy tokens equal wherever the oracle's top-2
margin exceeds 4e-2, the exact accepted length of a planted speculative round
(qwen_runtime.cpp:1497-1501), and the rolled-back GDN state within fp32 1e-5 of the
oracle's replay of the same logs (qwen_ops.hip:413-539).  The oracle is also run in
the library's canonical K order (the one intended difference from the reference),
where the logits must agree to the same bar.
"""
import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

SEED = 5120
LOGIT_TOL = 2e-2
MARGIN = 2 * LOGIT_TOL


def _spec():
    from gfxinfer_amd.runtime import tiny_spec
    return tiny_spec(hidden_size=5120, intermediate_size=17408, layer_count=4, full_attention_interval=2,
                     attention_head_count=40, kv_head_count=8, rotary_size=64, gdn_key_head_count=16,
                     gdn_value_head_count=32, vocabulary_size=8192, tokenizer_vocabulary_size=8000,
                     mtp_draft_vocabulary=4096, w3_mlp_layers=2)


@pytest.fixture(scope="module")
def models(device, gx):
    from gfxinfer_amd.runtime import SyntheticModel
    from oracle.model import OracleModel
    spec = _spec()
    say("full-width 4-layer model on the GPU")
    gpu = SyntheticModel(spec, SEED)
    say("full-width oracle models (reference and library K order)")
    reference = OracleModel(spec.as_dict(), SEED)
    library = OracleModel(spec.as_dict(), SEED,
                          k_order=lambda rows, cols: int(gx.lib().gfxinfer_gemm_split_count(rows, cols, 1)))
    yield gpu, reference, library
    gpu.close()


def _margins(logits, vocab):
    top2 = np.sort(logits[:, :vocab], axis=1)[:, -2:]
    return top2[:, 1] - top2[:, 0]


def _prompt(seed, n):
    return [int(t) for t in np.random.default_rng(seed).integers(0, _spec().tokenizer_vocabulary_size, n)]


def test_full_width_verify_blocks_match_oracle(models):
    """A 5-token block from an empty context, then a 32-token block over it."""
    from gfxinfer_amd.runtime import QwenDecodeSession
    from oracle.model import OracleSession
    gpu, reference, library = models
    spec = _spec()
    V, Vt = spec.vocabulary_size, spec.tokenizer_vocabulary_size
    session = QwenDecodeSession(gpu, 128, 0, keep_logits=True)
    oracles = [OracleSession(reference, 128), OracleSession(library, 128)]
    try:
        for block in (_prompt(SEED, 5), _prompt(SEED + 1, 32)):
            say("full-width block", len(block))
            got = session.block_step(block)
            logits = session.buffer("logits", np.float32, len(block) * V).reshape(len(block), V)
            errors = []
            for oracle in oracles:
                want, want_logits = oracle.block_step(block)
                errors.append(float(np.abs(logits - want_logits).max()))
                sure = _margins(want_logits, Vt) > MARGIN
                assert sure.sum() >= len(block) // 2
                assert np.array_equal(np.asarray(got)[sure], np.asarray(want)[sure])
            say("max logit error vs reference / library K order", errors)
            assert max(errors) <= LOGIT_TOL, errors
            assert float(np.abs(logits).max()) > 1.0  # non-trivial logits
        # the GDN states after both blocks: within the logits' own propagation bar
        lib_oracle = oracles[1]
        got_states = session.buffer("gdn_states", np.float32).reshape(len(lib_oracle.state),
                                                                      *lib_oracle.state[0].shape)
        np.testing.assert_allclose(got_states, np.stack(lib_oracle.state), rtol=5e-3, atol=5e-4)
    finally:
        session.close()


def test_full_width_planted_round_and_rollback(models):
    """speculative == serial (cli/main.cpp:970-979) at full width: the oracle's greedy
    stream after a 5-token prompt is planted as drafts with the fourth one wrong, so the
    verifier accepts exactly 3; the GDN states left by the partial acceptance equal the
    oracle replay (orc_gdn_restore_*) of seed + 3 accepted tokens from the session's own
    logs onto the pre-round states, and the oracle's states after the same tokens."""
    from gfxinfer_amd.runtime import QwenDecodeSession
    from oracle import oracle as O
    from oracle.model import OracleSession
    gpu, _, library = models
    spec = _spec()
    Vt = spec.tokenizer_vocabulary_size
    prompt = _prompt(2, 5)
    oracle = OracleSession(library, 128)
    tokens, logits = oracle.block_step(prompt)
    assert _margins(logits, Vt)[-1] > MARGIN
    seed = tokens[-1]
    stream = []
    t = seed
    for _ in range(4):  # the oracle's greedy continuation, one token at a time
        out, logits = oracle.block_step([t])
        assert _margins(logits, Vt)[0] > MARGIN
        stream.append(out[0])
        t = out[0]
    drafts = list(stream)
    drafts[3] = (drafts[3] + 1) % Vt
    session = QwenDecodeSession(gpu, 128, 0)
    try:
        say("full-width prefill + planted round")
        assert session.prefill(prompt) == seed
        names = ("gdn_states", "conv_states")
        pre = {n: session.buffer(n) for n in names}
        r = session.speculative_step_planted(seed, drafts)
        assert r.accepted_drafts == 3 and r.tokens == stream[:4], (r.accepted_drafts, r.tokens, stream)
        assert session.position() == len(prompt) + 4
        post_s = session.buffer("gdn_states", np.float32)
        post_c = session.buffer("conv_states", np.uint16)
        B = 32  # the session's log depth (one verifier block)
        hk, hv, d = spec.gdn_key_head_count, spec.gdn_value_head_count, spec.gdn_head_size
        channels = 2 * hk * d + hv * d
        layers = 2
        key_log = session.buffer("key_log", np.float32).reshape(layers, B, hk * d)
        delta_log = session.buffer("delta_log", np.float32).reshape(layers, B, hv * d)
        decay_log = session.buffer("decay_log", np.float32)[:layers * B * hv].reshape(layers, B, hv)
        conv_log = session.buffer("conv_log", np.uint16).reshape(layers, B, channels)
    finally:
        session.close()
    states = pre["gdn_states"].view(np.float32).reshape(layers, hv, d, d).copy()
    convs = pre["conv_states"].view(np.uint16).reshape(layers, channels, 4).copy()
    got_s = post_s.reshape(layers, hv, d, d)
    got_c = post_c.reshape(layers, channels, 4)
    for layer in range(layers):
        want = np.ascontiguousarray(states[layer])
        O.lib().orc_gdn_restore_recurrent(O.ptr(want), O.ptr(np.ascontiguousarray(key_log[layer])),
                                          O.ptr(np.ascontiguousarray(delta_log[layer])),
                                          O.ptr(np.ascontiguousarray(decay_log[layer])), 4, hk, hv, d)
        scale = max(1.0, float(np.abs(want).max()))
        assert np.abs(got_s[layer] - want).max() <= 1e-5 * scale
        wc = np.ascontiguousarray(convs[layer])
        O.lib().orc_gdn_restore_conv(O.ptr(wc), O.ptr(np.ascontiguousarray(conv_log[layer])), channels, 4)
        assert np.array_equal(got_c[layer], wc)
    # the oracle that ran prompt + seed + 3 accepted tokens holds the same states
    np.testing.assert_allclose(got_s, np.stack(oracle.state), rtol=5e-3, atol=5e-4)
