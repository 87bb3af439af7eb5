"""Chunked prefill and the generate loop against the reference's own
serial loops (cli/main.cpp:1055-1069 prefill, 1072-1110 generation), run through the
same session API on the same synthetic model."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu
SEED = 91
CONTEXT = 256


@pytest.fixture(scope="module")
def model(device):
    from gfxinfer_amd.runtime import SyntheticModel, tiny_spec
    say("synthetic model for prefill/generate")
    m = SyntheticModel(tiny_spec(full_attention_interval=2, gdn_key_head_count=4), SEED)
    yield m
    m.close()


def _session(model, graph_batch=0):
    from gfxinfer_amd.runtime import QwenDecodeSession
    return QwenDecodeSession(model, CONTEXT, graph_batch)


def _prompt(n, seed):
    return np.random.default_rng(seed).integers(0, 1000, n).astype(np.uint32)


def serial_prefill(s, prompt, mtp=True):
    """cli/main.cpp:1055-1069 (a fresh session's first token has no MTP entry; on an
    aligned session every token's entry is added before its target step)."""
    fresh = s.position() == 0
    nxt = None
    for i, t in enumerate(prompt):
        if mtp and not (fresh and i == 0):
            s.mtp_draft(int(t))
        nxt = s.greedy_step(int(t))
    return nxt


def reference_generate(s, prompt, maximum, depth, stops=()):
    """cli/main.cpp:1055-1110 without the tokenizer."""
    nxt = serial_prefill(s, prompt, depth != 0)
    out = [nxt]
    rounds = proposed = accepted = emitted = 0
    while len(out) < maximum and nxt not in stops:
        if depth == 0 or maximum - len(out) == 1:
            nxt = s.greedy_step(nxt)
            out.append(nxt)
            continue
        r = s.speculative_step(nxt, min(depth, maximum - len(out) - 1))
        rounds += 1
        proposed += r.proposed_drafts
        accepted += r.accepted_drafts
        terminal = False
        for t in r.tokens:
            if len(out) == maximum:
                break
            out.append(t)
            emitted += 1
            nxt = t
            if t in stops:
                terminal = True
                break
        if terminal:
            break
    return out, dict(speculative_rounds=rounds, proposed_drafts=proposed, accepted_drafts=accepted,
                     speculative_emitted=emitted)


STATE = (("conv_states", np.float16), ("gdn_states", np.float32), ("key_caches", np.float16),
         ("value_caches", np.float16), ("mtp_key_cache", np.float16), ("mtp_value_cache", np.float16))


def _written(session, name, dtype):
    """A state buffer, or the written positions of a K/V cache ([layers][ctx][row])."""
    data = session.buffer(name, dtype)
    if "cache" not in name:
        return data
    positions = session.mtp_position() if name.startswith("mtp") else session.position()
    spec = session.model.spec
    row = spec.kv_head_count * spec.attention_head_size
    return data.reshape(-1, CONTEXT, row)[:, :positions]


def _same_state(a, b, names=STATE):
    """Positions and every state bit for bit (the GEMMs sum K in one canonical order at
    every batch, so a block of tokens equals one-token steps exactly)."""
    assert (a.position(), a.mtp_position()) == (b.position(), b.mtp_position())
    for name, dtype in names:
        assert np.array_equal(_written(a, name, dtype), _written(b, name, dtype)), name


@pytest.mark.parametrize("n", [1, 2, 32, 45, 70])
def test_prefill_leaves_the_serial_loop_state(model, n):
    prompt = _prompt(n, n)
    a, b = _session(model), _session(model)
    say("serial prefill", n)
    want = serial_prefill(a, prompt)
    say("chunked prefill", n)
    got = b.prefill(prompt)
    assert got == want
    _same_state(a, b)
    if n > 1:  # the next rounds see the same target and MTP state
        for _ in range(2):
            ra, rb = a.speculative_step(got, 4), b.speculative_step(got, 4)
            assert (ra.tokens, ra.accepted_drafts) == (rb.tokens, rb.accepted_drafts)
            got = rb.tokens[-1]
        _same_state(a, b)
    a.close()
    b.close()


def test_prefill_after_rounds_and_without_mtp(model):
    a, b = _session(model), _session(model)
    p1, p2 = _prompt(9, 1), _prompt(40, 2)
    say("prefill, rounds, prefill")
    x = serial_prefill(a, p1)
    y = b.prefill(p1)
    assert x == y
    for _ in range(2):
        ra, rb = a.speculative_step(x, 3), b.speculative_step(y, 3)
        assert ra.tokens == rb.tokens
        x, y = ra.tokens[-1], rb.tokens[-1]
    # a second prompt segment on an aligned, non-fresh session
    assert serial_prefill(a, np.concatenate([[x], p2])) == b.prefill(np.concatenate([[y], p2]))
    _same_state(a, b)
    a.close()
    b.close()
    # without the MTP update only the target advances
    c, d = _session(model), _session(model)
    assert serial_prefill(c, p2, mtp=False) == d.prefill(p2, sync_mtp=False)
    assert d.position() == len(p2) and d.mtp_position() == 0
    _same_state(c, d, STATE[:4])
    c.close()
    d.close()


@pytest.mark.parametrize("depth,maximum,graph", [(0, 12, 0), (4, 20, 0), (3, 17, 4), (31, 40, 0)])
def test_generate_matches_reference_loop(model, depth, maximum, graph):
    prompt = _prompt(23, depth + maximum)
    a, b = _session(model, graph), _session(model, graph)
    say("reference generate", depth, maximum, graph)
    want, want_stats = reference_generate(a, prompt, maximum, depth)
    say("library generate", depth, maximum, graph)
    got, stats = b.generate(prompt, maximum, depth)
    assert got == want
    assert stats["prompt_tokens"] == len(prompt) and stats["output_tokens"] == len(want)
    for k, v in want_stats.items():
        assert stats[k] == v, k
    assert stats["prefill_ms"] > 0 and stats["decode_ms"] >= 0
    a.close()
    b.close()


def test_generate_adaptive_depth_emits_the_greedy_sequence(model):
    """Speculative decoding is exact: any depth schedule emits the target's greedy
    continuation."""
    prompt = _prompt(30, 7)
    a, b = _session(model), _session(model)
    say("greedy generate")
    greedy, _ = a.generate(prompt, 60, 0)
    say("adaptive generate")
    adaptive, stats = b.generate(prompt, 60, 8, adaptive_depth=True)
    assert adaptive == greedy
    assert stats["speculative_rounds"] > 0
    a.close()
    b.close()


def test_generate_stops_at_a_stop_token_and_checks_the_context(model):
    from gfxinfer_amd import GfxinferError
    prompt = _prompt(12, 5)
    a = _session(model)
    full, _ = a.generate(prompt, 24, 3)
    a.close()
    stop = full[6]
    k = full.index(stop)
    b = _session(model)
    got, stats = b.generate(prompt, 24, 3, stop_tokens=[stop, 10 ** 6])
    assert got == full[:k + 1]
    b.close()
    c = _session(model)
    with pytest.raises(GfxinferError):
        c.generate(prompt, CONTEXT, 3)  # prompt + output beyond the context
    c.close()
