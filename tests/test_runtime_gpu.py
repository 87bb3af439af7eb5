"""GPU tests of the decode runtime (include/gfxinfer_runtime.h) on seeded synthetic
checkpoints: the generator against its CPU restatement, and the reference's own
self-consistency invariants of QwenDecodeSession -- block == serial
(src/cli/main.cpp:880-887), speculative == serial (:970-979) -- plus graph == eager,
planted-draft acceptance lengths and rollback == prefix-run state."""
import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

SEED = 1234


def _spec():
    from gfxinfer_amd.runtime import tiny_spec
    return tiny_spec(full_attention_interval=2, gdn_key_head_count=4)


@pytest.fixture(scope="module")
def tiny(device):
    from gfxinfer_amd.runtime import SyntheticModel
    say("create tiny synthetic model")
    model = SyntheticModel(_spec(), SEED)
    yield model
    model.close()


def _session(model, graph=0, ctx=256):
    from gfxinfer_amd.runtime import QwenDecodeSession
    return QwenDecodeSession(model, ctx, graph)


def _law(name: str):
    """(mean, sigma) of a tensor, as gfxinfer_model_create_synthetic documents."""
    if name.endswith("conv1d.weight") or name.endswith("A_log") or name.endswith("dt_bias"):
        return 0.0, 0.5
    if name.endswith("linear_attn.norm.weight"):
        return 1.0, 0.02
    return 0.0, 0.02


@pytest.mark.parametrize("name", [
    "model.language_model.embed_tokens.weight",
    "lm_head.weight",
    "model.language_model.layers.0.mlp.gate_proj.weight",      # W3
    "model.language_model.layers.3.mlp.down_proj.weight",      # W4 tail
    "model.language_model.layers.0.linear_attn.in_proj_qkv.weight",
    "model.language_model.layers.0.linear_attn.in_proj_a.weight",
    "model.language_model.layers.1.self_attn.q_proj.weight",
    "mtp.fc.weight",
    "model.language_model.layers.0.linear_attn.conv1d.weight",
    "model.language_model.layers.0.linear_attn.A_log",
    "model.language_model.layers.2.linear_attn.norm.weight",
    "model.language_model.layers.1.self_attn.q_norm.weight",
])
def test_synthetic_weights_match_cpu_generator(tiny, gx, orc, name):
    view = tiny.find_tensor(name)
    rows, cols = int(view.rows), int(view.columns)
    mean, sigma = _law(name)
    values = orc.synthetic_values(SEED, name, rows * cols, sigma, mean).reshape(rows, cols)
    if view.format == 0:
        assert np.array_equal(tiny.tensor_bytes(name).view(np.uint16).reshape(rows, cols),
                              orc.f32_to_bf16_bits(values))
        return
    status, codes, scales = orc.quantize_group128(values, view.format)
    assert status == 0
    tcodes, tscales = gx.tile_group128(view.format, codes, scales, rows, cols)
    assert np.array_equal(tiny.tensor_bytes(name), tcodes)
    assert np.array_equal(tiny.tensor_bytes(name, auxiliary=True).view(np.uint16), tscales)


@pytest.mark.parametrize("count", [5, 9, 17, 32])
def test_block_step_equals_serial(tiny, count):
    """cli/main.cpp:880-887: a block of tokens gives the tokens and the state that
    one-token steps give, bit for bit, at every block size."""
    tokens = [int(t) for t in np.random.default_rng(count).integers(0, 1000, count)]
    serial = _session(tiny)
    say("serial greedy steps", count)
    outs = [serial.greedy_step(t) for t in tokens]
    block = _session(tiny)
    say("block step", count)
    assert block.block_step(tokens) == outs
    assert block.position() == serial.position() == len(tokens)
    for name in ("gdn_states", "conv_states", "hidden"):
        a, b = serial.buffer(name), block.buffer(name)
        if name == "hidden":  # the last token's row
            row = a.size // 32
            a, b = a[:row], b[(count - 1) * row:count * row]
        assert np.array_equal(a, b), name
    for name in ("key_caches", "value_caches"):  # the written positions
        assert np.array_equal(_kv_prefix(serial, name, count), _kv_prefix(block, name, count)), name


def _kv_prefix(session, name, positions, ctx=256):
    """Written positions [0, positions) of every layer of a K/V cache buffer."""
    spec = _spec()
    row = spec.kv_head_count * spec.attention_head_size
    cache = session.buffer(name, np.uint16)
    return cache.reshape(-1, ctx, row)[:, :positions]


def _serial_stream(model, first, n):
    s = _session(model)
    y = [s.greedy_step(first)]
    while len(y) < n:
        y.append(s.greedy_step(y[-1]))
    return y


@pytest.mark.parametrize("depth", [4, 7])
def test_planted_drafts_accept_the_serial_prefix(tiny, depth):
    """speculative == serial (cli/main.cpp:970-979) with drafts planted from the serial
    stream and cut at a seeded index, so the acceptance rule sees real matches."""
    rng = np.random.default_rng(depth)
    stream = _serial_stream(tiny, 11, 64)
    spec = _spec()
    session = _session(tiny)
    assert session.greedy_step(11) == stream[0]
    emitted = [stream[0]]
    cuts = [depth, 0, int(rng.integers(0, depth)), depth, int(rng.integers(0, depth)), 1]
    for cut in cuts:
        k = len(emitted)  # stream[k - 1] is the seed
        drafts = list(stream[k:k + depth])
        if cut < depth:
            drafts[cut] = (drafts[cut] + 1) % spec.tokenizer_vocabulary_size
        say("planted depth", depth, "cut", cut)
        r = session.speculative_step_planted(emitted[-1], drafts)
        assert r.accepted_drafts == cut and r.proposed_drafts == depth
        assert r.tokens == stream[k:k + cut + 1]
        emitted += r.tokens
        assert session.position() == len(emitted)
        assert session.mtp_position() + 1 == session.position()


@pytest.mark.parametrize("depth", [4, 7])
def test_graph_equals_eager_under_forced_acceptance(tiny, depth):
    rng = np.random.default_rng(100 + depth)
    graph = _session(tiny, graph=depth + 1)
    eager = _session(tiny)
    seed_a, seed_b = graph.greedy_step(7), eager.greedy_step(7)
    assert seed_a == seed_b
    for _ in range(6):
        accepted = int(min(np.argmax(rng.random(depth + 1) > 0.85), depth))
        say("forced depth", depth, "accepted", accepted)
        ra = graph.speculative_step_forced(seed_a, depth, accepted)
        rb = eager.speculative_step_forced(seed_b, depth, accepted)
        assert ra == rb and ra.accepted_drafts == accepted
        seed_a, seed_b = ra.tokens[-1], rb.tokens[-1]
    assert graph.position() == eager.position()
    assert graph.mtp_position() == eager.mtp_position()
    for name in ("gdn_states", "conv_states"):
        assert np.array_equal(graph.buffer(name), eager.buffer(name)), name
    for name in ("key_caches", "value_caches"):
        p = graph.position()
        assert np.array_equal(_kv_prefix(graph, name, p), _kv_prefix(eager, name, p)), name
    for name in ("mtp_key_cache", "mtp_value_cache"):
        p = graph.mtp_position()
        assert np.array_equal(_kv_prefix(graph, name, p), _kv_prefix(eager, name, p)), name


@pytest.mark.parametrize("cut", [4, 5, 6])
def test_rollback_state_equals_prefix_block(tiny, cut):
    """restore(accepted + 1) after a depth-7 window == a block over just those tokens
    (same kernel configuration for 5..8 tokens, so bit-identical)."""
    depth = 7
    stream = _serial_stream(tiny, 23, depth + 2)
    spec = _spec()
    drafts = list(stream[1:1 + depth])
    drafts[cut] = (drafts[cut] + 1) % spec.tokenizer_vocabulary_size
    a = _session(tiny)
    a.greedy_step(23)
    say("rollback cut", cut)
    r = a.speculative_step_planted(stream[0], drafts)
    assert r.accepted_drafts == cut
    b = _session(tiny)
    b.greedy_step(23)
    b.block_step([stream[0]] + drafts[:cut])
    assert a.position() == b.position()
    for name in ("gdn_states", "conv_states"):
        assert np.array_equal(a.buffer(name), b.buffer(name)), name
    for name in ("key_caches", "value_caches"):
        p = a.position()
        assert np.array_equal(_kv_prefix(a, name, p), _kv_prefix(b, name, p)), name


def test_session_rejects_misaligned_steps(tiny, gx):
    s = _session(tiny)
    with pytest.raises(gx.GfxinferError):
        s.speculative_step(1, 4)      # no target state yet
    s.greedy_step(1)
    with pytest.raises(gx.GfxinferError):
        s.speculative_step(1, 32)     # depth > 31
    with pytest.raises(gx.GfxinferError):
        s.block_step([])
    with pytest.raises(gx.GfxinferError):
        s.speculative_step_forced(1, 4, 5)


def test_session_outlives_its_model(device):
    """Destroying a model while a session on it is open defers the release to the end of
    the last session: the session keeps stepping on the model's stream and weights, and
    closing it frees both (a session destroyed after its model once synchronized a
    destroyed stream)."""
    from gfxinfer_amd.runtime import QwenDecodeSession, SyntheticModel
    model = SyntheticModel(_spec(), SEED)
    reference = _session(model)
    want = [reference.greedy_step(t) for t in (5, 6, 7)]
    reference.close()
    session = QwenDecodeSession(model, 256, 0)
    say("destroy the model under an open session")
    model.close()
    assert [session.greedy_step(t) for t in (5, 6, 7)] == want
    session.close()


def test_full_size_model_speculative_rounds(device):
    """The 27B-shaped synthetic model: generation, a graph session at depth 4 and 31,
    forced 85 % acceptance rounds and block == serial on the first tokens."""
    import time
    from gfxinfer_amd.runtime import QwenDecodeSession, SyntheticModel, qwen38_27b_spec
    say("create 27B-shaped model")
    t0 = time.time()
    model = SyntheticModel(qwen38_27b_spec(), 2026)
    say("generated", model.weight_bytes, "bytes in", round(time.time() - t0, 2), "s")
    try:
        serial = QwenDecodeSession(model, 4096, 0)
        outs = [serial.greedy_step(t) for t in (1, 2, 3)]
        block = QwenDecodeSession(model, 4096, 0)
        assert block.block_step([1, 2, 3]) == outs
        serial.close()
        block.close()
        rng = np.random.default_rng(5)
        for depth in (4, 31):
            s = QwenDecodeSession(model, 4096, depth + 1)
            seed = s.greedy_step(9)
            for _ in range(3):
                accepted = int(min(np.argmax(rng.random(depth + 1) > 0.85), depth))
                say("27B depth", depth, "accepted", accepted)
                r = s.speculative_step_forced(seed, depth, accepted)
                assert r.accepted_drafts == accepted and len(r.tokens) == accepted + 1
                assert all(0 <= t < 151936 for t in r.tokens)
                seed = r.tokens[-1]
            s.close()
    finally:
        model.close()
