"""End-to-end parity of the GPU decode session against the model-level CPU oracle
(oracle/model.py) on small synthetic models of the same structure: logits of
block steps (fresh state, then with K/V caches and GDN state carried over) and of an
MTP proposal within the BASELINE logit tolerance 2e-2 absolute, greedy tokens equal
wherever the oracle's top-1/top-2 margin exceeds twice that tolerance.  Two head
shapes: 128-dim attention heads with GDN ratio 4 (the BASELINE model's kind), and the
reference model's own 256-dim heads, six query heads per KV head, rotary 64 and GDN
16 key / 48 value heads (qwen38_spec.h:22-29)."""
import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

SEED = 4321
LOGIT_TOL = 2e-2


def _spec(shape="baseline"):
    from gfxinfer_amd.runtime import reference_tiny_spec, tiny_spec
    if shape == "reference":
        return reference_tiny_spec()
    return tiny_spec(full_attention_interval=2, gdn_key_head_count=4)


@pytest.fixture(scope="module", params=["baseline", "reference"])
def pair(device, request):
    from gfxinfer_amd.runtime import SyntheticModel
    from oracle.model import OracleModel
    spec = _spec(request.param)
    say("tiny model for oracle parity", request.param)
    gpu = SyntheticModel(spec, SEED)
    cpu = OracleModel(spec.as_dict(), SEED)
    yield gpu, cpu, spec
    gpu.close()


def _check_tokens(got, logits, some_sure=True):
    """Tokens equal the oracle's argmax wherever its top-2 margin exceeds twice the logit
    bar; some_sure: at least one such row (a block), not required of a single row."""
    top2 = np.sort(logits, axis=1)[:, -2:]
    margin = top2[:, 1] - top2[:, 0]
    want = np.argmax(logits, axis=1)
    sure = margin > 2 * LOGIT_TOL
    assert sure.any() or not some_sure
    assert np.array_equal(np.asarray(got)[sure], want[sure])


def test_block_steps_match_oracle(pair):
    from gfxinfer_amd.runtime import QwenDecodeSession
    from oracle.model import OracleSession
    gpu, cpu, spec = pair
    V, Vt = spec.vocabulary_size, spec.tokenizer_vocabulary_size
    s = QwenDecodeSession(gpu, 64, 0, keep_logits=True)
    o = OracleSession(cpu, 64)
    for block in ([3, 141, 59, 26, 535], [897, 9, 32], [384]):
        say("block", block)
        got = s.block_step(block)
        want, want_logits = o.block_step(block)
        logits = s.buffer("logits", np.float32, len(block) * V).reshape(len(block), V)
        err = np.abs(logits - want_logits).max()
        assert err <= LOGIT_TOL, err
        _check_tokens(got, want_logits[:, :Vt])
    gdn = s.buffer("gdn_states", np.float32).reshape(len(o.state), *o.state[0].shape)
    np.testing.assert_allclose(gdn, np.stack(o.state), rtol=5e-3, atol=5e-4)


def test_mtp_proposal_matches_oracle(pair):
    from gfxinfer_amd.runtime import QwenDecodeSession
    from oracle.model import OracleSession
    gpu, cpu, spec = pair
    s = QwenDecodeSession(gpu, 64, 0, keep_logits=True)
    o = OracleSession(cpu, 64)
    first = s.greedy_step(77)
    want_first, _ = o.block_step([77])
    assert first == want_first[0]
    say("mtp draft")
    draft = s.mtp_draft(first)
    want_draft, want_logits, _ = o.mtp_proposal(first, o.last_hidden, 0)
    logits = s.buffer("logits", np.float32, spec.mtp_draft_vocabulary)
    err = np.abs(logits - want_logits[0]).max()
    assert err <= LOGIT_TOL, err
    _check_tokens([draft], want_logits, some_sure=False)


def test_mtp_chain_drafts_match_oracle(pair):
    """The D drafts of a speculative round (each proposal after the first taking its token
    from the previous proposal's draft-head keys) equal the oracle's chain of MTP proposals
    (qwen_runtime.cpp:1448-1462: proposal i + 1 conditioned on proposal i's hidden row)
    wherever the oracle's top-2 margin is clear.  The oracle is teacher-forced on the
    session's own drafts (its hidden row does not depend on the pick), so a near tie at
    one step does not end the comparison."""
    from gfxinfer_amd.runtime import QwenDecodeSession
    from oracle.model import OracleSession
    gpu, cpu, spec = pair
    depth = 4
    s = QwenDecodeSession(gpu, 64, depth + 1)
    o = OracleSession(cpu, 64)
    first = s.greedy_step(77)
    want_first, _ = o.block_step([77])
    assert first == want_first[0]
    say("speculative round, depth", depth)
    s.speculative_step_forced(first, depth, 0)
    drafts = [int(t) for t in s.buffer("drafts", np.uint32, depth)]
    token, hidden = first, o.last_hidden
    checked = 0
    for i in range(depth):
        want, logits, hidden = o.mtp_proposal(token, hidden, i)
        top2 = np.sort(logits[0])[-2:]
        if top2[1] - top2[0] > 2 * LOGIT_TOL:
            assert drafts[i] == want, (i, drafts, want)
            checked += 1
        token = drafts[i]
    say("drafts", drafts, "checked", checked)
    assert checked >= 1
