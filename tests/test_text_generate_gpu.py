"""Text-level generation (cli/main.cpp:1023-1120): chat rendering, tokenizer encode,
the generate loop on the GPU, decode.  The tiny synthetic model's greedy vocabulary is
the tokenizer fixture's (tests/golden/tokenizer_small.json), so every generated id
decodes.  Checked: the prompt ids equal the CPU tokenizer oracle's, the generated ids
equal the reference's serial loop run through the same session API and, where the CPU
model oracle's top-2 margin is clear, its greedy token after the prompt; the decoded
bytes equal the oracle tokenizer's decode of the same ids."""
from __future__ import annotations

import os

import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu
SEED = 404
HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "tokenizer_small.json")
PROMPTS = ["What is 12*7? Answer briefly, please.", "héllo wörld — naïve café", ""]


@pytest.fixture(scope="module")
def setup(device):
    from gfxinfer_amd.runtime import SyntheticModel, Tokenizer, tiny_spec
    document = open(FIXTURE, "rb").read()
    tokenizer = Tokenizer(document)
    spec = tiny_spec(tokenizer_vocabulary_size=tokenizer.vocabulary_size, mtp_draft_vocabulary=512)
    say("tiny model with the fixture tokenizer's vocabulary")
    model = SyntheticModel(spec, SEED)
    yield tokenizer, document, spec, model
    model.close()
    tokenizer.close()


@pytest.mark.parametrize("depth", [0, 3])
@pytest.mark.parametrize("prompt", PROMPTS)
def test_generate_text_matches_serial_loop_and_oracles(setup, prompt, depth):
    from gfxinfer_amd.runtime import QwenDecodeSession, generate_text
    from oracle.tokenizer import OracleTokenizer, render_chat_prompt
    from test_prefill_generate_gpu import reference_generate
    tokenizer, document, spec, model = setup
    oracle = OracleTokenizer(document)
    say("generate_text", repr(prompt), depth)
    a = QwenDecodeSession(model, 256, depth + 1 if depth else 0)
    got = generate_text(a, tokenizer, prompt, 20, depth)
    a.close()
    assert got["prompt_ids"] == oracle.encode(render_chat_prompt(prompt))
    assert sorted(got["stop_ids"]) == sorted(oracle.ids[p] for p in ("<|im_end|>", "<|endoftext|>"))
    b = QwenDecodeSession(model, 256, depth + 1 if depth else 0)
    want, _ = reference_generate(b, np.asarray(got["prompt_ids"], np.uint32), 20, depth, tuple(got["stop_ids"]))
    b.close()
    assert got["tokens"] == want
    assert all(t < tokenizer.vocabulary_size for t in got["tokens"])
    assert got["text"] == oracle.decode_bytes(got["tokens"])
    stopped = got["tokens"][-1] in got["stop_ids"]
    assert len(got["tokens"]) == 20 or stopped


def test_first_token_matches_model_oracle(setup):
    """The token after the rendered prompt against the CPU model oracle (oracle/model.py)
    where its top-2 logit margin exceeds the parity bar."""
    from gfxinfer_amd.runtime import QwenDecodeSession, generate_text
    from oracle.model import OracleModel, OracleSession
    tokenizer, document, spec, model = setup
    s = QwenDecodeSession(model, 256, 0)
    got = generate_text(s, tokenizer, PROMPTS[0], 1, 0)
    s.close()
    cpu = OracleSession(OracleModel(spec.as_dict(), SEED), 256)
    ids = got["prompt_ids"]
    for start in range(0, len(ids), 32):  # the prompt in verifier-sized blocks
        _, logits = cpu.block_step(ids[start:start + 32])
    last = logits[-1, :spec.tokenizer_vocabulary_size]
    top2 = np.sort(last)[-2:]
    if top2[1] - top2[0] > 4e-2:
        assert got["tokens"][0] == int(np.argmax(last))
    else:
        say("oracle margin below the bar; first token unchecked")


def test_generate_text_refuses_a_prompt_beyond_the_context(setup):
    from gfxinfer_amd import GfxinferError
    from gfxinfer_amd.runtime import QwenDecodeSession, generate_text
    tokenizer, _, _, model = setup
    s = QwenDecodeSession(model, 64, 0)
    with pytest.raises(GfxinferError):
        generate_text(s, tokenizer, "word " * 80, 8, 0)
    s.close()
