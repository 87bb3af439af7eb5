"""Loading models from .gfxi artifacts on the GPU.

- gfx950 recipe: a synthetic model written by the library and loaded back is the same
  model byte for byte and gives the same tokens and logits; the reference reader
  (oracle/_ref, where built) accepts the file.
- gfx1200 recipe: synthetic weights quantized, gfx12-tiled and written by the
  reference's own code (quantizer, tile_group128_for_gfx12, ArtifactWriter) in the CPU
  container (a committed fixture; no reference code runs on the GPU box) load into the
  identical gfx950 arena.
- The converter's MTP draft head (ranked LM-head rows + token ids) drives the MTP
  proposal through the token-id map.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu
SEED = 77


def _spec():
    from gfxinfer_amd.runtime import tiny_spec
    return tiny_spec(full_attention_interval=2, gdn_key_head_count=4)


@pytest.fixture(scope="module")
def model(device):
    from gfxinfer_amd.runtime import SyntheticModel
    say("synthetic model for artifacts")
    m = SyntheticModel(_spec(), SEED)
    yield m
    m.close()


def _names(path):
    from gfxinfer_amd.runtime import Artifact
    with Artifact(path) as a:
        return [(t.name.decode(), t.quantization, t.shape) for t in a.tensors()]


def _same_arena(a, b, names):
    for name, quant, _ in names:
        assert np.array_equal(a.tensor_bytes(name), b.tensor_bytes(name)), name
        if quant != 0:
            assert np.array_equal(a.tensor_bytes(name, True), b.tensor_bytes(name, True)), name


def _outputs(model):
    """Verifier tokens and logits of one 4-token block, and one greedy step's MTP proposal."""
    from gfxinfer_amd.runtime import QwenDecodeSession
    spec = model.spec
    s = QwenDecodeSession(model, 64, 0, keep_logits=True)
    try:
        tokens = s.block_step([5, 77, 301, 9])
        logits = s.buffer("logits", np.float32, 4 * spec.vocabulary_size)
    finally:
        s.close()
    s = QwenDecodeSession(model, 64, 0, keep_logits=True)
    try:
        first = s.greedy_step(42)
        draft = s.mtp_draft(first)
        draft_logits = s.buffer("logits", np.float32, spec.mtp_draft_vocabulary)
    finally:
        s.close()
    return tokens + [first, draft], logits, draft_logits


def test_gfx950_artifact_round_trip(model, orc, tmp_path):
    from gfxinfer_amd.runtime import Artifact, SyntheticModel
    path = tmp_path / "tiny_gfx950.gfxi"
    say("write gfx950 artifact")
    model.write_artifact(path, "synthetic-77")
    names = _names(path)
    with Artifact(path) as a:
        ident = a.identity()
        assert (ident["target_arch"], ident["weights_id"]) == ("gfx950", "synthetic-77")
        conv = [t for t in a.tensors() if t.name.decode().endswith("conv1d.weight")][0]
        assert conv.rank == 3 and conv.dimensions[1] == 1
    if orc.ref_lib() is not None:
        assert orc.ref_open_artifact(path, True) == (0, len(names))
    say("load gfx950 artifact")
    loaded = SyntheticModel.from_artifact(_spec(), path)
    try:
        _same_arena(model, loaded, names)
        say("sessions on both models")
        want, got = _outputs(model), _outputs(loaded)
    finally:
        loaded.close()
    assert got[0] == want[0]
    assert np.array_equal(got[1], want[1]) and np.array_equal(got[2], want[2])


def test_gfx1200_artifact_from_reference_writer(device):
    """tests/golden/artifact_gfx1200_tiny_model.gfxi holds the synthetic model of
    artifact_tiny_spec() (seed 77) as the reference's own quantizer, gfx12 tiler and
    ArtifactWriter wrote it in this repository's CPU container: loading it re-tiles every
    matrix into exactly the arena the device generator fills."""
    import os
    from gfxinfer_amd.runtime import SyntheticModel, artifact_tiny_spec, spec_tensors
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "artifact_gfx1200_tiny_model.gfxi")
    spec = artifact_tiny_spec()
    say("load the reference-written gfx1200 artifact")
    loaded = SyntheticModel.from_artifact(spec, path)
    generated = SyntheticModel(spec, SEED)
    try:
        names = [(t["name"], max(t["format"], 0), None) for t in spec_tensors(spec)]
        _same_arena(generated, loaded, names)
    finally:
        loaded.close()
        generated.close()


def test_reference_shape_artifact_loads_and_runs(device):
    """tests/golden/artifact_gfx1200_reference_shape_model.gfxi: a model of the reference's
    own head shapes (256-dim attention heads, six query heads per KV head, rotary 64, GDN
    16 key / 48 value heads; qwen38_spec.h:22-29) written in this repository's CPU
    container by the reference's quantizer, gfx12 tiler and ArtifactWriter.  It loads into
    the arena the device generator fills for the same spec, and a verifier block and an
    MTP proposal on it match the CPU model oracle (logits within 2e-2)."""
    import os
    from gfxinfer_amd.runtime import QwenDecodeSession, SyntheticModel, artifact_reference_tiny_spec, spec_tensors
    from oracle.model import OracleModel, OracleSession
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "artifact_gfx1200_reference_shape_model.gfxi")
    spec = artifact_reference_tiny_spec()
    say("load the reference-shaped gfx1200 artifact")
    loaded = SyntheticModel.from_artifact(spec, path)
    generated = SyntheticModel(spec, SEED)
    try:
        names = [(t["name"], max(t["format"], 0), None) for t in spec_tensors(spec)]
        _same_arena(generated, loaded, names)
        V, Vt = spec.vocabulary_size, spec.tokenizer_vocabulary_size
        oracle = OracleSession(OracleModel(spec.as_dict(), SEED), 64)
        s = QwenDecodeSession(loaded, 64, 0, keep_logits=True)
        try:
            block = [5, 77, 201, 9, 130]
            say("reference-shaped block step")
            got = s.block_step(block)
            want, want_logits = oracle.block_step(block)
            logits = s.buffer("logits", np.float32, len(block) * V).reshape(len(block), V)
            assert np.abs(logits - want_logits).max() <= 2e-2
            assert float(want_logits.std()) > 0.01
            top2 = np.sort(want_logits[:, :Vt], axis=1)[:, -2:]
            sure = top2[:, 1] - top2[:, 0] > 4e-2
            assert np.array_equal(np.asarray(got)[sure], np.asarray(want)[sure])
        finally:
            s.close()
        oracle = OracleSession(OracleModel(spec.as_dict(), SEED), 64)
        s = QwenDecodeSession(loaded, 64, 0, keep_logits=True)
        try:
            say("reference-shaped greedy step + MTP proposal")
            first = s.greedy_step(42)
            want_first, _ = oracle.block_step([42])
            draft = s.mtp_draft(first)
            want_draft, draft_logits, _ = oracle.mtp_proposal(first, oracle.last_hidden, 0)
            got_logits = s.buffer("logits", np.float32, spec.mtp_draft_vocabulary)
            assert np.abs(got_logits - draft_logits[0]).max() <= 2e-2
            top2 = np.sort(draft_logits[0])[-2:]
            if top2[1] - top2[0] > 4e-2:
                assert draft == want_draft
        finally:
            s.close()
    finally:
        loaded.close()
        generated.close()


def test_draft_head_artifact_uses_token_ids(model, tmp_path):
    from gfxinfer_amd.runtime import SyntheticModel
    spec = _spec()
    n = spec.mtp_draft_vocabulary
    rng = np.random.default_rng(5)
    # (a) the same candidate rows in another order: the proposal is unchanged
    perm = rng.permutation(n).astype(np.uint32)
    path = tmp_path / "draft_perm.gfxi"
    say("artifact with a permuted draft head")
    model.write_artifact(path, "synthetic-77", draft_rows=perm)
    loaded = SyntheticModel.from_artifact(spec, path)
    try:
        assert np.array_equal(loaded.tensor_bytes("mtp.draft_head_token_ids").view(np.uint32), perm)
        want, got = _outputs(model), _outputs(loaded)
    finally:
        loaded.close()
    assert got[0] == want[0]
    assert np.array_equal(got[2], want[2][perm])  # the draft logits come in the artifact's row order
    # (b) other rows: the proposal is ids[argmax of the draft head's own logits]
    rows = rng.choice(spec.vocabulary_size, n, replace=False).astype(np.uint32)
    path = tmp_path / "draft_other.gfxi"
    model.write_artifact(path, "synthetic-77", draft_rows=rows)
    loaded = SyntheticModel.from_artifact(spec, path)
    try:
        got = _outputs(loaded)
    finally:
        loaded.close()
    draft, logits = got[0][-1], got[2]
    assert draft == int(rows[int(np.argmax(logits))])


def test_load_rejects_mismatched_spec(model, tmp_path):
    from gfxinfer_amd import GfxinferError
    from gfxinfer_amd.runtime import SyntheticModel, tiny_spec
    path = tmp_path / "tiny.gfxi"
    model.write_artifact(path, "synthetic-77")
    with pytest.raises(GfxinferError) as e:
        SyntheticModel.from_artifact(tiny_spec(full_attention_interval=2, gdn_key_head_count=2), path)
    assert e.value.code == 3  # corrupt_artifact: shape does not match the spec
