""".gfxi reader, checksum and gfx12 -> gfx950 conversion on the host (no GPU).

Pinned by a fixture the reference's own ArtifactWriter and gfx12 tiler wrote
(tests/golden/make_artifact_golden.py), by the published CRC-64/ECMA-182 check value,
and, where oracle/_ref is built, by the reference reader's verdict on the same files.
"""
from __future__ import annotations

import os
import shutil

import numpy as np
import pytest

from conftest import golden

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "artifact_gfx1200_small.gfxi")
OK, INVALID, IO, CORRUPT, UNSUPPORTED = 0, 1, 2, 3, 4


def _open_rc(path, verify=True):
    import ctypes
    from gfxinfer_amd import lib
    handle = ctypes.c_void_p()
    rc = lib().gfxinfer_artifact_open(str(path).encode(), int(verify), ctypes.byref(handle))
    if rc == OK:
        lib().gfxinfer_artifact_close(handle)
    return rc


def test_crc64_ecma_check_value(orc):
    from gfxinfer_amd.runtime import crc64_ecma
    assert crc64_ecma(b"123456789") == 0x6C40DF5F0B497347  # CRC-64/ECMA-182 check value
    assert crc64_ecma(b"") == 0
    # incremental == one shot, and agreement with the reference on random data
    data = np.random.default_rng(3).integers(0, 256, 1000, dtype=np.uint8).tobytes()
    assert crc64_ecma(data[700:], crc64_ecma(data[:700])) == crc64_ecma(data)
    R = orc.ref_lib()
    if R is not None:
        for n in (1, 7, 8, 9, 1000):
            assert crc64_ecma(data[:n]) == R.ref_crc64_ecma(data[:n], n)


def test_reads_reference_written_artifact():
    from gfxinfer_amd.runtime import Artifact
    g = golden("artifact_gfx1200_small.npz")
    with Artifact(FIXTURE) as a:
        assert a.identity() == {"target_arch": "gfx1200", "model_id": "qwen3.8-27b",
                                "weights_id": "golden-small",
                                "recipe_id": "qwen38-code-w3seq-w4-wmma-tiled-v9"}
        tensors = {t.name.decode(): t for t in a.tensors()}
        assert list(tensors) == ["layers.0.mlp.gate_proj.weight", "layers.0.self_attn.q_proj.weight",
                                 "layers.1.mlp.down_proj.weight", "layers.0.input_layernorm.weight",
                                 "layers.0.linear_attn.conv1d.weight", "mtp.draft_head_token_ids"]
        q = tensors["layers.0.self_attn.q_proj.weight"]
        assert (q.dtype, q.quantization, q.shape) == (1, 3, (48, 384))
        assert q.data_bytes == 48 * 384 // 2 and q.aux_bytes == 48 * 3 * 2
        assert q.data_offset % 256 == 0 and q.aux_offset % 256 == 0
        conv = tensors["layers.0.linear_attn.conv1d.weight"]
        assert (conv.dtype, conv.shape) == (4, (16, 1, 4))
        assert np.array_equal(a.payload(conv).view(np.uint16), g["conv"])
        ids = a.find("mtp.draft_head_token_ids")
        assert ids.dtype == 2 and np.array_equal(a.payload(ids).view(np.int32), g["ids"])
        norm = a.find("layers.0.input_layernorm.weight")
        assert np.array_equal(a.payload(norm).view(np.uint16), g["norm"])


@pytest.mark.parametrize("name,fmt,rows,cols", [("layers.0.mlp.gate_proj.weight", 2, 32, 256),
                                                ("layers.0.self_attn.q_proj.weight", 3, 48, 384),
                                                ("layers.1.mlp.down_proj.weight", 2, 16, 640)])
def test_gfx12_tiles_convert_to_gfx950_tiles(orc, gx, name, fmt, rows, cols):
    """The loader's conversion of the reference's gfx12 tiles equals the library's own
    tiling of the same packed codes; scales need none (same [tile][group][16] order)."""
    from gfxinfer_amd.runtime import Artifact, retile_gfx12_for_gfx950
    g = golden("artifact_gfx1200_small.npz")
    key = name.replace(".", "_")
    want_codes, want_scales = gx.tile_group128(fmt, g[key + "__packed"], g[key + "__scales"], rows, cols)
    with Artifact(FIXTURE) as a:
        t = a.find(name)
        got = retile_gfx12_for_gfx950(fmt, a.payload(t))
        scales = a.payload(t, auxiliary=True).view(np.uint16)
    assert np.array_equal(got, want_codes)
    assert np.array_equal(scales, want_scales)


@pytest.mark.parametrize("rows,cols", [(16, 128), (32, 640)])
def test_gfx12_w2_tiles_convert_to_gfx950_tiles(orc, gx, rows, cols):
    """W2 (no fixture holds it): the reference quantizer and gfx12 tiler compiled in place
    make the gfx1200-recipe codes; re-tiling them gives the library's own gfx950 tiling
    of the same packed codes, and the codes decode to the reference's levels."""
    if orc.ref_lib() is None:
        pytest.skip("oracle/_ref (the reference quantizer and gfx12 tiler) is not built")
    from gfxinfer_amd.runtime import retile_gfx12_for_gfx950
    w = (np.random.default_rng(rows + cols).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    status, codes, scales = orc.ref_quantize_group128(w, 1)
    assert status == 0
    gfx12, gscales = orc.ref_tile_gfx12(codes, scales, rows, cols, 1)
    want, want_scales = gx.tile_group128(1, codes, scales, rows, cols)
    got = retile_gfx12_for_gfx950(1, gfx12)
    assert np.array_equal(got, want)
    assert np.array_equal(orc.f32_to_f16_bits(gscales).reshape(-1), want_scales)
    wq, _ = gx.untile_group128(1, got, want_scales, rows, cols)
    assert np.array_equal(wq, orc.unpack_weights(codes, rows, cols, 1))
    assert set(np.unique(wq)) <= {-3, -1, 1, 3}


def _corrupt(tmp_path, edit):
    path = tmp_path / "c.gfxi"
    shutil.copy(FIXTURE, path)
    data = bytearray(path.read_bytes())
    data = edit(data)
    path.write_bytes(bytes(data))
    return path


@pytest.mark.parametrize("case,want,want_unverified", [
    ("payload_byte", CORRUPT, OK),      # tensor checksum
    ("name_byte", CORRUPT, CORRUPT),    # manifest checksum, then the name check
    ("magic", CORRUPT, CORRUPT),
    ("version", UNSUPPORTED, UNSUPPORTED),
    ("truncated", CORRUPT, CORRUPT),
    ("short", CORRUPT, CORRUPT),
])
def test_rejects_damaged_artifacts(orc, tmp_path, case, want, want_unverified):
    from gfxinfer_amd.runtime import Artifact
    with Artifact(FIXTURE) as a:
        q = a.find("layers.0.self_attn.q_proj.weight")
    first_name = 256 + 6 * 128  # header + directory

    def edit(d):
        if case == "payload_byte":
            d[q.data_offset + 5] ^= 0x40
        elif case == "name_byte":
            d[first_name] = ord("!")
        elif case == "magic":
            d[0] ^= 1
        elif case == "version":
            d[8] = 2
        elif case == "truncated":
            d = d[:-100]
        elif case == "short":
            d = d[:100]
        return d

    path = _corrupt(tmp_path, edit)
    assert _open_rc(path, True) == want
    assert _open_rc(path, False) == want_unverified
    if orc.ref_lib() is not None:  # the reference reader agrees
        assert orc.ref_open_artifact(path, True)[0] == want
        assert orc.ref_open_artifact(path, False)[0] == want_unverified


def test_missing_file_is_io_error(tmp_path):
    assert _open_rc(tmp_path / "absent.gfxi") == IO


TINY_MODEL = os.path.join(HERE, "golden", "artifact_gfx1200_tiny_model.gfxi")
RECIPE_OFFSET = 168  # header: magic .. manifest CRC (88 bytes), target 16, model 32, weights 32


@pytest.mark.parametrize("recipe", [
    "qwen38-code-w3seq-w4-rowmajor-v9",  # row-major codes (no "tiled-v")
    "qwen38-code-w4-wmma-tiled-v7",      # W3 tensors without "w3seq": bit-plane W3
])
def test_loader_refuses_gfx1200_layouts_it_does_not_retile(tmp_path, recipe):
    """qwen_runtime.cpp:957-960: the reference reads gfx1200 codes as tiles only under a
    "tiled-v" recipe and W3 as sequential fragments only under "w3seq".  The loader
    refuses the other layouts with GFXI_UNSUPPORTED before any device work (the recipe id
    is outside the checksummed manifest, so the patched file still opens)."""
    import ctypes
    from gfxinfer_amd import lib
    from gfxinfer_amd.runtime import Artifact, artifact_tiny_spec
    path = tmp_path / "patched.gfxi"
    data = bytearray(open(TINY_MODEL, "rb").read())
    assert bytes(data[RECIPE_OFFSET:RECIPE_OFFSET + 34]) == b"qwen38-code-w3seq-w4-wmma-tiled-v9"
    data[RECIPE_OFFSET:RECIPE_OFFSET + 64] = recipe.encode().ljust(64, b"\0")
    path.write_bytes(bytes(data))
    with Artifact(path) as a:
        assert a.identity()["recipe_id"] == recipe
    spec = artifact_tiny_spec()
    handle = ctypes.c_void_p()
    rc = lib().gfxinfer_model_create_from_artifact(ctypes.byref(spec), str(path).encode(), 1, 0,
                                                   ctypes.byref(handle))
    assert rc == UNSUPPORTED, lib().gfxinfer_last_error()
    assert not handle.value


def test_tiny_model_fixture_covers_the_spec():
    """The committed gfx1200 model fixture holds every tensor the tiny spec binds, in the
    converter's shapes, with the quantization the spec gives it."""
    from gfxinfer_amd.runtime import Artifact, artifact_tiny_spec, spec_tensors
    with Artifact(TINY_MODEL) as a:
        assert a.identity()["weights_id"] == "synthetic-77"
        found = {t.name.decode(): t for t in a.tensors()}
    want = spec_tensors(artifact_tiny_spec())
    assert sorted(found) == sorted(t["name"] for t in want)
    for t in want:
        e = found[t["name"]]
        assert e.quantization == max(t["format"], 0)
        assert int(np.prod(e.shape)) == t["rows"] * t["columns"]
