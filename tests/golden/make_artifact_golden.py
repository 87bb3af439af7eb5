"""Writes the .gfxi artifact fixture from the reference's own code.

The reference's src/quantization.cpp and src/artifact.cpp are compiled where they lie by
`make -C oracle ref` into oracle/_ref/libgfxref.so.  This script quantizes seeded
matrices with the reference quantizer, tiles them with the reference's gfx12 tiler
(quantization.cpp:253-318) and writes them, with bf16 and int32 vectors, through the
reference ArtifactWriter (artifact.cpp:427-545) as a "gfx1200" artifact — the layout the
reference converter emits (converter.cpp:345-393), under the recipe id the converter
gives a W3-sequential tiled checkpoint (converter.cpp:540-541): the reference runtime
reads codes as tiled only when the recipe names "tiled-v" and W3 as sequential only
when it names "w3seq" (qwen_runtime.cpp:957-960).  The inputs (packed codes, float
scales) are stored next to it so the tests can build the expected gfx950 tiles with the
library's own tiler.

A second file holds a whole synthetic model (the smallest spec the kernels take, seed
77) in the same recipe, every matrix quantized by the reference quantizer and tiled by
the reference tiler, for the GPU test that loads it into the library's arena.  A third
holds the same kind of model at the reference model's own head shapes (256-dim
attention heads, six query heads per KV head, GDN 16 key / 48 value heads:
artifact_reference_tiny_spec()).  Only data is committed; re-running reproduces the
files.

    python tests/golden/make_artifact_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

RECIPE = "qwen38-code-w3seq-w4-wmma-tiled-v9"
IDENTITY = ("gfx1200", "qwen3.8-27b", "golden-small", RECIPE)
MODEL_SEED = 77
MATRICES = [("layers.0.mlp.gate_proj.weight", 2, 32, 256),   # W3
            ("layers.0.self_attn.q_proj.weight", 3, 48, 384),  # W4
            ("layers.1.mlp.down_proj.weight", 2, 16, 640)]     # W3, five groups


def main() -> None:
    if O.ref_lib() is None:
        raise SystemExit("oracle/_ref is not built (make -C oracle ref)")
    rng = np.random.default_rng(0x5EED0A27)
    tensors, arrays = [], {}
    for name, fmt, rows, cols in MATRICES:
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        _, codes, scales = O.ref_quantize_group128(w, fmt)
        tiled, tscales = O.ref_tile_gfx12(codes, scales, rows, cols, fmt)
        key = name.replace(".", "_")
        arrays[key + "__packed"] = codes
        arrays[key + "__scales"] = scales
        tensors.append(dict(name=name, dtype=1, quantization=fmt, dims=(rows, cols), data=tiled.tobytes(),
                            aux=O.f32_to_f16_bits(tscales).tobytes()))
    norm = O.f32_to_bf16_bits(rng.standard_normal(64).astype(np.float32))
    conv = O.f32_to_bf16_bits(rng.standard_normal(16 * 4).astype(np.float32))
    ids = rng.permutation(1024)[:16].astype(np.int32)
    arrays["norm"] = norm
    arrays["conv"] = conv
    arrays["ids"] = ids
    tensors.append(dict(name="layers.0.input_layernorm.weight", dtype=4, quantization=0, dims=(64,),
                        data=norm.tobytes(), aux=None))
    tensors.append(dict(name="layers.0.linear_attn.conv1d.weight", dtype=4, quantization=0, dims=(16, 1, 4),
                        data=conv.tobytes(), aux=None))
    tensors.append(dict(name="mtp.draft_head_token_ids", dtype=2, quantization=0, dims=(16,),
                        data=ids.tobytes(), aux=None))
    path = os.path.join(HERE, "artifact_gfx1200_small.gfxi")
    if os.path.exists(path):
        os.remove(path)
    rc = O.ref_write_artifact(path, IDENTITY, tensors)
    if rc != 0:
        raise SystemExit(f"reference writer failed: {rc}")
    np.savez(os.path.join(HERE, "artifact_gfx1200_small.npz"), **arrays)
    print("wrote", path, os.path.getsize(path), "bytes")
    from gfxinfer_amd.runtime import artifact_reference_tiny_spec, artifact_tiny_spec
    write_tiny_model(artifact_tiny_spec(), "artifact_gfx1200_tiny_model.gfxi")
    write_tiny_model(artifact_reference_tiny_spec(), "artifact_gfx1200_reference_shape_model.gfxi")


def write_tiny_model(spec, filename) -> None:
    """The synthetic model of `spec` as the reference converter would write it."""
    from gfxinfer_amd.runtime import spec_tensors
    tensors = []
    for t in spec_tensors(spec):
        name, fmt, rows, cols = t["name"], t["format"], t["rows"], t["columns"]
        values = O.synthetic_values(MODEL_SEED, name, rows * cols, t["sigma"], t["mean"])
        if fmt == 0:
            dims = (rows, 1, cols) if name.endswith("conv1d.weight") else ((cols,) if rows == 1 else (rows, cols))
            tensors.append(dict(name=name, dtype=4, quantization=0, dims=dims,
                                data=O.f32_to_bf16_bits(values).tobytes(), aux=None))
            continue
        status, codes, scales = O.ref_quantize_group128(values.reshape(rows, cols), fmt)
        assert status == 0, name
        tiled, tscales = O.ref_tile_gfx12(codes, scales, rows, cols, fmt)
        tensors.append(dict(name=name, dtype=1, quantization=fmt, dims=(rows, cols), data=tiled.tobytes(),
                            aux=O.f32_to_f16_bits(tscales).tobytes()))
    path = os.path.join(HERE, filename)
    if os.path.exists(path):
        os.remove(path)
    rc = O.ref_write_artifact(path, ("gfx1200", "qwen3.8-27b", f"synthetic-{MODEL_SEED}", RECIPE), tensors)
    if rc != 0:
        raise SystemExit(f"reference writer failed: {rc}")
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
