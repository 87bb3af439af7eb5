"""Writes the quantizer golden fixtures from the reference's own code.

The reference's src/quantization.cpp is compiled where it lies by
`make -C oracle ref` into oracle/_ref/libgfxref.so; this script feeds it seeded
inputs and stores inputs and outputs (packed codes, float scales and the
reference dequantization) as .npz files next to this script.  Only the data is
committed.  Re-running it must reproduce the committed files byte for byte.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def cases() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(0x5EED0003)
    out: dict[str, np.ndarray] = {}
    # quantization_test.cpp:12-21 shape and plants: 3x256 ~N(0,0.25), 0 / +2 / -2.
    a = (rng.standard_normal((3, 256)) * 0.25).astype(np.float32)
    a[0, 0] = 0.0
    a[1, 17] = 2.0
    a[2, 93] = -2.0
    out["planted_3x256"] = a
    # quantization_test.cpp:49-55 shape: 32x256 ~N(0,0.5).
    out["normal_32x256"] = (rng.standard_normal((32, 256)) * 0.5).astype(np.float32)
    # BASELINE distribution N(0, 0.02), 16 rows x 4 groups.
    out["baseline_16x512"] = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    # Edge groups, one per row (16 rows x 128):
    e = np.zeros((16, 128), dtype=np.float32)
    e[1, 5] = 1.0                                   # single non-zero
    e[2, :] = np.float32(0.75)                      # constant group
    e[3, :] = np.linspace(-1, 1, 128, dtype=np.float32)
    e[4, :] = (np.arange(128) - 64).astype(np.float32) * np.float32(0.125)  # exact multiples
    e[5, :] = (np.arange(128) % 16 - 8).astype(np.float32) + np.float32(0.5)  # ties at .5
    e[6, :] = rng.standard_normal(128).astype(np.float32) * np.float32(1e-38)  # subnormal-ish
    e[7, :] = rng.standard_normal(128).astype(np.float32) * np.float32(1e30)   # huge
    e[8, :] = -np.abs(rng.standard_normal(128)).astype(np.float32)             # one-signed
    e[9, :] = np.abs(rng.standard_normal(128)).astype(np.float32)
    e[10, 0] = np.float32(3.0)
    e[10, 1:] = np.float32(-1.0)                    # large positive outlier
    e[11, 0] = np.float32(-3.0)
    e[11, 1:] = np.float32(1.0)                     # large negative outlier
    e[12, :] = rng.standard_normal(128).astype(np.float32) * np.float32(0.02)
    e[12, 64] = np.float32(0.3)                     # one big value in N(0,0.02)
    e[13, :] = np.float32(np.finfo(np.float32).tiny)
    e[14, ::2] = np.float32(1.0)
    e[14, 1::2] = np.float32(-1.0)
    e[15, :] = rng.standard_t(2, 128).astype(np.float32)                       # heavy tails
    out["edges_16x128"] = e
    return out


def main() -> None:
    if O.ref_lib() is None:
        O.build(reference=True)
    if O.ref_lib() is None:
        raise SystemExit("oracle/_ref/libgfxref.so is unavailable (needs the reference tree)")
    for fmt, name in ((O.W2, "w2"), (O.W3, "w3"), (O.W4, "w4")):
        arrays = {}
        for key, w in cases().items():
            status, codes, scales = O.ref_quantize_group128(w, fmt)
            assert status == 0, (name, key, status)
            deq = np.empty_like(w)
            R = O.ref_lib()
            st = R.ref_dequantize_group128(O.ptr(codes), O.ptr(scales), w.shape[0], w.shape[1], fmt, O.ptr(deq))
            assert st == 0
            arrays[f"{key}__input"] = w
            arrays[f"{key}__codes"] = codes
            arrays[f"{key}__scales"] = scales
            arrays[f"{key}__dequant"] = deq
        # A rejected input: K = 127 (quantization_test.cpp:126-132) and a NaN row.
        bad = np.zeros((1, 127), dtype=np.float32)
        arrays["reject_k127__status"] = np.array([O.ref_quantize_group128(bad, fmt)[0]], dtype=np.int32)
        nan = np.zeros((1, 128), dtype=np.float32)
        nan[0, 3] = np.nan
        arrays["reject_nan__status"] = np.array([O.ref_quantize_group128(nan, fmt)[0]], dtype=np.int32)
        path = os.path.join(HERE, f"quant_{name}.npz")
        np.savez_compressed(path, **arrays)
        print("wrote", path)


if __name__ == "__main__":
    main()
