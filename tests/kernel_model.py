"""numpy model of gfxinfer_amd/csrc/lowbit_gemv.hip's GEMM kernel.

Replays the kernel's operand expansion (the shift/mask bit tricks) and its lane
mapping (group packing GP, token slots, lane blocks) on the CPU, with the MFMA
modelled as C[m][n] += sum over (lane block kb, byte j) of
A[lane m+16kb][j] * B[lane n+16kb][j] -- i.e. assuming only that the A and B
operands of v_mfma_i32_16x16x64_i8 share one K-slot order and that lane l of C
holds rows 4*(l//16)..+3 of column l%16.  The GPU probe test checks that
assumption on the hardware; these tests check the rest on the CPU.
"""
from __future__ import annotations

import numpy as np

W2, W3, W4 = 1, 2, 3


def lane_bytes(fmt: int) -> int:
    return {W2: 8, W3: 12}.get(fmt, 16)


def i8(x: np.ndarray) -> np.ndarray:
    """uint32 array -> int8 bytes [..., 4] (little endian)."""
    return np.ascontiguousarray(x, dtype=np.uint32).view(np.int8).reshape(x.shape + (4,))


def expand_nibbles(x0, x1):
    """expand_nibbles(): four operand registers (value 16*x)."""
    M = np.uint32(0xF0F0F0F0)
    return [(x0 << np.uint32(4)) & M, x0 & M, (x1 << np.uint32(4)) & M, x1 & M]


def expand_w2(d):
    """expand_w2(): four operand registers (value 32*w, w = 2c - 3)."""
    M, X = np.uint32(0xC0C0C0C0), np.uint32(0xA0A0A0A0)
    return [((d << np.uint32(s)) & M) ^ X for s in (6, 4, 2, 0)]


def expand_w3(s0, s1, s2):
    E = np.uint32(0xE0E0E0E0)
    h0 = [(s0 << np.uint32(5)) & E, (s0 << np.uint32(2)) & E, (s1 << np.uint32(5)) & E, (s1 << np.uint32(2)) & E]
    h1 = [(s2 << np.uint32(5)) & E, (s2 << np.uint32(2)) & E,
          (s0 & np.uint32(0xC0C0C0C0)) | ((s1 >> np.uint32(1)) & np.uint32(0x20202020)),
          (s2 & np.uint32(0xC0C0C0C0)) | ((s1 >> np.uint32(2)) & np.uint32(0x20202020))]
    return h0, h1


def perm(hi, lo, sel):
    """v_perm_b32 restricted to byte selectors 0..7."""
    src = np.concatenate([i8(lo).view(np.uint8), i8(hi).view(np.uint8)], axis=-1)
    out = np.zeros(lo.shape, dtype=np.uint32)
    for i in range(4):
        s = (sel >> (8 * i)) & 0xFF
        out |= src[..., s].astype(np.uint32) << np.uint32(8 * i)
    return out


def permute_i8(d0, d1, d2, d3):
    return [perm(d1, d0, 0x06040200), perm(d1, d0, 0x07050301), perm(d3, d2, 0x06040200), perm(d3, d2, 0x07050301)]


def regs_to_bytes(regs) -> np.ndarray:
    """list of 4 uint32 registers [...] -> int8 [..., 16] in operand byte order."""
    return np.concatenate([i8(r) for r in regs], axis=-1)


def simulate_partials(fmt: int, tiled: np.ndarray, abits: int, acts: np.ndarray, rows: int,
                      columns: int, batch: int) -> np.ndarray:
    """int32 P[batch, rows, G] as the kernel computes it (exact integer model).

    Each group is one MFMA pair: A lane l = layout lane l of the group; B lane
    (column n, block kb) is live only when n // TPAD is the group's window in its
    pack and the token slot n % TPAD (+16 t) is below the batch."""
    G = columns // 128
    LB = lane_bytes(fmt)
    F = (16 if fmt == W4 else 32) * (16 if abits == 4 else 1)
    if batch <= 8:
        GP, NTB = 2, 1
    elif batch <= 16:
        GP, NTB = 1, 1
    else:
        GP, NTB = 1, 2
    TPAD = 16 // GP
    chunks = tiled.reshape(rows // 16, G, 64, LB)
    lanes = np.arange(64)
    n = lanes % 16
    kb = lanes // 16
    slot = n % TPAD
    window = n // TPAD
    out = np.zeros((batch, rows, G), dtype=np.int64)
    packs = (G + GP - 1) // GP
    for tile in range(rows // 16):
        for pack in range(packs):
            C = np.zeros((NTB, 16, 16), dtype=np.int64)  # [t][row][column]
            for j in range(GP):
                g = pack * GP + j
                if g >= G:
                    break
                d = chunks[tile, g].copy().view(np.uint32).reshape(64, LB // 4)
                if fmt == W2:
                    h0, h1 = expand_w2(d[:, 0]), expand_w2(d[:, 1])
                elif fmt == W3:
                    h0, h1 = expand_w3(d[:, 0], d[:, 1], d[:, 2])
                else:
                    h0, h1 = expand_nibbles(d[:, 0], d[:, 1]), expand_nibbles(d[:, 2], d[:, 3])
                A = [regs_to_bytes(h0).astype(np.int64), regs_to_bytes(h1).astype(np.int64)]
                for t in range(NTB):
                    token = t * 16 + slot
                    on = (window == j) & (token < batch)
                    Bh = [np.zeros((64, 16), dtype=np.int64), np.zeros((64, 16), dtype=np.int64)]
                    for l in range(64):
                        if not on[l]:
                            continue
                        col = g * 128 + kb[l] * 32
                        if abits == 4:
                            x = acts[token[l], col // 2: col // 2 + 16].copy().view(np.uint32)
                            regs = [expand_nibbles(x[0:1], x[1:2]), expand_nibbles(x[2:3], x[3:4])]
                        else:
                            x = acts[token[l], col: col + 32].copy().view(np.uint32)
                            regs = [permute_i8(x[0:1], x[1:2], x[2:3], x[3:4]),
                                    permute_i8(x[4:5], x[5:6], x[6:7], x[7:8])]
                        for h in range(2):
                            Bh[h][l] = regs_to_bytes(regs[h])[0]
                    for h in range(2):
                        # MFMA: C[row][col] += sum_kb sum_j A[row+16kb][j] * B[col+16kb][j]
                        Ar = A[h].reshape(4, 16, 16)   # [kb][row][j]
                        Br = Bh[h].reshape(4, 16, 16)  # [kb][col][j]
                        C[t] += np.einsum("krj,kcj->rc", Ar, Br)
            for t in range(NTB):
                for col in range(16):
                    token = t * 16 + col % TPAD
                    g_c = pack * GP + col // TPAD
                    if token < batch and g_c < G:
                        v = C[t][:, col]
                        assert np.all(v % F == 0)
                        out[token, tile * 16:(tile + 1) * 16, g_c] = v // F
                    else:
                        assert np.all(C[t][:, col] == 0)
    return out.astype(np.int32)
