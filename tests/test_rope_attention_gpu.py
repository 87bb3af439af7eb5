"""GPU parity of the fused Q/K RMSNorm + RoPE + K/V append + attention entry
(gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4[_indirect_position]).

The fused entry must give what its three-launch form gives (the RoPE launch with the K/V
append, then the attention launch with the A4 quantizer), bit for bit, with its cos / sin
evaluated and read from gfxinfer_launch_rope_table's table alike: the attention output,
its A4 codes and scales, and every cache row.  The cases put the block's new
positions inside one split, across a split boundary, at the start of the context and at
the end of the cache, at both model head shapes; the cache rows outside the block must
keep their contents.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import dev, empty, host, say

pytestmark = pytest.mark.gpu


def _bf16(x):
    x = np.asarray(x, dtype=np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def _fp16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


CASES = [
    # (HQ, HKV, D, rotary, T, position): 64-position splits at D = 128, 32 at D = 256
    (40, 8, 128, 32, 1, 400),
    (40, 8, 128, 32, 5, 1234),  # five tokens: two on the first wave
    (40, 8, 128, 32, 5, 61),    # positions 61..65 across the split boundary at 64
    (40, 8, 128, 32, 3, 0),     # the context's first tokens
    (40, 8, 128, 32, 6, 2042),  # the last rows of a 2048-row cache
    (24, 4, 256, 64, 1, 0),
    (24, 4, 256, 64, 5, 30),    # across the 32-position split boundary
    (24, 4, 256, 64, 2, 1500),
    (8, 1, 128, 64, 4, 100),    # eight query heads per KV head
    (8, 4, 128, 64, 8, 100),    # eight tokens: two per wave
    (16, 8, 256, 64, 8, 29),    # eight tokens across a split boundary at head size 256
]


@pytest.mark.parametrize("HQ,HKV,D,rot,T,position", CASES)
def test_fused_rope_attention_equals_three_launches(device, gx, HQ, HKV, D, rot, T, position):
    theta, cap = np.float32(1e7), 2048
    rng = np.random.default_rng(position * 7 + T + D)
    qin = rng.standard_normal((T, HQ, 2 * D)).astype(np.float32)  # query half then gate half per head
    kin = rng.standard_normal((T, HKV, D)).astype(np.float32)
    vin = rng.standard_normal((T, HKV * D)).astype(np.float32)
    qw, kw = _bf16(rng.standard_normal(D) * 0.1), _bf16(rng.standard_normal(D) * 0.1)
    # cached positions before the block hold plausible fp16 K/V; the rest is noise
    fill_k = _fp16(rng.standard_normal((cap, HKV * D)))
    fill_v = _fp16(rng.standard_normal((cap, HKV * D)))
    L = gx.lib()
    wb = gx.lib().gfxinfer_attention_workspace_bytes(T, HQ, D, cap)
    dq, dk, dv, dqw, dkw = dev(qin), dev(kin), dev(vin), dev(qw), dev(kw)
    work = empty((wb // 4,), np.float32)

    # three launches: RoPE + K/V append, then attention + A4
    kc, vc = dev(fill_k), dev(fill_v)
    qo, ko = empty((T, HQ, D), np.uint16), empty((T, HKV, D), np.uint16)
    out = empty((T, HQ * D), np.uint16)
    codes, scales = empty((T, HQ * D // 2), np.uint8), empty((T, HQ * D // 128), np.uint16)
    say("rope + attention, three launches", HQ, HKV, D, T, position)
    gx.check(L.gfxinfer_launch_qk_rms_norm_rope_kv_append_block(
        dq.data_ptr(), dqw.data_ptr(), qo.data_ptr(), HQ, 2 * D, dk.data_ptr(), dkw.data_ptr(), ko.data_ptr(),
        HKV, D, D, rot, dv.data_ptr(), kc.data_ptr(), vc.data_ptr(), cap, position, T, theta, None))
    gx.check(L.gfxinfer_launch_gated_attention_decode_block_quantize_i4(
        qo.data_ptr(), dq.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), codes.data_ptr(),
        scales.data_ptr(), position + 1, cap, T, HQ, HKV, D, work.data_ptr(), wb, None))
    want = [host(x, np.uint16) for x in (out, scales, kc, vc)] + [host(codes)]
    # the block's cache rows were written, the others kept
    assert not np.array_equal(want[2][position:position + T], fill_k[position:position + T])
    pos = dev(np.array([position], np.uint64))
    table = empty((L.gfxinfer_rope_table_bytes(cap, rot) // 4,), np.float32)
    gx.check(L.gfxinfer_launch_rope_table(table.data_ptr(), cap, rot, theta, None))
    for indirect, rope_table in ((False, None), (False, table.data_ptr()), (True, table.data_ptr())):
        kc2, vc2 = dev(fill_k), dev(fill_v)
        out2 = empty((T, HQ * D), np.uint16)
        codes2, scales2 = empty((T, HQ * D // 2), np.uint8), empty((T, HQ * D // 128), np.uint16)
        work.zero_()
        say("fused rope attention", HQ, HKV, D, T, position, indirect, rope_table is not None)
        args = (dq.data_ptr(), dqw.data_ptr(), 2 * D, dk.data_ptr(), dkw.data_ptr(), D, dv.data_ptr(), rot, theta,
                rope_table, dq.data_ptr(), kc2.data_ptr(), vc2.data_ptr(), out2.data_ptr(), codes2.data_ptr(),
                scales2.data_ptr())
        tail = (cap, T, HQ, HKV, D, work.data_ptr(), wb, None)
        if indirect:
            gx.check(L.gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4_indirect_position(
                *args, pos.data_ptr(), *tail))
        else:
            gx.check(L.gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4(*args, position, *tail))
        got = [host(x, np.uint16) for x in (out2, scales2, kc2, vc2)] + [host(codes2)]
        for name, g, w in zip(("output", "scales", "key cache", "value cache", "codes"), got, want):
            assert np.array_equal(g, w), name


def test_fused_rope_attention_limits(device, gx):
    """Blocks of more tokens or query rows per KV head than the fused kernel keeps are refused
    (GFXI_UNSUPPORTED, the caller runs the three launches); bad arguments fail closed."""
    L = gx.lib()
    assert L.gfxinfer_fused_rope_attention_supported(6, 40, 8, 128) == 1   # 30 rows
    assert L.gfxinfer_fused_rope_attention_supported(7, 40, 8, 128) == 0   # 35 rows
    assert L.gfxinfer_fused_rope_attention_supported(8, 8, 4, 128) == 1    # 16 rows, 8 tokens
    assert L.gfxinfer_fused_rope_attention_supported(9, 8, 8, 128) == 0    # 9 tokens
    assert L.gfxinfer_fused_rope_attention_supported(4, 8, 1, 128) == 1    # 32 rows
    assert L.gfxinfer_fused_rope_attention_supported(4, 8, 1, 256) == 0    # 32 rows > 30
    assert L.gfxinfer_fused_rope_attention_supported(1, 16, 1, 128) == 0   # 16 query heads per KV head
    assert L.gfxinfer_fused_rope_attention_supported(1, 40, 8, 64) == 0
    HQ, HKV, D, cap = 40, 8, 128, 256
    buf = empty((1 << 20,), np.float32)
    p = buf.data_ptr()
    wb = L.gfxinfer_attention_workspace_bytes(8, HQ, D, cap)
    # 5 x 7 = 35 rows > 32
    assert L.gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4(
        p, p, 2 * D, p, p, D, p, 32, np.float32(1e7), None, p, p, p, p, p, p, 0, cap, 7, HQ, HKV, D, p, wb, None
    ) == gx.UNSUPPORTED
    # position + batch beyond the cache
    assert L.gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4(
        p, p, 2 * D, p, p, D, p, 32, np.float32(1e7), None, p, p, p, p, p, p, cap - 2, cap, 3, HQ, HKV, D, p, wb, None
    ) == gx.INVALID_ARGUMENT
    # odd rotary size, null device position
    assert L.gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4(
        p, p, 2 * D, p, p, D, p, 31, np.float32(1e7), None, p, p, p, p, p, p, 0, cap, 3, HQ, HKV, D, p, wb, None
    ) == gx.INVALID_ARGUMENT
    # the table entry's own limits
    assert L.gfxinfer_rope_table_bytes(4096, 64) == 4096 * 32 * 8
    assert L.gfxinfer_rope_table_bytes(4096, 63) == 0
    assert L.gfxinfer_launch_rope_table(None, 4096, 64, np.float32(1e7), None) == gx.INVALID_ARGUMENT
    assert L.gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4_indirect_position(
        p, p, 2 * D, p, p, D, p, 32, np.float32(1e7), None, p, p, p, p, p, p, None, cap, 3, HQ, HKV, D, p, wb, None
    ) == gx.INVALID_ARGUMENT
