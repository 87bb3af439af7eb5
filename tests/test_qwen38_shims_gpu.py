"""The reference's scratch-free launch signatures at its own model's shapes
(qwen_ops.h:101-127, :246-276; attention 24 Q / 4 KV heads x 256, GDN 16 key / 48 value
heads x 128): eager results equal the parameterized launchers bit for bit and the oracle
within the BASELINE bars, the calls are captured into a hipGraph through the C ABI on a
stream whose scratch was bound before the capture, and every replay of the graph equals
the eager results bit for bit (the reference captures these calls the same way,
qwen_runtime.cpp:653-654)."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import dev, empty, host, say

pytestmark = pytest.mark.gpu

HQ, HKV, AD = 24, 4, 256
HK, HV, D = 16, 48, 128
C = 2 * HK * D + HV * D
T, BASE, CAPACITY = 5, 300, 1024


def _half(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def _bf16(x):
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.fixture(scope="module")
def inputs(device):
    rng = np.random.default_rng(3838)
    n = BASE + T - 1
    kc = np.zeros((CAPACITY, HKV, AD), np.uint16)
    vc = np.zeros((CAPACITY, HKV, AD), np.uint16)
    kc[:n] = _half(rng.standard_normal((n, HKV, AD)))
    vc[:n] = _half(rng.standard_normal((n, HKV, AD)))
    host_inputs = dict(
        q=_half(rng.standard_normal((T, HQ, AD))), gate=rng.standard_normal((T, HQ, 2 * AD)).astype(np.float32),
        kc=kc, vc=vc, qkv=_half(rng.standard_normal((T, C))),
        z=rng.standard_normal((T, HV * D)).astype(np.float32), a=rng.standard_normal((T, HV)).astype(np.float32),
        b=rng.standard_normal((T, HV)).astype(np.float32), a_log=_bf16(rng.standard_normal(HV) * 0.5),
        dt=_bf16(rng.standard_normal(HV) * 0.5), nw=_bf16(1 + rng.standard_normal(D) * 0.02),
        s0=(rng.standard_normal((HV, D, D)) * 0.1).astype(np.float32))
    devs = {k: dev(v) for k, v in host_inputs.items()}
    devs["pos"] = dev(np.array([BASE - 1], np.uint64))
    return host_inputs, devs


def _outputs():
    return dict(att=empty((T, HQ, AD), np.uint16), att_ind=empty((T, HQ, AD), np.uint16),
                att1=empty((1, HQ, AD), np.uint16), fin=empty((HV, D, D), np.float32),
                out=empty((T, HV * D), np.uint16), kl=empty((T, HK * D), np.float32),
                dl=empty((T, HV * D), np.float32), yl=empty((T, HV), np.float32),
                state1=empty((HV, D, D), np.float32), out1=empty((1, HV * D), np.uint16))


def _shim_sequence(gx, d, o, stream):
    """One layer's worth of the reference's calls: the GDN window with logs, a one-token
    GDN step in place, block attention (direct and device position) and one-token
    attention, every one through the fixed-shape entries."""
    L = gx.lib()
    gx.check(L.gfxinfer_qwen38_launch_gdn_recurrent_decode_block(
        d["qkv"].data_ptr(), d["z"].data_ptr(), d["a"].data_ptr(), d["b"].data_ptr(), d["a_log"].data_ptr(),
        d["dt"].data_ptr(), d["nw"].data_ptr(), d["s0"].data_ptr(), o["fin"].data_ptr(), o["out"].data_ptr(),
        o["kl"].data_ptr(), o["dl"].data_ptr(), o["yl"].data_ptr(), T, stream))
    o["state1"].copy_(d["s0"])
    gx.check(L.gfxinfer_qwen38_launch_gdn_recurrent_decode(
        d["qkv"].data_ptr(), d["z"].data_ptr(), d["a"].data_ptr(), d["b"].data_ptr(), d["a_log"].data_ptr(),
        d["dt"].data_ptr(), d["nw"].data_ptr(), o["state1"].data_ptr(), o["out1"].data_ptr(), stream))
    args = (d["q"].data_ptr(), d["gate"].data_ptr(), d["kc"].data_ptr(), d["vc"].data_ptr())
    gx.check(L.gfxinfer_qwen38_launch_gated_attention_decode_block(*args, o["att"].data_ptr(), BASE, CAPACITY, T,
                                                                   stream))
    gx.check(L.gfxinfer_qwen38_launch_gated_attention_decode_block_indirect_position(
        *args, o["att_ind"].data_ptr(), d["pos"].data_ptr(), CAPACITY, T, stream))
    gx.check(L.gfxinfer_qwen38_launch_gated_attention_decode(*args, o["att1"].data_ptr(), BASE, CAPACITY, stream))


def test_shims_equal_parameterized_launchers_and_oracle(gx, orc, inputs):
    import torch
    h, d = inputs
    L = gx.lib()
    stream = torch.cuda.Stream()
    nbytes = L.gfxinfer_qwen38_scratch_bytes(T, CAPACITY)
    scratch = empty((nbytes,), np.uint8)
    o = _outputs()
    with torch.cuda.stream(stream):
        s = stream.cuda_stream
        say("qwen38 shims: unbound stream rejected")
        assert L.gfxinfer_qwen38_launch_gated_attention_decode_block(
            d["q"].data_ptr(), d["gate"].data_ptr(), d["kc"].data_ptr(), d["vc"].data_ptr(), o["att"].data_ptr(),
            BASE, CAPACITY, T, s) == gx.INVALID_ARGUMENT
        gx.check(L.gfxinfer_qwen38_bind_scratch(s, scratch.data_ptr(), nbytes, T, CAPACITY))
        say("qwen38 shims: eager sequence")
        _shim_sequence(gx, d, o, s)
        # batch and capacity above the binding's are rejected without a launch
        assert L.gfxinfer_qwen38_launch_gated_attention_decode_block(
            d["q"].data_ptr(), d["gate"].data_ptr(), d["kc"].data_ptr(), d["vc"].data_ptr(), o["att"].data_ptr(),
            BASE, CAPACITY + 1, T, s) == gx.INVALID_ARGUMENT
        assert L.gfxinfer_qwen38_launch_gdn_recurrent_decode_block(
            *(d[k].data_ptr() for k in ("qkv", "z", "a", "b", "a_log", "dt", "nw", "s0")), o["fin"].data_ptr(),
            o["out"].data_ptr(), None, None, None, T + 1, s) == gx.INVALID_ARGUMENT
    stream.synchronize()
    gx.check(L.gfxinfer_qwen38_unbind_scratch(stream.cuda_stream))
    assert L.gfxinfer_qwen38_unbind_scratch(stream.cuda_stream) == gx.INVALID_ARGUMENT

    # the parameterized launchers with a workspace of their own, on the default stream
    wb = L.gfxinfer_attention_workspace_bytes(T, HQ, AD, CAPACITY)
    work = empty((wb // 4,), np.float32)
    att = empty((T, HQ, AD), np.uint16)
    say("qwen38 shims: parameterized attention")
    gx.check(L.gfxinfer_launch_gated_attention_decode_block(
        d["q"].data_ptr(), d["gate"].data_ptr(), d["kc"].data_ptr(), d["vc"].data_ptr(), att.data_ptr(), BASE,
        CAPACITY, T, HQ, HKV, AD, work.data_ptr(), wb, None))
    assert np.array_equal(host(o["att"], np.uint16), host(att, np.uint16))
    assert np.array_equal(host(o["att_ind"], np.uint16), host(att, np.uint16))
    fin, out, mixed = empty((HV, D, D), np.float32), empty((T, HV * D), np.uint16), empty((T, HV * D), np.float32)
    say("qwen38 shims: parameterized GDN")
    gx.check(L.gfxinfer_launch_gdn_recurrent_decode_block(
        *(d[k].data_ptr() for k in ("qkv", "z", "a", "b", "a_log", "dt", "nw", "s0")), fin.data_ptr(),
        out.data_ptr(), None, None, None, T, HK, HV, D, mixed.data_ptr(), None))
    assert np.array_equal(host(o["fin"]), host(fin))
    assert np.array_equal(host(o["out"], np.uint16), host(out, np.uint16))

    # the oracle (BASELINE bars: attention 1e-2, GDN state fp32 1e-5)
    want = np.empty((T, HQ, AD), np.uint16)
    orc.lib().orc_gated_attention(orc.ptr(h["q"]), orc.ptr(h["gate"]), orc.ptr(h["kc"]), orc.ptr(h["vc"]),
                                  orc.ptr(want), BASE, T, HQ, HKV, AD, np.float32(1 / np.sqrt(AD)))
    got = host(o["att"], np.uint16).view(np.float16).astype(np.float32)
    w = want.view(np.float16).astype(np.float32)
    assert np.abs(got - w).max() <= 1e-2 * max(1.0, np.abs(w).max())
    want_s = np.empty_like(h["s0"])
    want_o = np.empty((T, HV * D), np.uint16)
    orc.lib().orc_gdn_recurrent(*(orc.ptr(h[k]) for k in ("qkv", "z", "a", "b", "a_log", "dt", "nw", "s0")),
                                orc.ptr(want_s), orc.ptr(want_o), None, None, None, T, HK, HV, D)
    assert np.abs(host(o["fin"]) - want_s).max() <= 1e-5 * max(1.0, np.abs(want_s).max())
    want_1 = np.empty_like(h["s0"])
    orc.lib().orc_gdn_recurrent(*(orc.ptr(h[k]) for k in ("qkv", "z", "a", "b", "a_log", "dt", "nw", "s0")),
                                orc.ptr(want_1), orc.ptr(np.empty((1, HV * D), np.uint16)), None, None, None, 1,
                                HK, HV, D)
    assert np.abs(host(o["state1"]) - want_1).max() <= 1e-5 * max(1.0, np.abs(want_1).max())


def test_shim_sequence_captured_in_a_graph_replays_bit_identically(gx, inputs):
    import torch
    _, d = inputs
    L = gx.lib()
    stream = torch.cuda.Stream()
    nbytes = L.gfxinfer_qwen38_scratch_bytes(T, CAPACITY)
    scratch = empty((nbytes,), np.uint8)
    gx.check(L.gfxinfer_qwen38_bind_scratch(stream.cuda_stream, scratch.data_ptr(), nbytes, T, CAPACITY))
    try:
        eager = _outputs()
        say("qwen38 shims: eager before capture")
        with torch.cuda.stream(stream):
            _shim_sequence(gx, d, eager, stream.cuda_stream)
        stream.synchronize()
        want = {k: host(v) for k, v in eager.items()}
        captured = _outputs()
        graph = torch.cuda.CUDAGraph()
        say("qwen38 shims: capture")
        with torch.cuda.graph(graph, stream=stream):
            _shim_sequence(gx, d, captured, stream.cuda_stream)
        for replay in range(3):
            for v in captured.values():
                v.zero_()                      # eager work between replays
            torch.cuda.synchronize()
            say("qwen38 shims: replay", replay)
            graph.replay()
            torch.cuda.synchronize()
            for k, v in captured.items():
                assert np.array_equal(host(v), want[k]), (replay, k)
    finally:
        torch.cuda.synchronize()
        gx.check(L.gfxinfer_qwen38_unbind_scratch(stream.cuda_stream))
