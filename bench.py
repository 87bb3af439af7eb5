"""Benchmark of the gfx950 speculative-verify hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline (BASELINE.json metric, config 2): W3A4 GEMV [17408, 5120] at batch 5.
One step = quantize the fp16 activations to A4 + the W3A4 GEMM, exactly the unit
the reference times (src/cli/main.cpp:1381-1445).  Weights are synthetic
N(0, 0.02) quantized on the device with the reference W3G128 rules, replicated
into 16 distinct buffers (557 MB) that the steps rotate through so the 256 MB
Infinity Cache cannot serve repeats; steps are replayed from a hipGraph.

value = algorithmic bytes per step / step time (GB/s).  Algorithmic bytes are
every compulsory byte once: N*K*3/8 codes + N*K/128*2 scales + B*K/2 activation
codes + B*K/128*2 activation scales + B*N*4 output.
roofline: the GEMM kernel alone, timed with HIP events on its stream.
cpu_baseline: the CPU restatement of the reference quantize + dequant-GEMV
(W3A8) on the host cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "W3A4 verify GEMM GB/s (% HBM peak) + verified tok/s at k=4..31, 27B shapes"


def algorithmic_bytes(rows, cols, batch, wbits=3, abits=4):
    return (rows * cols * wbits // 8 + rows * (cols // 128) * 2 + batch * cols * abits // 8
            + batch * (cols // 128) * 2 + batch * rows * 4)


def gemv_bench(steps, warmup, rows=17408, cols=5120, batch=5, copies=16, windows=5):
    """The headline step, timed exactly: `warmup` untimed steps, then `windows` timing
    windows of exactly `steps` steps each (HIP events on the launch stream around graph
    replays); the median window is reported.  Step i uses weight copy i % copies."""
    import numpy as np
    import torch
    import gfxinfer_amd as gx

    device = torch.device("cuda:0")
    fmt = gx.W3G128
    torch.manual_seed(0x5EED)
    w = torch.randn(rows, cols, device=device, dtype=torch.float32) * 0.02
    codes0 = torch.empty(gx.tile_bytes(fmt, rows, cols), dtype=torch.uint8, device=device)
    scales0 = torch.empty(rows * cols // 128, dtype=torch.int16, device=device)
    gx.launch_quantize_group128(fmt, w, rows, cols, codes0, scales0)
    del w
    codes = [codes0] + [codes0.clone() for _ in range(copies - 1)]
    scales = [scales0] + [scales0.clone() for _ in range(copies - 1)]
    x = (torch.randn(batch, cols, device=device) * 1.0).to(torch.float16)
    acodes = torch.empty(batch, cols // 2, dtype=torch.uint8, device=device)
    ascales = torch.empty(batch, cols // 128, dtype=torch.int16, device=device)
    y = torch.empty(batch, rows, dtype=torch.float32, device=device)
    torch.cuda.synchronize()

    stream = torch.cuda.Stream()

    def step(i, s):
        gx.launch_quantize_activation_i4(x, acodes, ascales, cols, batch, stream=s)
        gx.launch_i4_gemm(fmt, codes[i % copies], scales[i % copies], acodes, ascales, y, rows, cols, batch, stream=s)

    def gemm_only(i, s):
        gx.launch_i4_gemm(fmt, codes[i % copies], scales[i % copies], acodes, ascales, y, rows, cols, batch, stream=s)

    def capture(fn, n):
        """Graph of steps 0 .. n-1 (n a multiple of `copies` keeps the rotation aligned)."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            for i in range(min(n, copies)):  # warm the kernels outside capture
                fn(i, stream)
            stream.synchronize()
            with torch.cuda.graph(g, stream=stream):
                for i in range(n):
                    fn(i, stream)
        return g

    # `steps` = full * chunk + rest: `full` replays of a chunk graph plus one remainder graph.
    chunk = min(steps, 32 * copies) // copies * copies or steps
    full, rest = divmod(steps, chunk)

    def runner(fn):
        main = capture(fn, chunk)
        tail = capture(fn, rest) if rest else None

        def run_steps(n_full, with_tail):
            for _ in range(n_full):
                main.replay()
            if with_tail and tail is not None:
                tail.replay()
        return run_steps

    def timed(fn):
        run_steps = runner(fn)
        with torch.cuda.stream(stream):
            wfull, wrest = divmod(warmup, chunk)
            run_steps(wfull, False)
            if wrest:  # the warmup's remainder as eager steps
                for i in range(wrest):
                    fn(i, stream)
            torch.cuda.synchronize()
            results = []
            for _ in range(windows):
                start = torch.cuda.Event(enable_timing=True)
                stop = torch.cuda.Event(enable_timing=True)
                start.record(stream)
                run_steps(full, True)
                stop.record(stream)
                stop.synchronize()
                results.append(start.elapsed_time(stop) / steps)  # ms per step
            torch.cuda.synchronize()
        return float(np.median(results)), results

    ms_step, step_windows = timed(step)
    ms_gemm, gemm_windows = timed(gemm_only)
    return dict(ms_step=ms_step, ms_gemm=ms_gemm, steps=steps, warmup=warmup, windows=windows,
                step_windows_ms=[round(v, 6) for v in step_windows],
                gemm_windows_ms=[round(v, 6) for v in gemm_windows],
                rows=rows, cols=cols, batch=batch, copies=copies,
                weight_bytes=sum(c.numel() for c in codes) + 2 * sum(s.numel() for s in scales))


def verify_gemm_bench(batches=(5, 16, 32), budget=640e6, reps=20):
    """one dense decoder block's projection set in W3A4 (q/k/v from
    hidden 5120 with 40 Q / 8 KV heads x 128 -- q the gated query + gate rows, 2 x 40 x 128
    = 10240, as the verifier's q_proj --, o, SwiGLU MLP 5120 -> 17408 -> 5120) at
    k + 1 = 5, 16, 32 rows, launched the way the verifier launches them (q/k/v and
    gate/up fused into one grid each, o and down as split-K planes), and the W4 LM head
    [151936, 5120] with the fused greedy argmax.  Each launch is timed alone under graph
    replay over rotating weight copies: every projection gets enough copies that one
    pass over them reads about `budget` bytes, beyond the 256 MB Infinity Cache, as the
    verifier's pass over the whole model does.  One JSON line per (projection, rows)."""
    import ctypes
    import torch
    import gfxinfer_amd as gx

    H, I, V = 5120, 17408, 151936
    w3, w4 = gx.W3G128, gx.W4G128

    def matrix(fmt, rows, cols, n):
        w = torch.randn(rows, cols, device="cuda") * 0.02
        c0 = torch.empty(gx.tile_bytes(fmt, rows, cols), dtype=torch.uint8, device="cuda")
        s0 = torch.empty(rows * cols // 128, dtype=torch.int16, device="cuda")
        gx.launch_quantize_group128(fmt, w, rows, cols, c0, s0)
        del w
        return [(c0, s0)] + [(c0.clone(), s0.clone()) for _ in range(n - 1)]

    torch.manual_seed(0x5EED)
    mats = {"q": (w3, 2 * H, H), "k": (w3, 1024, H), "v": (w3, 1024, H), "o": (w3, H, H),
            "gate": (w3, I, H), "up": (w3, I, H), "down": (w3, H, I)}
    groups = {"qkv": ("q", "k", "v"), "o": ("o",), "gate_up": ("gate", "up"), "down": ("down",)}
    copies = {}
    for label, names in groups.items():
        case_bytes = sum(algorithmic_bytes(mats[m][1], mats[m][2], 1) for m in names)
        for m in names:
            copies[m] = max(4, math.ceil(budget / case_bytes))
    weights = {name: matrix(f, r, c, copies[name]) for name, (f, r, c) in mats.items()}
    head = matrix(w4, V, H, 1)[0]
    out = []
    stream = torch.cuda.Stream()
    for batch in batches:
        acts = {}
        for cols in (H, I):
            x = torch.randn(batch, cols, device="cuda").half()
            a = torch.empty(batch, cols // 2, dtype=torch.uint8, device="cuda")
            sa = torch.empty(batch, cols // 128, dtype=torch.int16, device="cuda")
            gx.launch_quantize_activation_i4(x, a, sa, cols, batch)
            acts[cols] = (a, sa)
        ys = {name: torch.empty(8, batch, r, device="cuda") for name, (_, r, _) in mats.items()}
        keys_bytes = int(gx.lib().gfxinfer_gemm_argmax_workspace_bytes(V, batch))
        keys = torch.empty(keys_bytes, dtype=torch.uint8, device="cuda")
        tokens = torch.empty(batch, dtype=torch.int32, device="cuda")

        def fused(names, i, s):
            a, sa = acts[H]
            gx.launch_i4_gemm_fused(w3, [(weights[n][i][0], weights[n][i][1], ys[n], mats[n][1]) for n in names],
                                    a, sa, H, batch, stream=s)

        def split(name, i, s):
            f, r, c = mats[name]
            a, sa = acts[c]
            gx.launch_i4_gemm_split(f, weights[name][i][0], weights[name][i][1], a, sa, ys[name], r, c, batch,
                                    gx.gemm_split_count(r, c, batch), stream=s)

        def lm_head(i, s):
            a, sa = acts[H]
            gx.check(gx.lib().gfxinfer_launch_gfx950_i4_gemm_argmax(
                w4, head[0].data_ptr(), head[1].data_ptr(), a.data_ptr(), sa.data_ptr(), None, V, H, batch,
                V, None, keys.data_ptr(), keys_bytes, tokens.data_ptr(), ctypes.c_void_p(s.cuda_stream)))

        cases = [("qkv", ("q", "k", "v"), lambda i, s: fused(("q", "k", "v"), i, s)),
                 ("o", ("o",), lambda i, s: split("o", i, s)),
                 ("gate_up", ("gate", "up"), lambda i, s: fused(("gate", "up"), i, s)),
                 ("down", ("down",), lambda i, s: split("down", i, s)),
                 ("lm_head_argmax", None, lm_head)]
        for label, names, fn in cases:
            n = copies[names[0]] if names is not None else 1
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(stream):
                for i in range(n):
                    fn(i, stream)
                stream.synchronize()
                with torch.cuda.graph(g, stream=stream):
                    for i in range(n):
                        fn(i, stream)
                for _ in range(3):
                    g.replay()
                torch.cuda.synchronize()
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    g.replay()
                e1.record(stream)
                e1.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * n)
            if names is None:
                nbytes = algorithmic_bytes(V, H, batch, wbits=4)
            else:
                nbytes = sum(algorithmic_bytes(mats[m][1], mats[m][2], batch) for m in names)
            line = {"verify_gemm": label, "rows": batch, "us": round(us, 3), "bytes": nbytes,
                    "gbs": round(nbytes / us / 1e3, 1), "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
            out.append(line)
            print(json.dumps(line), flush=True)
    return out


def _graph_time(stream, fn, n, reps):
    """Average microseconds of fn(i) for i in 0..n-1, captured once and replayed reps times."""
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for i in range(n):
            fn(i)
        stream.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n):
                fn(i)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * n)


def gemv_table_bench(reps=40, budget=600e6):
    """W3A4 and W4A4 GEMV on [17408, 5120] (up/gate) and
    [5120, 17408] (down) at batch 1 and 5, the plain product over rotating weight copies
    (about 600 MB, beyond the 256 MB Infinity Cache), plus the down shape as the
    verifier launches it (split-K planes).  One JSON line per case; bit-exact int32
    partials of the same kernels are checked by tests/test_gemm_gpu.py."""
    import torch
    import gfxinfer_amd as gx

    torch.manual_seed(0x6E7)
    stream = torch.cuda.Stream()
    out = []
    for fmt, wbits in ((gx.W3G128, 3), (gx.W4G128, 4)):
        for rows, cols in ((17408, 5120), (5120, 17408)):
            w = torch.randn(rows, cols, device="cuda") * 0.02
            c0 = torch.empty(gx.tile_bytes(fmt, rows, cols), dtype=torch.uint8, device="cuda")
            s0 = torch.empty(rows * cols // 128, dtype=torch.int16, device="cuda")
            gx.launch_quantize_group128(fmt, w, rows, cols, c0, s0)
            del w
            n = max(2, int(budget // c0.numel()))
            weights = [(c0, s0)] + [(c0.clone(), s0.clone()) for _ in range(n - 1)]
            for batch in (1, 5):
                x = torch.randn(batch, cols, device="cuda").half()
                a = torch.empty(batch, cols // 2, dtype=torch.uint8, device="cuda")
                sa = torch.empty(batch, cols // 128, dtype=torch.int16, device="cuda")
                gx.launch_quantize_activation_i4(x, a, sa, cols, batch)
                splits = gx.gemm_split_count(rows, cols, batch)
                y = torch.empty(splits, batch, rows, device="cuda")
                cases = [("plain", 1)] + ([("split", splits)] if splits > 1 else [])
                for mode, sp in cases:
                    if sp == 1:
                        def fn(i):
                            gx.launch_i4_gemm(fmt, weights[i][0], weights[i][1], a, sa, y, rows, cols, batch,
                                              stream=stream)
                    else:
                        def fn(i):
                            gx.launch_i4_gemm_split(fmt, weights[i][0], weights[i][1], a, sa, y, rows, cols, batch,
                                                    sp, stream=stream)
                    us = _graph_time(stream, fn, n, reps)
                    nbytes = algorithmic_bytes(rows, cols, batch, wbits=wbits) + (sp - 1) * batch * rows * 4
                    line = {"gemv": f"W{wbits}A4", "rows": rows, "columns": cols, "batch": batch, "mode": mode,
                            "splits": sp, "us": round(us, 3), "bytes": nbytes, "gbs": round(nbytes / us / 1e3, 1),
                            "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
                    out.append(line)
                    print(json.dumps(line), flush=True)
            del weights
    return out


def gemm_family_bench(reps=40, budget=600e6, batches=(1, 2, 3, 4, 5, 8), headline=False):
    """The two A4 GEMM kernel families side by side (v_mfma_i32_16x16x64_i8 against
    v_dot8_i32_i4) at 1-8 tokens on the config-2 shapes, the down shape as split-K planes
    and the MTP draft head (W4 [98304, 5120]), over rotating weight copies beyond the
    Infinity Cache.  One JSON line per (shape, batch, family); the families' outputs are
    bit-identical (tests/test_gemm_dot_gpu.py)."""
    import torch
    import gfxinfer_amd as gx

    torch.manual_seed(0x6E8)
    stream = torch.cuda.Stream()
    out = []
    shapes = ((gx.W3G128, 3, 17408, 5120), (gx.W4G128, 4, 17408, 5120), (gx.W3G128, 3, 5120, 17408),
              (gx.W4G128, 4, 5120, 17408), (gx.W4G128, 4, 98304, 5120))
    if headline:  # the profiled subset: the headline shape at 1 and 5 tokens
        shapes, batches = shapes[:1], (1, 5)
    for fmt, wbits, rows, cols in shapes:
        w = torch.randn(rows, cols, device="cuda") * 0.02
        c0 = torch.empty(gx.tile_bytes(fmt, rows, cols), dtype=torch.uint8, device="cuda")
        s0 = torch.empty(rows * cols // 128, dtype=torch.int16, device="cuda")
        gx.launch_quantize_group128(fmt, w, rows, cols, c0, s0)
        del w
        n = max(2, int(budget // c0.numel()))
        weights = [(c0, s0)] + [(c0.clone(), s0.clone()) for _ in range(n - 1)]
        for batch in batches:
            x = torch.randn(batch, cols, device="cuda").half()
            a = torch.empty(batch, cols // 2, dtype=torch.uint8, device="cuda")
            sa = torch.empty(batch, cols // 128, dtype=torch.int16, device="cuda")
            gx.launch_quantize_activation_i4(x, a, sa, cols, batch)
            splits = gx.gemm_split_count(rows, cols, batch)
            y = torch.empty(splits, batch, rows, device="cuda")
            for sp in sorted({1, splits}):
                for family, name in ((gx.GEMM_MFMA, "mfma"), (gx.GEMM_DOT, "dot")):
                    def fn(i, family=family, sp=sp):
                        gx.check(gx.debug_gemm_family(family, fmt, weights[i][0], weights[i][1], a, sa, rows,
                                                      cols, batch, out=y, splits=sp, stream=stream))
                    us = _graph_time(stream, fn, n, reps)
                    nbytes = algorithmic_bytes(rows, cols, batch, wbits=wbits) + (sp - 1) * batch * rows * 4
                    line = {"gemm_family": name, "format": f"W{wbits}A4", "rows": rows, "columns": cols,
                            "batch": batch, "splits": sp, "us": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
                            "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
                    out.append(line)
                    print(json.dumps(line), flush=True)
        del weights
    return out


def attention_bench(reps=50, contexts=(400, 4064)):
    """Gated GQA decode attention with the A4 quantizer of the o projection
    (split + combine launches) at the verifier's block sizes, for both head shapes, at a
    short and a 4 K context: microseconds per call from HIP events around graph replays,
    and the K/V bytes it reads (every visible position of every KV head, fp16)."""
    import torch
    import gfxinfer_amd as gx

    L = gx.lib()
    stream = torch.cuda.Stream()
    capacity = 4096 + 32
    out = []
    for hq, hkv, d in ((40, 8, 128), (24, 4, 256)):
        kc = (torch.randn(capacity, hkv, d, device="cuda") * 0.5).half()
        vc = (torch.randn(capacity, hkv, d, device="cuda") * 0.5).half()
        for t in (1, 5, 32):
            q = torch.randn(t, hq, d, device="cuda").half()
            gate = torch.randn(t, hq, 2 * d, device="cuda")
            o = torch.empty(t, hq, d, device="cuda").half()
            codes = torch.empty(t, hq * d // 2, dtype=torch.uint8, device="cuda")
            scales = torch.empty(t, hq * d // 128, dtype=torch.int16, device="cuda")
            wb = L.gfxinfer_attention_workspace_bytes(t, hq, d, capacity)
            work = torch.empty(wb // 4, device="cuda")
            for base in contexts:
                def fn(_i, base=base):
                    gx.check(L.gfxinfer_launch_gated_attention_decode_block_quantize_i4(
                        q.data_ptr(), gate.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(),
                        codes.data_ptr(), scales.data_ptr(), base, capacity, t, hq, hkv, d, work.data_ptr(), wb,
                        stream.cuda_stream))
                us = _graph_time(stream, fn, 8, reps)
                kv = (base + t - 1) * hkv * d * 2 * 2
                line = {"attention": f"{hq}/{hkv}x{d}", "tokens": t, "positions": base + t - 1, "us": round(us, 3),
                        "kv_bytes": kv, "gbs": round(kv / us / 1e3, 1)}
                out.append(line)
                print(json.dumps(line), flush=True)
    return out


def read_floor_bench(reps=20, budget=640e6, total=1280 << 20):
    """Yardstick for the GEMV roofline: one launch of a plain streaming read of the
    headline GEMV's algorithmic bytes, half and twice that, and the LM head's size,
    rotating over copies (about 640 MB, beyond the 256 MB Infinity Cache).  Two read
    shapes: the grid-stride loop (gfxinfer_debug_stream_read) over launch widths, and
    the one-shot read (gfxinfer_debug_stream_read_oneshot: every load of a lane issued
    at once, non-temporal) over loads per lane.  One JSON line per case and one per
    size and shape with the fastest case."""
    import math
    import torch
    import gfxinfer_amd as gx

    stream = torch.cuda.Stream()
    data = torch.randint(0, 2**31 - 1, (total // 4,), dtype=torch.int32, device="cuda")
    widths = (1024, 1088, 2048, 4096, 8192)  # 1088: the headline GEMV's workgroup count
    headline = algorithmic_bytes(17408, 5120, 5)
    sizes = (headline // 2, headline, 2 * headline, 423624704)
    # grid-stride: one entry per lane; one-shot: one entry per 16-byte piece
    sink = torch.zeros(max(max(widths) * 256, max(sizes) // 16), dtype=torch.int32, device="cuda")
    out = []
    for nbytes in sizes:
        nbytes -= nbytes % 16
        slot = (nbytes + 255) // 256 * 256
        copies = max(1, min(total // slot, math.ceil(budget / slot)))
        best = None
        for width in widths:
            def fn(i, width=width):
                gx.debug_stream_read(data.data_ptr() + (i % copies) * slot, nbytes, sink, width, stream=stream)
            us = _graph_time(stream, fn, max(copies, 16) // copies * copies, reps)
            line = {"read_floor": nbytes, "shape": "grid-stride", "workgroups": width, "copies": copies,
                    "us": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
                    "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
            print(json.dumps(line), flush=True)
            if best is None or us < best["us"]:
                best = line
        out.append(dict(best, best=True))
        print(json.dumps(out[-1]), flush=True)
        best = None
        for loads in (1, 2, 4, 8):
            def fn(i, loads=loads):
                gx.debug_stream_read_oneshot(data.data_ptr() + (i % copies) * slot, nbytes, sink, loads,
                                             stream=stream)
            us = _graph_time(stream, fn, max(copies, 16) // copies * copies, reps)
            line = {"read_floor": nbytes, "shape": "one-shot", "loads_per_lane": loads,
                    "workgroups": -(-nbytes // (4096 * loads)), "copies": copies, "us": round(us, 3),
                    "gbs": round(nbytes / us / 1e3, 1), "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
            print(json.dumps(line), flush=True)
            if best is None or us < best["us"]:
                best = line
        out.append(dict(best, best=True))
        print(json.dumps(out[-1]), flush=True)
    return out


def gdn_window_bench(tokens=32, layers=48, reps=20, seed=2026, value_heads=32):
    """the GDN verify window at 27B shapes (32 value heads x 128 x 128
    fp32 state, 16 key heads x 128) over `tokens` tokens with every per-token log the
    rollback needs (conv inputs, normalized keys, deltas, decays), for `layers` layers'
    own buffers, then the prefix restore of all layers to a seeded accepted length drawn
    uniformly from [0, tokens].  Inputs follow the config: projected q/k/v ~ N(0, 1),
    a, b ~ N(0, 1) (decay = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b)).
    value_heads=48 times the reference model's GDN (qwen38_spec.h:26-29).
    Correctness of both launches: tests/test_ops_gpu.py, tests/test_runtime_gpu.py."""
    import numpy as np
    import torch
    import gfxinfer_amd as gx

    HK, HV, D, T = 16, value_heads, 128, tokens
    C = 2 * HK * D + HV * D
    L = gx.lib()
    torch.manual_seed(seed)
    accepted = int(np.random.default_rng(seed).integers(0, T + 1))
    f32 = dict(device="cuda", dtype=torch.float32)
    proj = [torch.randn(T, C, **f32) for _ in range(layers)]
    conv_w = (torch.randn(C, 4, **f32) * 0.5).to(torch.bfloat16)
    a = torch.randn(T, HV, **f32)
    b = torch.randn(T, HV, **f32)
    a_log = (torch.randn(HV, **f32) * 0.5).to(torch.bfloat16)
    dt_bias = (torch.randn(HV, **f32) * 0.5).to(torch.bfloat16)
    conv_states = torch.randn(layers, C, 4, **f32).half()
    conv_final = torch.empty_like(conv_states)
    states = torch.randn(layers, HV, D, D, **f32) * 0.1
    states_final = torch.empty_like(states)
    mixed = torch.empty(T, HV * D, **f32)
    conv_log = torch.empty(layers, T, C, device="cuda", dtype=torch.float16)
    key_log = torch.empty(layers, T, HK * D, **f32)
    delta_log = torch.empty(layers, T, HV * D, **f32)
    decay_log = torch.empty(layers, T, HV, **f32)
    stream = torch.cuda.Stream()
    p = lambda t: t.data_ptr()  # noqa: E731

    def window(i):
        gx.check(L.gfxinfer_launch_gdn_conv_window(
            p(proj[i]), p(conv_w), p(conv_states[i]), p(conv_final[i]), p(conv_log[i]), p(a), p(b), p(a_log),
            p(dt_bias), p(states[i]), p(states_final[i]), p(mixed), p(key_log[i]), p(delta_log[i]),
            p(decay_log[i]), T, HK, HV, D, stream.cuda_stream))

    def restore(_):
        gx.check(L.gfxinfer_launch_gdn_restore_prefix_all(
            p(conv_states), p(states), p(conv_log), p(key_log), p(delta_log), p(decay_log), C, layers, T,
            accepted, HK, HV, D, stream.cuda_stream))

    window_us = _graph_time(stream, window, layers, reps)
    restore_us = _graph_time(stream, restore, 1, reps)
    state = HV * D * D * 4
    window_bytes = (2 * state + T * C * 4 + T * HV * 8 + T * HV * D * 4 + C * 4 * 2 * 2
                    + T * (C * 2 + HK * D * 4 + HV * D * 4 + HV * 4))
    restore_bytes = layers * (2 * state + C * 4 * 2 * 2 + accepted * (C * 2 + HK * D * 4 + HV * D * 4 + HV * 4))
    lines = [{"gdn": "conv_window", "tokens": T, "value_heads": HV, "us_per_layer": round(window_us, 3),
              "bytes": window_bytes,
              "gbs": round(window_bytes / window_us / 1e3, 1)},
             {"gdn": "restore_prefix_all", "value_heads": HV, "layers": layers, "accepted": accepted,
              "us": round(restore_us, 3),
              "bytes": restore_bytes, "gbs": round(restore_bytes / restore_us / 1e3, 1),
              "frac_hbm": round(restore_bytes / restore_us / 1e3 / HBM_PEAK_GBS, 4)}]
    for line in lines:
        print(json.dumps(line), flush=True)
    return lines


def _forced_acceptance(rng, depth):
    """Seeded Bernoulli(0.85) per draft; accepted = index of the first failure."""
    trials = rng.random(depth) < 0.85
    return int(depth if trials.all() else int(trials.argmin()))


def _matrix_bytes(model, names):
    total = 0
    for name in names:
        v = model.find_tensor(name)
        total += int(v.data_bytes) + int(v.auxiliary_bytes)
    return total


def verify_bench(depths=(4, 31), rounds=60, warmup=8, seed=2026, reference_rates=True, shape="27b",
                 long_context=3584):
    """Full synthetic 27B-shaped model: hipGraph-captured MTP chain +
    64-layer verifier of depth D, forced seeded 85 % Bernoulli acceptance, rollback or
    state swap per round.  Emitted tok/s = sum(accepted + 1) / time, verified tok/s =
    sum(D + 1) / time (the reference's evaluated target tokens).  shape "27b": the
    BASELINE configs' heads (40/8 x 128 attention, 16/32 GDN, vocabulary 151936);
    "reference": the reference's own model (qwen38_spec.h:16-34: 24/4 x 256 attention,
    16/48 GDN, vocabulary 248320), same widths, depth and formats otherwise.  The rounds
    run in a 4096-token context from its start (positions below ~450), and again
    (`depth_D_from_P` entries) after a chunked prefill of `long_context` seeded tokens, so
    that attention reads the keys and values of ~3.6-4.1 K positions."""
    import numpy as np
    from gfxinfer_amd.runtime import QwenDecodeSession, SyntheticModel, qwen38_27b_spec, qwen38_reference_spec

    spec = qwen38_reference_spec() if shape == "reference" else qwen38_27b_spec()
    t0 = time.perf_counter()
    model = SyntheticModel(spec, seed)
    create_s = time.perf_counter() - t0
    names = [t for t in _tensor_names(spec)]
    mtp = [n for n in names if n.startswith("mtp.")]
    verifier = [n for n in names if not n.startswith("mtp.") and "embed_tokens" not in n]
    head = model.find_tensor("lm_head.weight")
    head_bytes = int(head.data_bytes) + int(head.auxiliary_bytes)
    verifier_bytes = _matrix_bytes(model, verifier)
    proposal_bytes = _matrix_bytes(model, mtp) + head_bytes * spec.mtp_draft_vocabulary // spec.vocabulary_size
    results = {}
    try:
        for depth in depths:
            session = QwenDecodeSession(model, 4096, depth + 1)
            rng = np.random.default_rng(seed + depth)
            token = session.greedy_step(1)
            for _ in range(warmup):
                token = session.speculative_step_forced(token, depth, _forced_acceptance(rng, depth)).tokens[-1]
            emitted = verified = 0
            n = min(rounds, (4096 - session.position()) // (depth + 1) - 1)
            t0 = time.perf_counter()
            for _ in range(n):
                r = session.speculative_step_forced(token, depth, _forced_acceptance(rng, depth))
                emitted += len(r.tokens)
                verified += depth + 1
                token = r.tokens[-1]
            elapsed = time.perf_counter() - t0
            session.close()
            round_bytes = verifier_bytes + depth * proposal_bytes
            results[f"depth_{depth}"] = {
                "rounds": n,
                "ms_per_round": round(elapsed / n * 1e3, 4),
                "emitted_tok_s": round(emitted / elapsed, 2),
                "verified_tok_s": round(verified / elapsed, 2),
                "acceptance": round((emitted - n) / (n * depth), 4),
                "weight_bytes_per_round": round_bytes,
                "weight_gbs": round(round_bytes * n / elapsed / 1e9, 1),
                "weight_frac_of_hbm_peak": round(round_bytes * n / elapsed / 1e9 / HBM_PEAK_GBS, 4),
            }
            if long_context:
                session = QwenDecodeSession(model, 4096, depth + 1)
                prompt = rng.integers(0, spec.tokenizer_vocabulary_size, long_context)
                token = session.prefill([int(t) for t in prompt])
                for _ in range(2):
                    token = session.speculative_step_forced(token, depth, _forced_acceptance(rng, depth)).tokens[-1]
                start = session.position()
                emitted = verified = 0
                n = min(rounds, (4096 - start) // (depth + 1) - 1)
                t0 = time.perf_counter()
                for _ in range(n):
                    r = session.speculative_step_forced(token, depth, _forced_acceptance(rng, depth))
                    emitted += len(r.tokens)
                    verified += depth + 1
                    token = r.tokens[-1]
                elapsed = time.perf_counter() - t0
                end = session.position()
                session.close()
                results[f"depth_{depth}_from_{long_context}"] = {
                    "rounds": n, "positions": [start, end],
                    "ms_per_round": round(elapsed / n * 1e3, 4),
                    "emitted_tok_s": round(emitted / elapsed, 2),
                    "verified_tok_s": round(verified / elapsed, 2),
                }
        if reference_rates:
            results.update(reference_bench_rates(model, spec))
    finally:
        model.close()
    return {"model": {"shape": shape, "attention_heads": spec.attention_head_count, "kv_heads": spec.kv_head_count,
                      "head_size": spec.attention_head_size, "gdn_key_heads": spec.gdn_key_head_count,
                      "gdn_value_heads": spec.gdn_value_head_count, "vocabulary": spec.vocabulary_size},
            "model_weight_bytes": verifier_bytes + proposal_bytes, "create_s": round(create_s, 3),
            "verifier_weight_bytes": verifier_bytes, "proposal_weight_bytes": proposal_bytes,
            **results}


def reference_bench_rates(model, spec, block_sizes=(5, 32), blocks=12, mtp_steps=40):
    """The reference's own verifier-only and proposal-only rates, measured the way its CLI
    measures them on the same session API:
    - block-bench (cli/main.cpp:846-915): block_step over B tokens, each block's outputs
      feeding the next, wall clock per call; tokens/s = blocks * B / total time;
    - mtp-bench (cli/main.cpp:1140-1207): greedy_step and mtp_draft alternating; target
      and MTP-draft steps/s = calls / time spent in each."""
    from gfxinfer_amd.runtime import QwenDecodeSession
    out = {}
    for batch in block_sizes:
        session = QwenDecodeSession(model, 4096, 0)
        try:
            inputs = [(1 + i) % spec.tokenizer_vocabulary_size for i in range(batch)]
            inputs = session.block_step(inputs)  # warm-up block (kernels, caches)
            total = 0.0
            for _ in range(blocks):
                t0 = time.perf_counter()
                inputs = session.block_step(inputs)
                total += time.perf_counter() - t0
        finally:
            session.close()
        out[f"block_step_{batch}"] = {"blocks": blocks, "ms_per_block": round(total / blocks * 1e3, 4),
                                      "evaluated_tok_s": round(blocks * batch / total, 2)}
    session = QwenDecodeSession(model, 4096, 0)
    try:
        target_s = draft_s = 0.0
        token = session.greedy_step(1)
        candidate = session.mtp_draft(token)
        for _ in range(mtp_steps):
            t0 = time.perf_counter()
            token = session.greedy_step(token)
            t1 = time.perf_counter()
            candidate = session.mtp_draft(token)
            t2 = time.perf_counter()
            target_s += t1 - t0
            draft_s += t2 - t1
    finally:
        session.close()
    out["mtp_bench"] = {"steps": mtp_steps, "target_steps_s": round(mtp_steps / target_s, 2),
                        "mtp_draft_steps_s": round(mtp_steps / draft_s, 2)}
    del candidate
    return out


def prefill_bench(prompt_tokens=512, serial_tokens=64, seed=2026, context=4096):
    """Chunked prefill against the reference's serial prefill loop on the synthetic
    27B-shaped model: time to the first generated token for a `prompt_tokens` prompt
    with the MTP cache kept in step (gfxinfer_session_prefill, 32-token verifier blocks
    + batched MTP cache update), and the per-token rate of the loop the reference CLI
    runs (greedy_step + mtp_draft per prompt token, cli/main.cpp:1055-1069), timed over
    `serial_tokens` tokens.  Both leave the same state (tests/test_prefill_generate_gpu.py)."""
    import numpy as np
    import torch
    from gfxinfer_amd.runtime import QwenDecodeSession, SyntheticModel, qwen38_27b_spec

    spec = qwen38_27b_spec()
    model = SyntheticModel(spec, seed)
    prompt = np.random.default_rng(seed).integers(0, spec.tokenizer_vocabulary_size, prompt_tokens)
    prompt = [int(t) for t in prompt]
    try:
        chunked = QwenDecodeSession(model, context, 0)
        chunked.prefill(prompt[:64])  # warm-up of the block kernels
        chunked.close()
        chunked = QwenDecodeSession(model, context, 0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        chunked.prefill(prompt)
        chunked_s = time.perf_counter() - t0
        chunked.close()
        serial = QwenDecodeSession(model, context, 0)
        serial.greedy_step(prompt[0])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in prompt[1:1 + serial_tokens]:
            serial.mtp_draft(t)
            serial.greedy_step(t)
        serial_s = time.perf_counter() - t0
        serial.close()
    finally:
        model.close()
    line = {"prefill": "chunked", "prompt_tokens": prompt_tokens, "seconds": round(chunked_s, 4),
            "tok_s": round(prompt_tokens / chunked_s, 1),
            "serial_tok_s": round(serial_tokens / serial_s, 1),
            "speedup": round((prompt_tokens / chunked_s) / (serial_tokens / serial_s), 2)}
    print(json.dumps(line), flush=True)
    return line


def _tensor_names(spec):
    """Matrix and vector names of the synthetic checkpoint (converter naming)."""
    names = ["lm_head.weight", "model.language_model.norm.weight"]
    for i in range(spec.layer_count):
        p = f"model.language_model.layers.{i}."
        names += [p + s for s in ("input_layernorm.weight", "post_attention_layernorm.weight",
                                  "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")]
        if (i + 1) % spec.full_attention_interval == 0:
            names += [p + "self_attn." + s for s in ("q_proj.weight", "k_proj.weight", "v_proj.weight",
                                                     "o_proj.weight", "q_norm.weight", "k_norm.weight")]
        else:
            names += [p + "linear_attn." + s for s in ("in_proj_qkv.weight", "in_proj_z.weight",
                                                       "in_proj_a.weight", "in_proj_b.weight",
                                                       "conv1d.weight", "A_log", "dt_bias", "norm.weight",
                                                       "out_proj.weight")]
    names += ["mtp.fc.weight", "mtp.pre_fc_norm_embedding.weight", "mtp.pre_fc_norm_hidden.weight",
              "mtp.norm.weight"]
    p = "mtp.layers.0."
    names += [p + s for s in ("input_layernorm.weight", "post_attention_layernorm.weight",
                              "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")]
    names += [p + "self_attn." + s for s in ("q_proj.weight", "k_proj.weight", "v_proj.weight",
                                             "o_proj.weight", "q_norm.weight", "k_norm.weight")]
    return names


def cpu_baseline(rows=17408, cols=5120, seconds=10.0):
    """Oracle W3A8 quantize + dequant-dot GEMV on host cores: the
    GEMV repeats for about `seconds` of CPU time and the median run is reported."""
    import tempfile
    import numpy as np
    from oracle import oracle as O

    build_dir = tempfile.mkdtemp(prefix="gfxi_cpu_baseline_")
    try:
        flags = O.use_native_build(build_dir)
    except (OSError, subprocess.CalledProcessError) as e:  # no compiler: the prebuilt -O2 oracle
        flags = f"prebuilt oracle/liboracle.so (-O2; native build failed: {e})"
    rng = np.random.default_rng(0x5EED0001)
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    x16 = rng.standard_normal((1, cols)).astype(np.float16).view(np.uint16)
    tq = []
    for _ in range(2):
        t0 = time.perf_counter()
        _, codes, scales = O.quantize_group128(w, O.W3)
        tq.append(time.perf_counter() - t0)
    a, as16 = O.quantize_activation_i8(x16)
    O.dequant_dot_gemv_packed(codes, O.W3, scales, a, as16, rows, cols)  # warmup
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < seconds or len(times) < 5:
        t0 = time.perf_counter()
        O.dequant_dot_gemv_packed(codes, O.W3, scales, a, as16, rows, cols)
        times.append(time.perf_counter() - t0)
    repeats = len(times)
    gemv = sorted(times)[len(times) // 2]
    nbytes = algorithmic_bytes(rows, cols, 1, wbits=3, abits=8)
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(nbytes / gemv / 1e9, 3),
        "unit": "GB/s",
        "cores": O.max_threads(),
        "kind": "port",
        "sample": (f"BASELINE config 1: W3G128 [{rows},{cols}] x A8 batch 1 dequant-dot GEMV, median of "
                   f"{repeats} runs = {gemv * 1e3:.1f} ms over {nbytes} algorithmic bytes; "
                   f"quantize_group128 of the same matrix {min(tq):.2f} s; CPU {model}, "
                   f"nproc {os.cpu_count()}; oracle/oracle.c built with {flags}, OpenMP over rows"),
    }


PROFILE = os.path.join(ROOT, "profiles", "gemv_w3a4_17408x5120_b5.txt")
COPY_BYTES = 256 << 20


def pmc_probe(launches=8, rows=17408, cols=5120, batch=5):
    """Workload for the rocprofv3 --pmc passes: one device copy of COPY_BYTES (the
    calibration kernel: it reads and writes exactly COPY_BYTES) and `launches` plain
    launches of the headline GEMM on distinct weight buffers."""
    import torch
    import gfxinfer_amd as gx
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    fmt = gx.W3G128
    w = torch.randn(rows, cols, device="cuda") * 0.02
    codes = [torch.empty(gx.tile_bytes(fmt, rows, cols), dtype=torch.uint8, device="cuda") for _ in range(launches)]
    scales = [torch.empty(rows * cols // 128, dtype=torch.int16, device="cuda") for _ in range(launches)]
    for c, s in zip(codes, scales):
        gx.launch_quantize_group128(fmt, w, rows, cols, c, s)
    x = torch.randn(batch, cols, device="cuda").half()
    a = torch.empty(batch, cols // 2, dtype=torch.uint8, device="cuda")
    sa = torch.empty(batch, cols // 128, dtype=torch.int16, device="cuda")
    y = torch.empty(batch, rows, device="cuda")
    gx.launch_quantize_activation_i4(x, a, sa, cols, batch)
    torch.cuda.synchronize()
    for c, s in zip(codes, scales):
        gx.launch_i4_gemm(fmt, c, s, a, sa, y, rows, cols, batch)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "gemm_launches": launches,
                      "gemm_algorithmic_bytes": algorithmic_bytes(rows, cols, batch)}))


def headline_kernel_digest():
    """SHA-256 (first 16 hex digits) of the headline kernel's source: lowbit_gemv.hip from
    its operand expansion through lowbit_gemm_kernel, plus common.hpp.  A committed
    profile records the digest of the source it measured, so a changed kernel shows up
    as a stale profile instead of passing its old counters on."""
    import hashlib
    csrc = os.path.join(ROOT, "gfxinfer_amd", "csrc")
    text = open(os.path.join(csrc, "lowbit_gemv.hip")).read()
    begin, end = text.index("// Operand expansion."), text.index("// Direct-operand GEMM.")
    digest = hashlib.sha256(text[begin:end].encode())
    digest.update(open(os.path.join(csrc, "common.hpp"), "rb").read())
    return digest.hexdigest()[:16]


def committed_profile():
    """The headline kernel's committed rocprofv3 summary: its file, average dispatch
    duration (kernel trace) and HBM bytes per launch (FETCH_SIZE + WRITE_SIZE passes,
    calibrated), or None where the summary lacks them.  When the kernel source no longer
    has the digest the summary records, the traffic figure is withheld (None) and the
    summary is marked stale."""
    out = {"file": os.path.relpath(PROFILE, ROOT), "kernel_us": None, "traffic": None}
    recorded = None
    try:
        for line in open(PROFILE):
            if line.startswith("traffic_bytes_per_launch"):
                out["traffic"] = int(line.split("=")[1].split()[0])
            elif line.startswith("kernel_avg_us"):
                out["kernel_us"] = float(line.split("=")[1].split()[0])
            elif line.startswith("tree"):
                out["tree"] = line.split("=", 1)[1].strip()
            elif line.startswith("kernel_source_sha256"):
                recorded = line.split("=", 1)[1].strip()
    except (OSError, ValueError, IndexError):
        pass
    out["kernel_source_sha256"] = headline_kernel_digest()
    out["source_matches"] = recorded == out["kernel_source_sha256"]
    if not out["source_matches"]:
        out["stale"] = "the kernel source differs from the one the summary measured: traffic withheld"
        out["traffic"] = None
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-verify", action="store_true")
    ap.add_argument("--verify-rounds", type=int, default=60)
    ap.add_argument("--no-reference-rates", action="store_true",
                    help="skip the verifier-only block_step and proposal-only rates (a round profile "
                         "then ends with the last round)")
    ap.add_argument("--verify-model", choices=("27b", "reference"), default="27b",
                    help="verify-round model heads: the BASELINE 27B shape or the reference's own model")
    ap.add_argument("--long-context", type=int, default=3584,
                    help="prefill length before the long-context verify rounds (0: skip them)")
    ap.add_argument("--verify-depths", default="4,8,16,31",
                    help="comma-separated MTP depths of the verify-round measurement")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run the rocprofv3 --pmc workload (calibration copy + plain GEMM launches)")
    ap.add_argument("--probe-rows", type=int, default=17408, help="--pmc-probe GEMM rows")
    ap.add_argument("--probe-batch", type=int, default=5, help="--pmc-probe GEMM tokens")
    ap.add_argument("--verify-gemms", action="store_true",
                    help="time BASELINE config 3 (one block's projections + LM head argmax at 5/16/32 rows)")
    ap.add_argument("--gemv-table", action="store_true",
                    help="time BASELINE config 2 (W3A4/W4A4 GEMV, up and down shapes, batch 1 and 5)")
    ap.add_argument("--gemm-families", nargs="?", const="all", choices=("all", "headline"),
                    help="time the MFMA and v_dot8 A4 GEMM kernel families at 1-8 tokens side by side "
                         "(headline: W3A4 [17408,5120] at 1 and 5 tokens only)")
    ap.add_argument("--attention", action="store_true",
                    help="time gated decode attention (+A4) at 1/5/32 tokens, short and 4 K contexts")
    ap.add_argument("--attention-context", type=int, default=0,
                    help="--attention at this one context (visible positions of the first token) only")
    ap.add_argument("--prefill", action="store_true",
                    help="time chunked prefill against the reference's serial prefill loop (27B shapes)")
    ap.add_argument("--read-floor", action="store_true",
                    help="time a plain streaming read of the GEMV's bytes (what one launch can reach)")
    ap.add_argument("--gdn-window", action="store_true",
                    help="time BASELINE config 4 (32-token GDN window with logs + restore to a seeded length)")
    ap.add_argument("--gdn-tokens", type=int, default=32, help="--gdn-window tokens per window")
    ap.add_argument("--gdn-value-heads", type=int, default=32,
                    help="--gdn-window value heads (32: the BASELINE config; 48: the reference model)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's path runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration)", file=sys.stderr)
        sys.exit(2)
    import gfxinfer_amd as gx
    gx.check(gx.lib().gfxinfer_require_gfx950_device(0))
    if args.pmc_probe:
        pmc_probe(rows=args.probe_rows, batch=args.probe_batch)
        return
    if args.verify_gemms:
        verify_gemm_bench()
        return
    if args.gemv_table:
        gemv_table_bench()
        return
    if args.attention:
        attention_bench(contexts=(args.attention_context,) if args.attention_context else (400, 4064))
        return
    if args.gemm_families:
        gemm_family_bench(headline=args.gemm_families == "headline")
        return
    if args.gdn_window:
        gdn_window_bench(tokens=args.gdn_tokens, value_heads=args.gdn_value_heads)
        return
    if args.read_floor:
        read_floor_bench()
        return
    if args.prefill:
        prefill_bench()
        return

    r = gemv_bench(args.steps, args.warmup)
    profile = committed_profile()
    nbytes = algorithmic_bytes(r["rows"], r["cols"], r["batch"])
    step_gbs = nbytes / (r["ms_step"] * 1e-3) / 1e9
    gemm_gbs = nbytes / (r["ms_gemm"] * 1e-3) / 1e9
    codes_only = r["rows"] * r["cols"] * 3 // 8
    out = {
        "metric": METRIC,
        "value": round(step_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": r["warmup"],
        "ms_per_step": round(r["ms_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": (f"W3A4 GEMV [{r['rows']},{r['cols']}] batch {r['batch']}: A4 quantize + "
                         f"W3A4 int8-MFMA GEMM, {r['copies']} rotating weight copies "
                         f"({r['weight_bytes'] / 1e6:.0f} MB), hipGraph replay"),
            "rows": r["rows"], "columns": r["cols"], "batch": r["batch"],
            "weights": "W3G128 (fp16 scales)", "activations": "A4G128",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gemm_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gemm_gbs / HBM_PEAK_GBS, 4),
            "traffic": profile["traffic"],
            "kernel": "lowbit_gemm_kernel<W3,A4,GP=2>",
            "kernel_us": round(r["ms_gemm"] * 1e3, 3),
            "algorithmic_bytes": nbytes,
            "timing": (f"median of {r['windows']} windows of exactly {r['steps']} launches after "
                       f"{r['warmup']} warmup launches, HIP events on the launch stream around "
                       "graph replays (includes the gap between consecutive dispatches)"),
            "profile": profile,
        },
        "step_windows_ms": r["step_windows_ms"],
        "gemm_windows_ms": r["gemm_windows_ms"],
        "reference_packed_gbps": round(codes_only / (r["ms_step"] * 1e-3) / 1e9, 2),
    }
    if profile["kernel_us"]:
        agree = abs(profile["kernel_us"] - r["ms_gemm"] * 1e3) / profile["kernel_us"]
        out["roofline"]["profile"]["frac"] = round(nbytes / profile["kernel_us"] / 1e3 / HBM_PEAK_GBS, 4)
        out["roofline"]["profile"]["events_vs_profile"] = round(agree, 4)
        if agree > 0.05:
            out["roofline"]["profile"]["why_they_differ"] = (
                "rocprofv3 times each dispatch from its first wave to its end; the events here time "
                "back-to-back graph launches, so they also hold the dispatch gap between launches")
    if not args.no_verify:
        depths = tuple(int(d) for d in args.verify_depths.split(",") if d)
        out["verify"] = verify_bench(depths=depths, rounds=args.verify_rounds,
                                     reference_rates=not args.no_reference_rates, shape=args.verify_model,
                                     long_context=args.long_context)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
