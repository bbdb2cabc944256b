#!/usr/bin/env python3
"""Heron train-step throughput on one MI355X (BASELINE.json metric).

Workload (config 4): one full Heron train step's GPU work, D=512, L=12,
T=2048, vocab 8192, F=2048, batch 1, rosa_grad = stop_grad_bits, with the
suffix-automaton output synthesised as Bernoulli(0.5) indices (+-e). Inputs
are resident in HBM before the timed region; a step is UllisHeron::
train_step_on from token ids: the embedding gather, ullis_hip_heron_step
(forward, head + streamed CE, backward, every parameter update) and the
embedding scatter-SGD (HeronTrainer.step_tokens). The timed
region is bracketed by stream synchronisation; HIP events on the library's
stream give the step time.

Prints ONE JSON line. `roofline` is for the launch that dominates the step
(the value backward pair) and `roofline_packed` for the dominant packed +-1
launch (the key backward pair), which the metric names. Each is timed over
its own passes of the same number of steps right after the reported ones
(ullis_hip_heron_probe): `avg_us` from every workgroup's start / end on the
device wall clock (earliest start to latest end), which does not perturb the
step; `rocprof_avg_us` is the rocprofv3 kernel-trace average of the same
launches from the committed profile, whose dispatch interval is ~2.4 us
longer. The probe passes are kept out of the reported steps.
`cpu_baseline` times the CPU oracle (a port of the reference's CPU backend)
single-threaded on windows of 256 tokens at full widths and depth (three
runs in child processes started before the GPU is touched; the median),
scaled per token.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

CONFIG = dict(d_model=512, n_layers=12, dim_ffn=2048, vocab=8192, batch=1, time=2048)
LR = 0.01
NO_IGNORE = 0xFFFFFFFF
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2516.6  # dense fp16 MFMA, MI355X

# HBM bytes per launch of the probed kernel, from two rocprofv3 --pmc passes
# (FETCH_SIZE, WRITE_SIZE; KiB per dispatch) over this script with
# --copy-mib 256, scaled by what the same counters read for the 256 MiB copy
# kernel (FETCH_SIZE reads half the bytes copied: x2.0; WRITE_SIZE x1.0).
# Summary: profiles/value_backward_hbm_traffic.txt. Re-measure when the kernel changes.
TRAFFIC_BYTES = {
    "value_backward": (21661.5 * 2.0 + 12294.0 * 1.0) * 1024,
}

# rocprofv3 kernel-trace average of the same launches in the timed pass of
# `rocprofv3 --kernel-trace --stats -- python3 bench.py --steps 20 --warmup 3
# --cpu-rows 0` (profiles/heron_step_kernel_trace.txt). The dispatch interval
# it reports also holds the ramp of the first workgroups and the end-of-kernel
# cache writeback (about 2.4 us a launch here), which the stamps cannot see,
# and the profiler slows the step. Re-measure when the kernels change.
ROCPROF_AVG_US = {"value_backward": 23.73, "key_backward": 22.15}

# Launch classes with a roofline object in the bench line: the step's dominant
# launch (the value backward pair, fp16) and its dominant packed +-1 launch
# (the key backward pair), which BASELINE.json's metric names.
ROOFLINE_PROBES = (("roofline", "value_backward"), ("roofline_packed", "key_backward"))


def cpu_sample(rows: int) -> None:
    """One oracle train step (config 4's widths and depth, a window of `rows`
    tokens), single-threaded; prints its wall time as JSON. Run as a child
    process of bench.py, started before bench.py touches the GPU."""
    from oracle import cpu_ref as o
    from ullis_amd.synth import heron_arena, step_inputs

    c = CONFIG
    dims = o.HeronDims(c["d_model"], c["n_layers"], c["dim_ffn"], c["vocab"])
    lay, total = o.heron_layout(dims)
    arena = heron_arena(lay, total, dims, seed=7)
    x, labels, idx = step_inputs(rows, c["d_model"], c["vocab"], c["n_layers"], 1, rows, seed=7)
    t0 = time.perf_counter()
    o.heron_train_step(dims, arena, x, labels, NO_IGNORE, 1, rows, LR, idx, want_qkv=True)
    print(json.dumps({"rows": rows, "seconds": time.perf_counter() - t0}), flush=True)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(rows: int, runs: int) -> dict:
    """The oracle's heron step (a port of the reference's CPU backend) timed on
    `runs` windows of `rows` tokens, each single-threaded in its own child
    process (run side by side), median of the runs, scaled per token."""
    import subprocess

    py = [sys.executable, os.path.abspath(__file__), "--cpu-sample", str(rows)]
    procs = [subprocess.Popen(py, stdout=subprocess.PIPE, text=True) for _ in range(runs)]
    secs = []
    for pr in procs:
        out, _ = pr.communicate()
        if pr.returncode != 0:
            raise RuntimeError("cpu sample failed")
        secs.append(json.loads(out.strip().splitlines()[-1])["seconds"])
    med = float(np.median(secs))
    return {
        "value": round(rows / med, 2),
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"oracle/cpu_ref.c heron step D512 L12 F2048 V8192 (full widths and depth) on "
                   f"a window of T={rows} tokens, single-threaded; median of {runs} runs "
                   f"({', '.join(f'{t:.1f}' for t in sorted(secs))} s), each in its own process, "
                   f"run side by side; host: {os.cpu_count()} logical CPUs, {cpu_model()}. "
                   "Tokens/s scales linearly in T for every op except the per-weight SGD, which "
                   "this window charges to fewer tokens than a T=2048 step"),
        "host_cpus": os.cpu_count(),
        "host_cpu_model": cpu_model(),
        "run_seconds": [round(t, 2) for t in secs],
    }


# Few-row forward products of a T = 1 greedy decode at batch 1 and 8 (the
# GEMV pass of the stress profile, config 5, and the same layers at config 4):
# (label, kind, out, in). Weight bytes per launch: out*in/8 for sign bits,
# 2*out*in for the fp16 CMix value.
DECODE_GEMV = [
    ("cfg5 head", "packed", 32768, 1024), ("cfg5 cmix key", "packed", 4096, 1024),
    ("cfg5 rosa q/k/v/o", "packed", 1024, 1024), ("cfg5 cmix value", "fp16", 1024, 4096),
    ("cfg4 head", "packed", 8192, 512), ("cfg4 cmix key", "packed", 2048, 512),
    ("cfg4 rosa q/k/v/o", "packed", 512, 512), ("cfg4 cmix value", "fp16", 512, 2048),
]


def decode_gemv(rt, reps: int) -> None:
    """One JSON line per decode product: kernel time of one launch (its own
    start / end timestamps, ullis_hip_time_next_launch), averaged over reps,
    and the weight bytes it streams against the HBM peak."""
    import ctypes as C

    lib, ctx = rt.lib, rt.ctx
    rng = np.random.default_rng(5)
    for label, kind, out_f, in_f in DECODE_GEMV:
        if kind == "packed":
            w = rt.put(rng.integers(0, 2 ** 32, out_f * in_f // 32, dtype=np.uint32))
            scale = rt.put(np.full(out_f, 0.02, np.float16).view(np.uint16))
            bias = rt.put(np.zeros(out_f, np.float16).view(np.uint16))
            wbytes = out_f * in_f / 8
        else:
            w = rt.put(rng.normal(0, 0.02, out_f * in_f).astype(np.float16).view(np.uint16))
            wbytes = 2.0 * out_f * in_f
        for m in (1, 8):
            x = rt.put(rng.standard_normal(m * in_f).astype(np.float16).view(np.uint16))
            y = rt.buffer(4 * m * out_f)

            def call():
                if kind == "packed":
                    return lib.ullis_hip_binary_linear(ctx, x.ptr, 1, w.ptr, scale.ptr, bias.ptr, m,
                                                       in_f, out_f, y.ptr, None)
                return lib.ullis_hip_fp16_linear(ctx, x.ptr, 1, w.ptr, m, in_f, out_f, y.ptr, None)

            total = 0.0
            for i in range(reps + 3):
                rt._check(lib.ullis_hip_time_next_launch(ctx, 2, 3), "arm")
                rt._check(call(), label)
                ms = C.c_float()
                rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 2, 3, C.byref(ms)), "elapsed")
                if i >= 3:
                    total += ms.value
            us = total / reps * 1e3
            gbs = wbytes / (us * 1e-6) / 1e9
            print(json.dumps({"decode_gemv": label, "kind": kind, "rows": m, "out": out_f,
                              "in": in_f, "avg_us": round(us, 2), "weight_bytes": int(wbytes),
                              "achieved_gbs": round(gbs, 1),
                              "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}), flush=True)


# LayerNorm launches timed alone (no other stream sharing the CUs): config 4's
# [2048, 512] and config 5's [32768, 1024] activations.
LN_ISOLATED = ((2048, 512), (32768, 1024))


def layer_norm_isolated(rt, reps: int) -> None:
    """One JSON line per LayerNorm launch and shape: the row kernel's own time
    (ullis_hip_time_next_launch, averaged over reps), its algorithmic HBM bytes
    (fp32 x in, fp16 y out forward; fp32 x, gy in and fp32 gx out backward)
    against the HBM peak, and a device copy of the same bytes (read + write)
    timed back to back with events as the floor a launch of that size meets.
    Launches cycle over enough buffer sets (>= 512 MiB) that their operands
    come from HBM, not from the 256 MB last-level cache."""
    import ctypes as C

    lib, ctx = rt.lib, rt.ctx
    rng = np.random.default_rng(3)
    for rows, ch in LN_ISOLATED:
        n = rows * ch
        nsets = max(2, -(-(512 << 20) // (14 * n)))
        w = rt.put(np.ones(ch, np.float16).view(np.uint16))
        b = rt.put(np.zeros(ch, np.float16).view(np.uint16))
        gw, gb = rt.buffer(4 * ch), rt.buffer(4 * ch)
        xs = [rt.put(rng.standard_normal(n).astype(np.float32)) for _ in range(nsets)]
        gys = [rt.put(rng.standard_normal(n).astype(np.float32)) for _ in range(nsets)]
        y16s = [rt.buffer(2 * n) for _ in range(nsets)]
        gxs = [rt.buffer(4 * n) for _ in range(nsets)]
        # copy-floor operands: up to the backward's 6n bytes each way
        srcs = [rt.buffer(6 * n) for _ in range(nsets)]
        dsts = [rt.buffer(6 * n) for _ in range(nsets)]

        def fwd(k):
            return lib.ullis_hip_layer_norm(ctx, xs[k].ptr, w.ptr, b.ptr, rows, ch, None,
                                            y16s[k].ptr)

        def bwd(k):
            return lib.ullis_hip_layer_norm_backward(ctx, xs[k].ptr, gys[k].ptr, w.ptr, rows, ch,
                                                     gxs[k].ptr, gw.ptr, gb.ptr)

        for name, nbytes, call in (("ln_forward", 6.0 * n, fwd),
                                   ("ln_backward_rows", 12.0 * n, bwd)):
            total = 0.0
            for i in range(reps + 3):
                rt._check(lib.ullis_hip_time_next_launch(ctx, 2, 3), "arm")
                rt._check(call(i % nsets), name)
                ms = C.c_float()
                rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 2, 3, C.byref(ms)), "elapsed")
                if i >= 3:
                    total += ms.value
            us = total / reps * 1e3
            # the same bytes moved by a device copy (half read, half written)
            half = int(nbytes // 2) // 16 * 16
            assert half <= 6 * n
            for k in range(3):
                rt._check(lib.ullis_hip_copy(ctx, dsts[k % nsets].ptr, srcs[k % nsets].ptr, half),
                          "copy")
            rt.sync()
            rt._check(lib.ullis_hip_event_record(ctx, 0), "event")
            for k in range(reps):
                rt._check(lib.ullis_hip_copy(ctx, dsts[k % nsets].ptr, srcs[k % nsets].ptr, half),
                          "copy")
            rt._check(lib.ullis_hip_event_record(ctx, 1), "event")
            rt.sync()
            ms = C.c_float()
            rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 0, 1, C.byref(ms)), "elapsed")
            copy_us = ms.value / reps * 1e3
            gbs = nbytes / (us * 1e-6) / 1e9
            print(json.dumps({"layer_norm": name, "rows": rows, "ch": ch, "avg_us": round(us, 2),
                              "algorithmic_bytes": int(nbytes), "achieved_gbs": round(gbs, 1),
                              "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "buffer_sets": nsets,
                              "same_bytes_copy_us": round(copy_us, 2),
                              "copy_gbs": round(2 * half / (copy_us * 1e-6) / 1e9, 1)}),
                  flush=True)
        del xs, gys, y16s, gxs, srcs, dsts


# Config 5, the stress profile of the MFMA path (a parity-test case, not the
# bench line): D=1024, L=24, T=4096, batch 8, vocab 32768, key 1024->4096.
STRESS = dict(d_model=1024, n_layers=24, dim_ffn=4096, vocab=32768, batch=8, time=4096)
STRESS_PROBES = ("value_backward", "key_backward", "o_backward", "key_forward",
                 "value_forward", "head_ce")


def stress_profile(rt, steps: int, warmup: int) -> None:
    """One JSON line: the config-5 train step (from token ids) and, from one
    probe pass per launch class, each class's MFMA rate at these shapes."""
    import ctypes as C
    from ullis_amd.runtime import HeronShape, HeronTrainer
    from ullis_amd.synth import heron_arena, step_inputs

    c = STRESS
    shape = HeronShape(**c)
    tr = HeronTrainer(rt, shape)
    tr.upload_arena(heron_arena(tr.layout, tr.arena_bytes, shape.dims(), seed=7))
    _, labels, idx = step_inputs(shape.rows, c["d_model"], c["vocab"], c["n_layers"], c["batch"],
                                 c["time"], seed=7)
    rng = np.random.default_rng(7)
    nd = shape.rows * c["d_model"]
    table = rt.put(rng.standard_normal(c["vocab"] * c["d_model"]).astype(np.float16).view(np.uint16))
    table_res = rt.zeros(np.float32, c["vocab"] * c["d_model"])
    tok = rt.put(rng.integers(0, c["vocab"], shape.rows).astype(np.uint32))
    dl, di = rt.put(labels), rt.put(idx)
    xe, g = rt.zeros(np.float32, nd), rt.zeros(np.float32, nd)
    st = rt.zeros(np.float32, 4)
    lib, ctx = rt.lib, rt.ctx

    def run(n):
        rt.sync()
        rt._check(lib.ullis_hip_event_record(ctx, 0), "event")
        for _ in range(n):
            tr.step_tokens(table, table_res, tok, dl, NO_IGNORE, LR, di, xe, g, stats=st)
        rt._check(lib.ullis_hip_event_record(ctx, 1), "event")
        rt.sync()
        ms = C.c_float()
        rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 0, 1, C.byref(ms)), "elapsed")
        return ms.value

    for _ in range(warmup):
        run(1)
    ms = run(steps) / steps
    # per layer: Q/K/V/O forward + O backward (6 D^2), key and value forward +
    # backward (6 D F); head: logits, recompute, backward (3 D V); 2 flops/MAC
    d, f = c["d_model"], c["dim_ffn"]
    flops = 2.0 * shape.rows * (c["n_layers"] * 6 * d * (d + f) + 3 * d * c["vocab"])
    kernels = {}
    for name in STRESS_PROBES:
        tr.probe_begin(name)
        run(1)
        k = tr.probe_end(name)
        if k["count"]:
            avg_s = k["total_ms"] / k["count"] / 1e3
            tf = k["work"] / avg_s / 1e12
            kernels[name] = {"kernel": k["name"], "avg_us": round(avg_s * 1e6, 1),
                             "achieved_tflops": round(tf, 1),
                             "frac": round(tf / FP16_PEAK_TFLOPS, 4), "launches": k["count"]}
    print(json.dumps({
        "stress": "config 5: heron D1024 L24 F4096 V32768 T4096 B8, stop_grad_bits, lr 0.01",
        "ms_per_step": round(ms, 2), "tokens_per_s": round(shape.rows / (ms / 1e3), 1),
        "algorithmic_tflop_per_step": round(flops / 1e12, 2),
        "achieved_tflops": round(flops / (ms / 1e3) / 1e12, 1),
        "loss_last_step": round(float(st.download(np.float32, 4)[0]), 5),
        "kernels": kernels}), flush=True)
    tr.close()


def rosa_live(rt, steps: int, warmup: int) -> None:
    """One JSON line: config 4's step with the suffix automaton driven live
    (ullis_hip_heron_step_sam: every layer's Q/K/V planes to the host, the
    indices back) against the same step with all layers' indices given up
    front. The host-side automaton here returns the same precomputed indices
    at once, so the difference is the hand-off itself: the copies, the host
    synchronisation per layer, and the Q/K/V branch moved onto the residual
    chain."""
    import ctypes as C
    from ullis_amd.runtime import HeronShape, HeronTrainer
    from ullis_amd.synth import heron_arena, step_inputs

    c = CONFIG
    shape = HeronShape(**c)
    tr = HeronTrainer(rt, shape)
    tr.upload_arena(heron_arena(tr.layout, tr.arena_bytes, shape.dims(), seed=7))
    x, labels, idx = step_inputs(shape.rows, c["d_model"], c["vocab"], c["n_layers"], c["batch"],
                                 c["time"], seed=7)
    nd = shape.rows * c["d_model"]
    dx, dl, di = rt.put(x), rt.put(labels), rt.put(idx)
    g = rt.zeros(np.float32, nd)
    idx_l = [np.ascontiguousarray(idx[l * nd:(l + 1) * nd]) for l in range(c["n_layers"])]
    lib, ctx = rt.lib, rt.ctx

    def run(live, n):
        rt.sync()
        rt._check(lib.ullis_hip_event_record(ctx, 0), "event")
        t0 = time.perf_counter()
        for _ in range(n):
            if live:
                tr.step_sam(lambda layer, planes: idx_l[layer], dx, dl, NO_IGNORE, LR, g)
            else:
                tr.step(dx, dl, NO_IGNORE, LR, di, g)
        rt._check(lib.ullis_hip_event_record(ctx, 1), "event")
        rt.sync()
        wall = time.perf_counter() - t0
        ms = C.c_float()
        rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 0, 1, C.byref(ms)), "elapsed")
        return ms.value / n, wall * 1e3 / n

    for live in (False, True):
        run(live, warmup)
    fused_ms, fused_wall = run(False, steps)
    live_ms, live_wall = run(True, steps)
    print(json.dumps({
        "rosa_live": "config 4 (D512 L12 T2048): automaton indices handed over per layer",
        "fused_ms_per_step": round(fused_ms, 4), "live_ms_per_step": round(live_ms, 4),
        "live_wall_ms_per_step": round(live_wall, 4),
        "handoff_us_per_layer": round((live_ms - fused_ms) * 1e3 / c["n_layers"], 2),
        "steps": steps}), flush=True)
    tr.close()


DECODE_CONFIGS = [
    ("config 4", dict(d_model=512, n_layers=12, dim_ffn=2048, vocab=8192)),
    ("config 5", dict(d_model=1024, n_layers=24, dim_ffn=4096, vocab=32768)),
]


def decode_weight_bytes(d: int, layers: int, ffn: int, vocab: int) -> int:
    """Bytes one T = 1 decode step must read at least: every layer's sign bits
    (Q/K/V/O d x d, key ffn x d), fp16 value weights (d x ffn), fp16 row scales
    and biases, mixes, e and LayerNorm parameters, then the head's bits, scale
    and bias. Activations (a few KiB) are left out."""
    per_layer = (4 * d * d + ffn * d) // 8 + 2 * ffn * d + 2 * (4 * 2 * d + ffn) + 2 * 8 * d
    return layers * per_layer + vocab * d // 8 + 2 * 2 * vocab + 2 * 2 * d


def decode_step_bench(rt, steps: int, warmup: int, graph: bool = True) -> None:
    """One JSON line per (config, batch): the T = 1 decode step
    (ullis_hip_heron_decode_step) with the automaton's indices given, timed by
    events on the library's stream over `steps` tokens, and the same with the
    indices handed over per layer through the host callback. The floor is the
    step's weight bytes at the HBM peak."""
    import ctypes as C
    from ullis_amd.runtime import HeronShape, HeronTrainer
    from ullis_amd.synth import heron_arena

    lib, ctx = rt.lib, rt.ctx
    for name, dims in DECODE_CONFIGS:
        shape = HeronShape(**dims, batch=1, time=2)
        tr = HeronTrainer(rt, shape)
        tr.upload_arena(heron_arena(tr.layout, tr.arena_bytes, shape.dims(), seed=7))
        d, L, V = dims["d_model"], dims["n_layers"], dims["vocab"]
        rng = np.random.default_rng(7)
        table = rt.put(rng.standard_normal(V * d).astype(np.float16).view(np.uint16))
        wbytes = decode_weight_bytes(d, L, dims["dim_ffn"], V)
        for batch in (1, 8):
            tokens = rt.put(rng.integers(0, V, batch).astype(np.uint32))
            idx_h = (rng.random(L * batch * d) < 0.5).astype(np.uint8)
            idx = rt.put(idx_h)
            idx_l = idx_h.reshape(L, batch, d)
            logits = rt.zeros(np.float32, batch * V)
            nxt = rt.zeros(np.uint32, batch)
            tr.decode_init(batch, graph=graph)

            def run(n, live):
                rt.sync()
                rt._check(lib.ullis_hip_event_record(ctx, 0), "event")
                t0 = time.perf_counter()
                for _ in range(n):
                    if live:
                        tr.decode_step(table, tokens, logits, next_tokens=nxt,
                                       sam=lambda layer, planes: idx_l[layer])
                    else:
                        tr.decode_step(table, tokens, logits, next_tokens=nxt, rosa_idx=idx)
                rt._check(lib.ullis_hip_event_record(ctx, 1), "event")
                rt.sync()
                wall = time.perf_counter() - t0
                ms = C.c_float()
                rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 0, 1, C.byref(ms)), "elapsed")
                return ms.value * 1e3 / n, wall * 1e6 / n

            run(warmup, False)
            us, wall_us = run(steps, False)
            run(warmup, True)
            live_us, _ = run(steps, True)
            floor_us = wbytes / (HBM_PEAK_GBS * 1e9) * 1e6
            print(json.dumps({
                "decode_step": f"{name}: D{d} L{L} F{dims['dim_ffn']} V{V}", "batch": batch,
                "us_per_step": round(us, 2), "wall_us_per_step": round(wall_us, 2),
                "tokens_per_s": round(batch / (us * 1e-6), 1),
                "weight_bytes": wbytes, "hbm_floor_us": round(floor_us, 2),
                "frac_of_floor": round(floor_us / us, 4),
                "live_us_per_step": round(live_us, 2), "graph": graph, "steps": steps}),
                  flush=True)
        tr.close()


VENDOR_SHAPES = [
    (2048, 2048, 512, "key fwd / value dX"), (2048, 512, 2048, "value fwd / key dX"),
    (512, 2048, 2048, "value dW / key dW"), (2048, 512, 512, "O fwd / dX"),
    (2048, 8192, 512, "head logits"), (2048, 512, 8192, "head dX"), (8192, 512, 2048, "head dW"),
    (32768, 4096, 1024, "config-5 key fwd"), (32768, 1024, 4096, "config-5 value fwd"),
]


def vendor_gemm(shapes=None) -> None:
    """One JSON line per heron GEMM shape: the vendor fp16 GEMM (torch.matmul,
    hipBLASLt) on dense fp16 operands, 20 (4 at config 5) launches captured in a
    graph and replayed 20 times between events, so host launch cost is out of
    the figure. A yardstick for the products here, which read sign bits and
    run epilogues; nothing in the library uses it."""
    import torch

    dev = torch.device("cuda:0")
    for m, n, k, name in shapes or VENDOR_SHAPES:
        a = torch.randn(m, k, device=dev, dtype=torch.float16)
        b = torch.randn(k, n, device=dev, dtype=torch.float16)
        c = torch.empty(m, n, device=dev, dtype=torch.float16)
        reps = 20 if m * n * k < 1e10 else 4
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            for _ in range(3):
                torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            for _ in range(reps):
                torch.matmul(a, b, out=c)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(20):
            g.replay()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / (20 * reps)
        tf = 2.0 * m * n * k / (us * 1e-6) / 1e12
        print(json.dumps({"vendor_gemm": name, "shape_MNK": [m, n, k], "us": round(us, 2),
                          "tflops": round(tf, 1), "frac": round(tf / FP16_PEAK_TFLOPS, 4)}),
              flush=True)


# The library's large forward products, alone, at the shapes the vendor line
# above times for config 5 (rows, in, out, kind).
PRODUCT_SHAPES = [(32768, 1024, 4096, "packed", "config-5 key fwd"),
                  (32768, 4096, 1024, "fp16", "config-5 value fwd")]


def product_gemm(rt, reps: int = 10, with_vendor: bool = True) -> None:
    """One JSON line per config-5 forward product of the library alone
    (ullis_hip_binary_linear / ullis_hip_fp16_linear, fp16 output, no epilogue
    beyond the row scale), `reps` calls between events on the library's stream;
    then (with_vendor) the vendor fp16 GEMM at the same shapes, so that one
    process holds both for `rocprofv3 --pmc` passes."""
    import ctypes as C

    from ullis_amd.synth import f16, pack_bits

    lib, ctx = rt.lib, rt.ctx
    rng = np.random.default_rng(0)
    for rows, k, n, kind, name in PRODUCT_SHAPES:
        x = rt.put(f16(rng.standard_normal(rows * k)))
        y = rt.buffer(2 * rows * n)
        if kind == "packed":
            bits = rt.put(pack_bits(rng.integers(0, 2, n * k).astype(bool)))
            sc = rt.put(f16(np.full(n, 0.01)))

            def call():
                rt._check(lib.ullis_hip_binary_linear(ctx, x.ptr, 1, bits.ptr, sc.ptr, None, rows,
                                                      k, n, None, y.ptr), "binary_linear")
        else:
            w = rt.put(f16(rng.standard_normal(n * k) * 0.02))

            def call():
                rt._check(lib.ullis_hip_fp16_linear(ctx, x.ptr, 1, w.ptr, rows, k, n, None, y.ptr),
                          "fp16_linear")
        for _ in range(3):
            call()
        rt.sync()
        rt._check(lib.ullis_hip_event_record(ctx, 0), "event")
        for _ in range(reps):
            call()
        rt._check(lib.ullis_hip_event_record(ctx, 1), "event")
        rt.sync()
        ms = C.c_float()
        rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 0, 1, C.byref(ms)), "elapsed")
        us = ms.value * 1e3 / reps
        tf = 2.0 * rows * k * n / (us * 1e-6) / 1e12
        print(json.dumps({"product_gemm": name, "kind": kind, "shape_MNK": [rows, n, k],
                          "us": round(us, 2), "tflops": round(tf, 1),
                          "frac": round(tf / FP16_PEAK_TFLOPS, 4)}), flush=True)
        del x, y
    if with_vendor:
        vendor_gemm([s for s in VENDOR_SHAPES if s[0] >= 32768])


def copy_calibration(rt, mib: int) -> None:
    """One copy kernel (ullis_hip_copy) that reads `mib` MiB and writes `mib` MiB.

    Under `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` its counter values give the factor
    between what the counters report and the bytes a kernel actually moves.
    """
    from ullis_amd.runtime import DeviceBuffer

    n = mib * (1 << 20)
    src = DeviceBuffer(rt, n)
    dst = DeviceBuffer(rt, n)
    rt._check(rt.lib.ullis_hip_copy(rt.ctx, dst.ptr, src.ptr, n), "copy")
    rt.sync()
    src.free()
    dst.free()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-rows", type=int, default=128,
                    help="tokens of each CPU-baseline window (0 disables it)")
    ap.add_argument("--cpu-runs", type=int, default=3,
                    help="CPU-baseline windows, run side by side; the median is reported")
    ap.add_argument("--cpu-sample", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--probe", default="auto",
                    help="'auto': roofline objects for the value and key backward pairs; a "
                         "launch class name: that class only; 'none': no roofline object")
    ap.add_argument("--decode-gemv", type=int, default=0, metavar="REPS",
                    help="instead of the train step, time the few-row (T = 1 decode) forward "
                         "products over REPS launches each and print one JSON line per product")
    ap.add_argument("--ln-isolated", type=int, default=0, metavar="REPS",
                    help="instead of the train step, time the LayerNorm row kernels alone over "
                         "REPS launches each, beside a device copy of the same bytes")
    ap.add_argument("--stress", action="store_true",
                    help="instead of the bench line, run config 5 (the MFMA stress profile) "
                         "and print its step time and per-kernel MFMA rates")
    ap.add_argument("--rosa-live", action="store_true",
                    help="instead of the bench line, time the step with the suffix automaton "
                         "driven live, layer by layer, against indices given up front")
    ap.add_argument("--decode-step", action="store_true",
                    help="instead of the bench line, time the T = 1 decode step at configs 4 "
                         "and 5, batch 1 and 8, against its weight-streaming floor")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="instead of the bench line, time the vendor fp16 GEMM (torch.matmul) at "
                         "the heron GEMM shapes, as a yardstick")
    ap.add_argument("--product-gemm", type=int, default=0, metavar="REPS",
                    help="instead of the bench line, time the library's config-5 forward products "
                         "alone (REPS calls each), then the vendor GEMM at the same shapes")
    ap.add_argument("--graph", type=int, default=None,
                    help="1: replay each step's launches from a captured HIP graph (default 0; "
                         "with --decode-step, default 1)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after the timed region, run one plain device copy kernel of this many "
                         "MiB (read + write) so HBM counters can be scaled against known bytes")
    args = ap.parse_args()
    if args.cpu_sample > 0:
        cpu_sample(args.cpu_sample)
        return 0
    if args.vendor_gemm:
        vendor_gemm()
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one MI355X only (no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    plain = (args.decode_gemv == 0 and not args.stress and args.ln_isolated == 0 and
             not args.rosa_live and not args.decode_step and args.product_gemm == 0)
    # the CPU baseline's child processes start before this process touches the GPU
    baseline = (cpu_baseline(args.cpu_rows, max(1, args.cpu_runs))
                if plain and args.cpu_rows > 0 else None)

    from ullis_amd.runtime import HeronShape, HeronTrainer, HipRuntime
    from ullis_amd.synth import heron_arena, step_inputs

    c = CONFIG
    shape = HeronShape(**c)
    if args.product_gemm > 0:
        # the vendor line needs torch's HIP runtime up before the library's
        import torch

        torch.cuda.init()
    rt = HipRuntime(0)
    if args.decode_gemv > 0:
        decode_gemv(rt, args.decode_gemv)
        return 0
    if args.product_gemm > 0:
        product_gemm(rt, args.product_gemm)
        return 0
    if args.stress:
        stress_profile(rt, args.steps, args.warmup)
        return 0
    if args.ln_isolated > 0:
        layer_norm_isolated(rt, args.ln_isolated)
        return 0
    if args.rosa_live:
        rosa_live(rt, args.steps, args.warmup)
        return 0
    if args.decode_step:
        decode_step_bench(rt, args.steps, args.warmup,
                          graph=True if args.graph is None else bool(args.graph))
        return 0
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=7)
    trainer.upload_arena(arena)
    trainer.set_graph(bool(args.graph or 0))
    x, labels, idx = step_inputs(shape.rows, c["d_model"], c["vocab"], c["n_layers"], c["batch"],
                                 c["time"], seed=7)
    dl, di = rt.put(labels), rt.put(idx)
    # embedding table [vocab, d] (f16 + fp32 carry) and token ids; the gather
    # writes x_emb each step
    rng = np.random.default_rng(7)
    table = rt.put(rng.standard_normal(c["vocab"] * c["d_model"]).astype(np.float16).view(np.uint16))
    table_res = rt.zeros(np.float32, c["vocab"] * c["d_model"])
    token_ids = rt.put(rng.integers(0, c["vocab"], shape.rows).astype(np.uint32))
    dx = rt.put(x)
    g = rt.zeros(np.float32, shape.rows * c["d_model"])
    rl = rt.zeros(np.float32, shape.rows)
    st = rt.zeros(np.float32, 4)
    words = (shape.rows * c["d_model"] + 31) // 32
    qkv = rt.zeros(np.uint32, c["n_layers"] * 3 * words)

    def step():
        trainer.step_tokens(table, table_res, token_ids, dl, NO_IGNORE, LR, di, dx, g, rl, st,
                            qkv)

    import ctypes as C

    lib, ctx = rt.lib, rt.ctx

    def timed(n):
        """n steps bracketed by events on the library's stream and stream syncs."""
        rt.sync()
        rt._check(lib.ullis_hip_event_record(ctx, 0), "event")
        t0 = time.perf_counter()
        for _ in range(n):
            step()
        rt._check(lib.ullis_hip_event_record(ctx, 1), "event")
        rt.sync()
        wall = time.perf_counter() - t0
        ms = C.c_float()
        rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 0, 1, C.byref(ms)), "elapsed")
        return ms.value, wall

    for _ in range(args.warmup):
        step()
    # the reported throughput: K steps with nothing armed
    total_ms, wall = timed(args.steps)
    ms_per_step = total_ms / args.steps
    tokens = shape.rows * args.steps
    value = tokens / (total_ms / 1e3)
    loss = float(st.download(np.float32, 4)[0])
    # the roofline objects: for each probed launch class, K more steps with
    # its launches timed by workgroup wall-clock stamps (kept out of the
    # reported steps). Kernel-timestamp events around a launch were tried too:
    # in the two-stream step they slow the probed launch (value backward pair
    # 26.1 -> 30.7 us under rocprofv3) and read 8 us above rocprofv3 besides.
    if args.probe == "auto":
        probes = ROOFLINE_PROBES
    elif args.probe == "none":
        probes = ()
    else:
        probes = (("roofline", args.probe),)
    rooflines = {}
    for key, name in probes:
        trainer.probe_begin(name)
        st_ms, _ = timed(args.steps)
        stp = trainer.probe_end(name)
        if not stp["count"]:
            continue
        avg_s = stp["total_ms"] / stp["count"] / 1e3
        mfma = stp["bound"] == "mfma"
        scale = 1e12 if mfma else 1e9
        peak = FP16_PEAK_TFLOPS if mfma else HBM_PEAK_GBS
        achieved = stp["work"] / avg_s / scale
        prof_us = ROCPROF_AVG_US.get(name)
        rooflines[key] = {
            "bound": stp["bound"], "achieved": round(achieved, 2), "peak": peak,
            "unit": "TFLOP/s" if mfma else "GB/s", "frac": round(achieved / peak, 4),
            "traffic": TRAFFIC_BYTES.get(name), "kernel": stp["name"], "probe": name,
            "avg_us": round(avg_s * 1e6, 2), "launches": stp["count"],
            "timing": "workgroup wall-clock stamps per launch (earliest start to latest end)",
            "rocprof_avg_us": prof_us,
            "rocprof_frac": (round(stp["work"] / (prof_us * 1e-6) / scale / peak, 4)
                             if prof_us else None),
            "probe_pass_ms_per_step": round(st_ms / args.steps, 4),
        }
    # the reference's TrainStepProfile phases (main-stream segments), over a
    # few more steps run eagerly, outside the reported ones
    phases = None
    if args.probe != "none":
        trainer.phases_begin()
        timed(5)
        ph = trainer.phases_end()
        phases = {k: round(v, 4) for k, v in ph["phases_ms"].items()}
    if args.copy_mib > 0:
        copy_calibration(rt, args.copy_mib)

    line = {
        "metric": "train tokens/s (heron D512 L12 T2048)",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded; random-init heron parameters and embedding table, uniform "
                "token ids and labels, ROSA indices Bernoulli(0.5))",
        "config": {"workload": "heron train step (config 4): D512 L12 F2048 V8192 T2048 B1, "
                               "stop_grad_bits, lr 0.01",
                   "global_batch": c["batch"], "seq_len": c["time"], "parallelism": "none (1 GPU)"},
        "wall_s": round(wall, 3),
        "loss_last_step": round(loss, 5),
        "roofline": rooflines.get("roofline"),
        "roofline_packed": rooflines.get("roofline_packed"),
        "cpu_baseline": baseline,
        "phases_ms": phases,
    }
    print(json.dumps(line), flush=True)
    trainer.close()
    rt.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
