#!/usr/bin/env python3
"""Decode-step benchmark on one MI355X.

Workload: one greedy decode step of a Qwen2.5-0.5B-shaped model (24 layers, hidden 896, ffn
4864, 14/2 heads, head_dim 64, tied vocab 151936), fp16 weights N(0, 0.02) from the portable
seeded generator, fp16 KV cache pre-filled with N(0, 1), steps centred on cache position 1024.
A "step" is one token: embed -> 24 x (norm+QKV+rope+append, attention, o_proj+residual,
norm+gate/up+swiglu+down+residual) -> norm + LM head + argmax, replayed as one hipGraph with the
greedy id fed back on the device; the feed-forward block is one launch in layers 0..22 and two
(gate/up, down) in layer 23. Inputs are resident in HBM before the timed region.

value = algorithmic HBM bytes of the timed steps / time (GB/s): every weight once as fp16, the KV
rows 0..p read once as fp16, the appended rows written, activations as f32 once per kernel that
reads or writes them. tok/s is reported beside it.

roofline: the kernel with the largest share of the step's time, the one-launch feed-forward
block (rms_norm + 2 x 4864 x 896 gate/up GEMV + swiglu + 896 x 4864 down GEMV, added into the
hidden state's partial vectors), timed with HIP events on its stream while it rotates over the
23 fused layers' weights (601 MB, more than the 256 MB MALL); its share of the step comes from
this run's per-kind timing (phases_us: each kernel kind graph-replayed over the layers it runs
in); its HBM traffic and L2 hit rate come from the counter runs of the same kernel inside whole
steps (traffic_source names them).

cpu_baseline: the reference's CPU path for the same workload (oracle/'s f32 step: HostMatVec-
order f32 sums, gcc -O3) on one host core, the median of 10 single-step timings; the same with
its row loops over every core the process may use (OpenMP) is reported beside it, with the CPU
model.

kernels: per-launch figures of the per-op launchers at the batched element-wise/reduction shapes
and the decode GEMV suite (inputs under 256 MB rotated over >= 512 MB of copies; the launches
replayed from a hipGraph), and torch's device copy for reference.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "muyo-llm_amd"))

METRIC = "F16 GEMV+norm HBM GB/s (% of MI355X peak); Qwen2.5-0.5B-shape decode tok/s"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK = 2.5e15  # dense fp16 matrix-core flop/s of MI355X
# HBM bytes per launch of the one-launch feed-forward block (0.5B shape) from rocprofv3 FETCH_SIZE /
# WRITE_SIZE, each scaled by what the counter reads for a 256 MiB device copy, and its L2 hit rate
# (TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum)), over whole steps launched kernel by kernel
# (profiles/decode_step_counters_0.5b.md: `--kernel-only step_05b`, `--summarize-counters`).
FFN_TRAFFIC_BYTES = 27_246_760
FFN_L2_HIT_RATE = 0.192
FFN_COUNTER_SOURCE = ("profiles/decode_step_counters_0.5b.md: rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE (each scaled "
                      "by a 256 MiB device copy) and TCC_HIT/TCC_MISS over whole steps, ffn rows")


def step_bytes(c: dict, position: int) -> int:
    """Algorithmic HBM bytes of one decode step at cache row `position` (keys 0..position)."""
    h, f, hd = c["hidden"], c["ffn"], c["head_dim"]
    q, kv = c["heads"] * hd, c["kv_heads"] * hd
    qkv = q + 2 * kv
    weights = c["layers"] * 2 * (qkv * h + h * q + 2 * f * h + h * f) + 2 * c["vocab"] * h
    small = c["layers"] * 4 * (qkv + 2 * h) + 4 * h  # qkv bias, two norm weights per layer, final norm
    cache = c["layers"] * (2 * 2 * kv * (position + 1) + 2 * 2 * kv)  # K+V rows read, k/v row written
    # Activations (f32), per layer: x read by QKV, q written/read, attention out written/read, x read
    # and x1 written by o_proj, x1 read by gate/up, act written/read, x1 read and x2 written by down.
    act = c["layers"] * 4 * (h + 2 * q + 2 * q + 2 * h + h + 2 * f + 2 * h)
    head = 2 * h + 4 * h + 4 * h + 4 * c["vocab"]  # embedding row, x write, x read, logits
    return weights + small + cache + act + head


def lm_head_bytes(c: dict) -> int:
    return 2 * c["vocab"] * c["hidden"] + 4 * c["hidden"] * 2 + 4 * c["vocab"]


def gate_up_bytes(c: dict) -> int:
    return 2 * 2 * c["ffn"] * c["hidden"] + 4 * c["hidden"] * 2 + 4 * c["ffn"]


def ffn_bytes(c: dict) -> int:
    """The one-launch feed-forward block: gate, up and down weights once, the input and the norm
    weight read, the hidden state's new value written once."""
    return 3 * 2 * c["ffn"] * c["hidden"] + 4 * c["hidden"] * 3


STEP_KINDS = ("QKV", "ATTENTION", "O_PROJ", "GATE_UP", "DOWN")


def ffn_fused(c: dict) -> bool:
    """True when the decoder runs the feed-forward block as one launch (MUYO_KERNEL_FFN) in every
    layer but the last: hidden sizes up to 1024 whose o_proj is not split by kv group, which holds
    for the 0.5B shape and not for the 7B one (the decoder's own test; launch counts are checked
    against muyo_decoder_launches_per_step where a decoder is at hand)."""
    return c["hidden"] <= 1024 and c["layers"] >= 2


def layer_kinds(c: dict, layer: int) -> tuple:
    """The kernels of layer `layer` in the step's launch order."""
    if ffn_fused(c) and layer + 1 < c["layers"]:
        return ("QKV", "ATTENTION", "O_PROJ", "FFN")
    return STEP_KINDS


def kind_layers(c: dict) -> dict:
    """Per kernel kind, the layers whose step runs it; GATE_UP and DOWN are also timed over every
    layer in their two-launch form, for comparison."""
    out = {kind: list(range(c["layers"])) for kind in STEP_KINDS}
    if ffn_fused(c):
        out["FFN"] = list(range(c["layers"] - 1))
    return out


def kernel_bytes(c: dict, kind: str, position: int) -> int:
    """Algorithmic HBM bytes of one launch of a decode-step kernel at cache row `position`: weights
    once as fp16, K/V rows 0..position once as fp16, f32 activations once per kernel touching them.
    Attention writes per-chunk partials (head_dim + 2 floats per chunk and query head) that the
    o_proj prologue reads: all of them (q dim <= 1024, 8 chunks), or, split by kv group (16 chunks),
    its group's, leaving one partial sum of the hidden state per kv group for gate/up's prologue
    to add up (gate/up then also stores that sum, the down projection's residual)."""
    h, f, hd, v = c["hidden"], c["ffn"], c["head_dim"], c["vocab"]
    q, kv = c["heads"] * hd, c["kv_heads"] * hd
    merged = q <= 1024
    chunks = min(8 if merged else 16, -(-c["max_seq"] // (2048 // hd)))
    partials = 4 * chunks * c["heads"] * (hd + 2)
    parts = 4 * c["kv_heads"] * h  # the grouped o_proj's per-group sums
    table = {
        "embed": 8 * 1024 + 2 * h + 4 * h,
        "qkv": 2 * (q + 2 * kv) * h + 4 * (q + 2 * kv) + 8 * h + 4 * q + 4 * kv,
        "attention": 4 * kv * (position + 1) + 4 * q + partials,
        "o_proj": 2 * h * q + partials + 4 * h + (4 * h if merged else parts),
        "gate_up": 4 * f * h + (8 * h if merged else parts + 8 * h) + 4 * f,
        "down": 2 * h * f + 4 * f + 8 * h,
        "ffn": ffn_bytes(c),
        "lm_head": lm_head_bytes(c),
    }
    return table[kind]


def chain_bytes_of(c: dict, position: int) -> list:
    """Algorithmic bytes of each launch of one step, in launch order."""
    seq = [kernel_bytes(c, "embed", position)]
    for layer in range(c["layers"]):
        seq += [kernel_bytes(c, kind.lower(), position) for kind in layer_kinds(c, layer)]
    return seq + [kernel_bytes(c, "lm_head", position)]


def enqueue_step(dec, shape, stream) -> None:
    """One decode step launched kernel by kernel (the graph's sequence, enqueued eagerly)."""
    dec.enqueue_kernel("EMBED", 0, stream)
    for layer in range(shape["layers"]):
        for kind in layer_kinds(shape, layer):
            dec.enqueue_kernel(kind, layer, stream)
    dec.enqueue_kernel("LM_HEAD", 0, stream)


def settle(torch) -> None:
    """Waits until the device is idle and then a little longer. Freeing a large device buffer (an
    earlier decoder's arena, torch's cache) starts work in the driver that keeps HBM busy for a
    while afterwards: a 7B-shape step measured 2.563 ms before such a free, 2.628 ms within
    0.25 s after freeing 15 GB and 2.563 ms again from 0.5 s on. Timed regions start after it."""
    torch.cuda.synchronize()
    time.sleep(0.75)


def time_decode(mh, torch, shape, position, steps, warmup, seed, sampler=None):
    """Returns (ms per step, positions timed, decoder launches per step, generated ids, median ms
    per step over 16 runs of the same positions). `sampler`: keyword
    parameters of the device sampler (greedy when None), with a synthetic prompt as history."""
    stream = torch.cuda.current_stream()
    start = max(1, position - steps // 2 - warmup)
    dec = mh.Decoder(mh.qwen2_config(**shape))
    try:
        dec.fill_random(seed)
        dec.fill_kv_random(start, seed + 1)
        if sampler is not None:
            dec.set_history([(7919 * i) % shape["vocab"] for i in range(start)])
            dec.set_sampler(**sampler)
        token = 9707
        dec.generate_async(token, start, warmup, stream.cuda_stream)
        torch.cuda.synchronize()
        warm_ids = dec.generated_ids(warmup)
        first = start + warmup
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        settle(torch)
        begin.record(stream)
        dec.generate_async(warm_ids[-1], first, steps, stream.cuda_stream)
        end.record(stream)
        torch.cuda.synchronize()
        ms = begin.elapsed_time(end) / steps
        ids = dec.generated_ids(steps)
        launches = dec.launches_per_step()
        # The same steps again as 16 runs of steps/16 graph replays, an event after each run (the
        # runs are queued ahead, so the GPU never waits on the host): the median run's time per
        # step, its set-up kernels spread over the run.
        runs = 16
        per_run = max(1, steps // runs)
        events = [torch.cuda.Event(enable_timing=True) for _ in range(runs + 1)]
        torch.cuda.synchronize()
        events[0].record(stream)
        for i in range(runs):
            dec.generate_async(ids[-1], first + i * per_run, per_run, stream.cuda_stream)
            events[i + 1].record(stream)
        torch.cuda.synchronize()
        per_step = sorted(events[i].elapsed_time(events[i + 1]) / per_run for i in range(runs))
        median_ms = (per_step[runs // 2 - 1] + per_step[runs // 2]) / 2
    finally:
        dec.close()
    return ms, list(range(first, first + steps)), launches, ids, median_ms


def prefill_flops(c: dict, prompt: int) -> int:
    """Algorithmic flops of a prompt fed from row 0, each multiply-add counted once: the layers'
    projections for every token, causal attention over rows 0..i for token i, and the LM head for
    the last token only."""
    hd, qdim = c["head_dim"], c["heads"] * c["head_dim"]
    qkv_rows = (c["heads"] + 2 * c["kv_heads"]) * hd
    per_token = 2 * (qkv_rows * c["hidden"] + c["hidden"] * qdim + 3 * c["ffn"] * c["hidden"])
    attention = 4 * hd * c["heads"] * prompt * (prompt + 1) // 2
    return c["layers"] * (per_token * prompt + attention) + 2 * c["vocab"] * c["hidden"]


def time_prefill(mh, torch, shape, prompt, reps, seed):
    """Milliseconds per muyo_decoder_prefill of `prompt` tokens at row 0 (a synchronous call:
    host clock around it, token upload and next-token readback included)."""
    tokens = [(7919 * i + 13) % shape["vocab"] for i in range(prompt)]
    dec = mh.Decoder(mh.qwen2_config(**shape))
    try:
        dec.fill_random(seed)
        first = dec.prefill(tokens, 0)
        settle(torch)
        begin = time.perf_counter()
        for _ in range(reps):
            again = dec.prefill(tokens, 0)
        ms = (time.perf_counter() - begin) * 1e3 / reps
        assert again == first
    finally:
        dec.close()
    return ms, first


def library_gemm(torch, m, n, k, reps=10):
    """TFLOP/s of the platform library's fp16 GEMM (torch.matmul: fp16 in, fp16 out) at one
    prefill GEMM shape, for comparison with the split-plane kernels."""
    x = torch.randn(m, k, device="cuda", dtype=torch.float16)
    w = torch.randn(n, k, device="cuda", dtype=torch.float16)
    for _ in range(2):
        torch.matmul(x, w.t())
    settle(torch)
    b, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b.record()
    for _ in range(reps):
        torch.matmul(x, w.t())
    e.record()
    torch.cuda.synchronize()
    ms = b.elapsed_time(e) / reps
    del x, w
    return round(2 * m * n * k / (ms * 1e-3) / 1e12, 1)


def prefill_line(mh, torch, shape, prompt, reps, seed, decode_ms):
    ms, first = time_prefill(mh, torch, shape, prompt, reps, seed)
    flops = prefill_flops(shape, prompt)
    rate = flops / (ms * 1e-3)
    return {
        "prompt_tokens": prompt, "ms": round(ms, 3), "tok_per_s": round(prompt / (ms * 1e-3), 1),
        # Each multiply-add counted once; the matrix cores execute twice that, since every
        # product takes the activation as two fp16 planes (hi + lo).
        "TFLOP/s": round(rate / 1e12, 1), "flops": flops,
        "pct_of_f16_mfma_peak": round(100 * rate / MFMA_F16_PEAK, 1),
        "mfma_executed_TFLOP/s": round(2 * rate / 1e12, 1),
        "pct_of_f16_mfma_peak_executed": round(200 * rate / MFMA_F16_PEAK, 1),
        "library_fp16_gemm_TFLOP/s_gate_up_shape": library_gemm(torch, prompt, 2 * shape["ffn"], shape["hidden"]),
        "token_by_token_ms": round(prompt * decode_ms, 2) if decode_ms else None,
        "next_token": first,
    }


def time_kernels(mh, torch, shape, seed, rounds):
    """Per-launch ms of the LM-head kernel and of the roofline kernel (the one-launch feed-forward
    block where the decoder runs it, else gate/up) rotated over the layers that run it."""
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream
    dec = mh.Decoder(mh.qwen2_config(**shape))
    out = {}
    try:
        dec.fill_random(seed)
        dec.set_state(1, 1, s)
        for _ in range(3):
            dec.enqueue_kernel("LM_HEAD", 0, s)
        b, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        settle(torch)
        b.record(stream)
        for _ in range(rounds):
            dec.enqueue_kernel("LM_HEAD", 0, s)
        e.record(stream)
        torch.cuda.synchronize()
        out["lm_head_ms"] = b.elapsed_time(e) / rounds
        kind = "FFN" if ffn_fused(shape) else "GATE_UP"
        layers = kind_layers(shape)[kind]
        for layer in layers:
            dec.enqueue_kernel(kind, layer, s)
        torch.cuda.synchronize()
        b.record(stream)
        for _ in range(max(1, rounds // 4)):
            for layer in layers:
                dec.enqueue_kernel(kind, layer, s)
        e.record(stream)
        torch.cuda.synchronize()
        out["roofline_kind"] = kind
        out["roofline_ms"] = b.elapsed_time(e) / (max(1, rounds // 4) * len(layers))
    finally:
        dec.close()
    return out


def time_phases(mh, torch, shape, position, seed, reps=20) -> dict:
    """Microseconds per launch of each per-layer kernel kind (kind_layers), each kind's launches
    over its layers captured into one graph (torch's CUDAGraph around the decoder's per-kernel
    launches) and replayed `reps` times: the kernels as the step's graph runs them, minus their
    data dependence on the neighbouring kinds."""
    stream = torch.cuda.Stream()
    dec = mh.Decoder(mh.qwen2_config(**shape))
    out = {}
    try:
        dec.fill_random(seed)
        dec.fill_kv_random(position, seed + 1)
        dec.set_state(9707, position, stream.cuda_stream)
        settle(torch)
        for kind, layers in kind_layers(shape).items():
            for layer in layers:
                dec.enqueue_kernel(kind, layer, stream.cuda_stream)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for layer in layers:
                    dec.enqueue_kernel(kind, layer, stream.cuda_stream)
            for _ in range(2):
                graph.replay()
            torch.cuda.synchronize()
            b, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                b.record(stream)
                for _ in range(reps):
                    graph.replay()
                e.record(stream)
            torch.cuda.synchronize()
            out[kind.lower()] = 1000.0 * b.elapsed_time(e) / (reps * len(layers))
            del graph
    finally:
        dec.close()
    return out


def floor_chain(torch, byte_list, reps=20) -> dict:
    """The streaming floor of a launch sequence (libmuyo_floor.so's muyo_floor_chain): each
    launch only reads its algorithmic bytes from its own buffer region, chained in one hipGraph;
    milliseconds per chain with 2, 3 and 4 workgroups of 512 threads per CU, and the best."""
    import ctypes

    lib = ctypes.CDLL(str(ROOT / "muyo-llm_amd" / "libmuyo_floor.so"))
    lib.muyo_floor_chain.restype = ctypes.c_int
    lib.muyo_floor_chain.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_uint32, ctypes.c_uint32,
                                     ctypes.c_uint32, ctypes.POINTER(ctypes.c_double)]
    arr = (ctypes.c_uint64 * len(byte_list))(*byte_list)
    out = {}
    for per_cu in (2, 3, 4):
        settle(torch)  # the previous chain's (or decoder's) freed buffer
        ms = ctypes.c_double(0.0)
        rc = lib.muyo_floor_chain(arr, len(byte_list), per_cu, reps, ctypes.byref(ms))
        if rc != 0:
            raise RuntimeError(f"muyo_floor_chain failed: hipError {rc}")
        out[f"{per_cu}_per_cu_ms"] = round(ms.value, 5)
    out["best_ms"] = min(v for k, v in out.items() if k.endswith("_ms"))
    return out


def floor_report(mh, torch, which: str) -> dict:
    """The decode step beside its streaming floor. `which`: 05b (0.5B shape, cache rows
    1014..1033, as the default bench line) or 7b (7B shape, rows 2032..2047).
    chain: the step's launch sequence (embed, per layer qkv / attention / o_proj and the
    feed-forward launch or launches, LM head) with each launch's algorithmic bytes at the window's
    middle row, as pure streams; phases: per kind, as many launches of its bytes as pure streams
    as the kind has layers, beside the step's own kernels (time_phases), microseconds per launch."""
    shape = dict(mh.QWEN25_05B if which == "05b" else mh.QWEN25_7B)
    steps, warmup, centre = (20, 5, 1024) if which == "05b" else (16, 4, 2040)
    seed = 20261201 if which == "05b" else 20261208
    ms, positions, launches, _, median = time_decode(mh, torch, shape, centre, steps, warmup, seed)
    position = positions[len(positions) // 2]
    chain_bytes = chain_bytes_of(shape, position)
    assert len(chain_bytes) == launches, (len(chain_bytes), launches)
    chain = floor_chain(torch, chain_bytes)
    total = sum(chain_bytes)
    step_bytes_mid = step_bytes(shape, position)
    kernels = time_phases(mh, torch, shape, position, seed)
    phases = {}
    for kind, layers in kind_layers(shape).items():
        nbytes = kernel_bytes(shape, kind.lower(), position)
        stream_ms = floor_chain(torch, [nbytes] * len(layers))["best_ms"]
        stream_us = 1000.0 * stream_ms / len(layers)
        phases[kind.lower()] = {"bytes": nbytes, "stream_us": round(stream_us, 2),
                                "kernel_us": round(kernels[kind.lower()], 2),
                                "excess_us": round(kernels[kind.lower()] - stream_us, 2)}
    return {
        "shape": which, "positions": f"{positions[0]}..{positions[-1]}", "launches": launches,
        "step_ms": round(ms, 5), "step_ms_median": round(median, 5),
        "step_pct_of_peak": round(100 * step_bytes_mid / (ms * 1e-3) / 1e12 / 8, 1),
        "chain_bytes": total, "chain": chain,
        "chain_pct_of_peak": round(100 * total / (chain["best_ms"] * 1e-3) / 1e12 / 8, 1),
        "step_over_chain": round(ms / chain["best_ms"], 3),
        "phases": phases,
    }


def launch_floor_report(mh, which: str) -> dict:
    """What a kernel boundary costs (muyo-llm_amd/launch_floor, a child process): empty kernels
    replayed from hipGraphs of 122 and 1952 kernels; empty kernels dispatched from an AQL queue with
    system, agent or no fence scopes; and the decode step's launch sequence (`which`: 05b at cache
    row 1024, 7b at row 2040, each launch's algorithmic bytes as in `floor_report`) read by
    pure-stream kernels with agent or no fences, and with an 896-float activation handed from launch
    to launch in five coherence schemes (times in microseconds per chain)."""
    import subprocess

    shape = dict(mh.QWEN25_05B if which == "05b" else mh.QWEN25_7B)
    position = 1024 if which == "05b" else 2040
    chain = chain_bytes_of(shape, position)
    tool = ROOT / "muyo-llm_amd" / "launch_floor"
    code = ROOT / "muyo-llm_amd" / "launch_floor_kernels.co"
    run = subprocess.run([str(tool), str(code)], input="\n".join(str(b) for b in chain), capture_output=True,
                         text=True, timeout=300)
    if run.returncode != 0:
        raise RuntimeError(f"launch_floor failed ({run.returncode}): {run.stderr.strip()}")
    out = json.loads(run.stdout)
    stream = out["aql_stream_us"]
    agent = min(stream["agent"], stream["agent_again"])
    none = min(stream["none"], stream["none_again"])
    return {"shape": which, "position": position, "launches": len(chain), "chain_bytes": sum(chain), **out,
            "fences_us_per_chain": round(agent - none, 1),
            "fences_us_per_launch": round((agent - none) / len(chain), 3)}


def time_ops(mh, torch, reps: int = 10) -> dict:
    """Per-launch time of each per-op launcher at the batched shapes of the element-wise and
    reduction set (4096 rows at Qwen2.5-0.5B widths) and of the decode GEMV suite, through the C
    ABI with the reference's push-constant fills. Inputs smaller than 256 MB rotate over enough
    copies to total >= 512 MB per timed loop, so they stream from HBM rather than the MALL."""
    lib = mh.load()
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    floor = 512 * 1024 * 1024

    def normal(n, seed, mean=0.0, std=1.0):
        t = torch.empty(n, dtype=torch.float32, device="cuda")
        mh.check(lib.muyo_fill_normal_f32(t.data_ptr(), n, seed, mean, std, sp))
        return t

    def normal16(n, seed, mean=0.0, std=1.0):
        t = torch.empty(n, dtype=torch.float16, device="cuda")
        mh.check(lib.muyo_fill_normal_f16(t.data_ptr(), n, seed, mean, std, sp))
        return t

    def copies_for(nbytes):
        return max(1, -(-floor // nbytes)) if nbytes < 256 * 1024 * 1024 else 1

    def timed(launches, graph=True):
        """ms per launch. With `graph` and several launches, they are captured once into a hipGraph
        and replayed, so the figure is the kernels' own time plus the GPU's inter-kernel gaps,
        without the host's launch cost; each launch takes the stream as `st`."""
        graph = graph and len(launches) > 1
        for launch in launches:
            mh.check(launch(st=sp))
        torch.cuda.synchronize()
        if graph:
            captured = torch.cuda.CUDAGraph()
            with torch.cuda.graph(captured):
                capture = torch.cuda.current_stream().cuda_stream
                for launch in launches:
                    mh.check(launch(st=capture))
            run = captured.replay
            run()
        else:
            def run():
                for launch in launches:
                    mh.check(launch(st=sp))
        torch.cuda.synchronize()
        b, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        b.record(stream)
        for _ in range(reps):
            run()
        e.record(stream)
        torch.cuda.synchronize()
        return b.elapsed_time(e) / (reps * len(launches))

    out = {}

    def record(name, nbytes, ms, copies):
        out[name] = {"launch_ms": round(ms, 5), "bytes_per_launch": nbytes, "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "pct_of_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1), "rotated_copies": copies}

    rows = 4096
    # rms_norm 4096 x 896, fp16 weight N(1, 0.1)
    nbytes = rows * (3584 + 3584) + 1792
    k = copies_for(nbytes)
    xs = [normal(rows * 896, 10 + i) for i in range(k)]
    ys = [torch.empty_like(x) for x in xs]
    w16 = normal16(896, 9, 1.0, 0.1)
    pc = mh.rows_push_constants(896, rows, 1e-6)
    record("rms_norm_4096x896", nbytes, timed([
        (lambda x=x, y=y, st=None: lib.muyo_rms_norm_f32_f16w(mh.ref(pc), 1, x.data_ptr(), w16.data_ptr(), y.data_ptr(), None,
                                                     rows, 1, 1, st)) for x, y in zip(xs, ys)]), k)
    # add 4096 x 896
    nbytes = rows * 10752
    k = copies_for(nbytes)
    bs = [normal(rows * 896, 40 + i) for i in range(k)]
    pc = mh.add_push_constants(rows * 896, row=896)
    record("add_4096x896", nbytes, timed([
        (lambda a=a, b=b, y=y, st=None: lib.muyo_add_f32(mh.ref(pc), 1, a.data_ptr(), b.data_ptr(), y.data_ptr(), None,
                                               *mh.add_dispatch(rows * 896), st)) for a, b, y in zip(xs, bs, ys)]), k)
    del xs, ys, bs
    # swiglu 4096 x (2 x 4864)
    n = rows * 4864
    nbytes = rows * 58368
    k = copies_for(nbytes)
    gs = [normal(n, 60 + i) for i in range(k)]
    us = [normal(n, 70 + i) for i in range(k)]
    ds = [torch.empty_like(g) for g in gs]
    pc = mh.glu_push_constants(n, 4864)
    record("swiglu_4096x4864", nbytes, timed([
        (lambda g=g, u=u, d=d, st=None: lib.muyo_swiglu_f32(mh.ref(pc), g.data_ptr(), u.data_ptr(), d.data_ptr(),
                                                  *mh.add_dispatch(n), st)) for g, u, d in zip(gs, us, ds)]), k)
    del gs, us, ds
    # rope_neox 4096 tokens x 16 heads x 64, theta 1e6, positions in [0, 2047]
    heads = 16
    nbytes = rows * (4096 + 4096 + 4)
    k = copies_for(nbytes)
    xs = [normal(rows * heads * 64, 80 + i) for i in range(k)]
    ys = [torch.empty_like(x) for x in xs]
    gen = torch.Generator(device="cuda").manual_seed(81)
    pos = torch.randint(0, 2048, (rows,), dtype=torch.int32, device="cuda", generator=gen)
    pc = mh.rope_push_constants(heads, 64, 1e6, tokens=rows)
    record("rope_neox_4096x16x64", nbytes, timed([
        (lambda x=x, y=y, st=None: lib.muyo_rope_neox_f32(mh.ref(pc), x.data_ptr(), pos.data_ptr(), None, y.data_ptr(), None,
                                                 heads * rows, 1, 1, st)) for x, y in zip(xs, ys)]), k)
    del xs, ys
    # softmax 4096 x 14 heads x 2048, N(0, 3)
    srows = rows * 14
    x = normal(srows * 2048, 90, 0.0, 3.0)
    y = torch.empty_like(x)
    pc = mh.soft_max_push_constants(srows, 2048, 1.0)
    record("soft_max_4096x14x2048", srows * 2048 * 8, timed([
        lambda st=None: lib.muyo_soft_max_f32(mh.ref(pc), x.data_ptr(), None, None, y.data_ptr(), *mh.row_dispatch(srows), st)]),
        1)
    del x, y
    # argmax 4096 x 151936, N(0, 2)
    x = normal(rows * 151936, 91, 0.0, 2.0)
    idx = torch.empty(rows, dtype=torch.int32, device="cuda")
    pc = mh.argmax_push_constants(151936, rows)
    record("argmax_4096x151936", rows * 151936 * 4 + rows * 4, timed([
        lambda st=None: lib.muyo_argmax_f32(mh.ref(pc), x.data_ptr(), idx.data_ptr(), *mh.row_dispatch(rows), st)]), 1)
    del x, idx
    # decode GEMV suite (Qwen2.5-0.5B): fp16 W N(0, 0.02), f32 x, f32 y (+ f32 bias for QKV)
    spec = mh.MuyoMatVecSpec(32, 1, 1)
    for name, r, c, bias in [("gemv_qkv_1152x896", 1152, 896, True), ("gemv_o_896x896", 896, 896, False),
                             ("gemv_gate_up_9728x896", 9728, 896, False), ("gemv_down_896x4864", 896, 4864, False),
                             ("gemv_lm_head_151936x896", 151936, 896, False)]:
        nbytes = 2 * r * c + 4 * c + 4 * r + (4 * r if bias else 0)
        k = copies_for(nbytes)
        ws = [normal16(r * c, 100 + i, 0.0, 0.02) for i in range(k)]
        xv = normal(c, 99, 0.0, 1.0)
        ys = [torch.empty(r, dtype=torch.float32, device="cuda") for _ in range(k)]
        bv = normal(r, 98, 0.0, 0.02) if bias else None
        pc = mh.mat_vec_push_constants(c, r, fusion_flags=mh.FUSION_BIAS0 if bias else 0)
        record(name, nbytes, timed([
            (lambda w=w, y=y, st=None: lib.muyo_mul_mat_vec_f16_f32_f32(mh.ref(pc), mh.ref(spec), w.data_ptr(), xv.data_ptr(),
                                                               y.data_ptr(), bv.data_ptr() if bias else None, None, r,
                                                               1, 1, st)) for w, y in zip(ws, ys)]), k)
        del ws, ys
    # device copy reference: torch's copy of 256 MiB (read + write)
    src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    record("device_copy_256MiB", 2 * src.numel() * 4, timed([lambda st=None: (dst.copy_(src), 0)[1]], graph=False), 1)
    del src, dst
    torch.cuda.empty_cache()
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(shape, position, samples, seed):
    """The reference's CPU path for the same workload, timed on this host (TEST INFRASTRUCTURE:
    oracle/'s oracle_decode_step_f32, built -O3: every projection and the LM head an f32 running
    sum in column order as src/MatVec.cpp:52-60 HostMatVec writes it, the reference's softmax,
    rms_norm, swiglu, rope and greedy loops, composed into tools/reference_qwen2.py:100-166's
    step). (a) one thread, the reference's own configuration; (b) its row loops split over every
    core sched_getaffinity grants (OpenMP). Each variant: one untimed step, then the median of
    `samples` single-step timings at consecutive cache rows from `position`."""
    import statistics

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    granted = len(os.sched_getaffinity(0))
    # The host's share of cores for this process: OMP_NUM_THREADS when the environment sets it.
    cores = min(granted, int(os.environ.get("OMP_NUM_THREADS", granted) or granted))
    model = oracle.Model(**shape)
    model.fill_random(seed)
    model.fill_kv_random(position, seed + 1)

    def run(threads, first):
        oracle.set_threads(threads)
        token = 9707 % shape["vocab"]
        model.step_f32(token, first)
        times = []
        for i in range(samples):
            t0 = time.perf_counter()
            model.step_f32(token, first + 1 + i)
            times.append(time.perf_counter() - t0)
        rows = list(range(first + 1, first + 1 + samples))
        sec = statistics.median(times)
        nbytes = statistics.median(step_bytes(shape, r) for r in rows)
        return sec, nbytes / sec / 1e9, rows

    sec1, gbs1, rows1 = run(1, position)
    secn, gbsn, rowsn = run(cores, rows1[-1] + 1)
    model_name = cpu_model()
    return {
        "value": round(gbs1, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"median of {samples} single decode steps of the same 0.5B-shape workload at cache rows "
                  f"{rows1[0]}..{rows1[-1]} ({sec1 * 1e3:.1f} ms a step, {1.0 / sec1:.3f} tok/s): the reference's "
                  f"CPU path (f32 HostMatVec-order sums), gcc -O3, 1 thread, on {model_name}",
        "tok_per_s": round(1.0 / sec1, 4),
        "cpu_model": model_name,
        "openmp": {"value": round(gbsn, 3), "unit": "GB/s", "cores": cores, "tok_per_s": round(1.0 / secn, 4),
                   "sample": f"median of {samples} steps at rows {rowsn[0]}..{rowsn[-1]} "
                             f"({secn * 1e3:.1f} ms a step), row loops over {cores} threads ({granted} cores in the "
                             f"affinity mask, OMP_NUM_THREADS {os.environ.get('OMP_NUM_THREADS', 'unset')})"},
    }


def kernel_only(mh, torch, which: str, launches: int) -> dict:
    """Launch one kernel `launches` times back to back (for rocprofv3 kernel traces and counters).

    lm_head: the 0.5B-shape LM-head kernel (272,884,224 algorithmic bytes per launch).
    copy:    torch's device copy of 256 MiB f32 (268,435,456 bytes read + the same written), the
             calibration for FETCH_SIZE / WRITE_SIZE.
    """
    stream = torch.cuda.current_stream()
    b, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if which == "lm_head":
        shape = dict(mh.QWEN25_05B)
        dec = mh.Decoder(mh.qwen2_config(**shape))
        try:
            dec.fill_random(20261201)
            dec.set_state(1, 1, stream.cuda_stream)
            for _ in range(3):
                dec.enqueue_kernel("LM_HEAD", 0, stream.cuda_stream)
            torch.cuda.synchronize()
            b.record(stream)
            for _ in range(launches):
                dec.enqueue_kernel("LM_HEAD", 0, stream.cuda_stream)
            e.record(stream)
            torch.cuda.synchronize()
        finally:
            dec.close()
        nbytes = lm_head_bytes(shape)
    elif which == "copy":
        n = 64 * 1024 * 1024
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        b.record(stream)
        for _ in range(launches):
            dst.copy_(src)
        e.record(stream)
        torch.cuda.synchronize()
        nbytes = 2 * 4 * n
    elif which in ("step_05b", "step_7b"):
        shape = dict(mh.QWEN25_05B if which == "step_05b" else mh.QWEN25_7B)
        position = 1024 if which == "step_05b" else 2040
        launches = min(launches, shape["max_seq"] - position)
        dec = mh.Decoder(mh.qwen2_config(**shape))
        try:
            dec.fill_random(20261201)
            dec.fill_kv_random(position, 20261202)
            dec.set_state(9707, position, stream.cuda_stream)
            torch.cuda.synchronize()
            b.record(stream)
            for _ in range(launches):
                enqueue_step(dec, shape, stream.cuda_stream)
            e.record(stream)
            torch.cuda.synchronize()
        finally:
            dec.close()
        nbytes = sum(step_bytes(shape, position + i) for i in range(launches)) // launches
    else:
        raise ValueError(which)
    ms = b.elapsed_time(e) / launches
    return {"kernel": which, "launches": launches, "avg_ms": round(ms, 5), "bytes_per_launch": nbytes,
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}


def step_kind(name: str, previous: str | None) -> str | None:
    """The decode-step kernel a rocprofv3 kernel name belongs to (None for anything else)."""
    if "BeginStep" in name:
        return "embed"
    if "QkvEpi" in name:
        return "qkv"
    if "AttentionChunk" in name:
        return "attention"
    if "AttentionMerge" in name:
        return "merge"
    if "OProjGroup" in name:
        return "o_proj"
    if "GateUpEpi" in name:
        return "gate_up"
    if "FfnFused" in name:
        return "ffn"
    if "LmHeadEpi" in name:
        return "lm_head"
    if "ResidualEpi" in name or "ResidualPartsEpi" in name:
        return "down" if previous == "gate_up" else "o_proj"
    return None


def summarize_counters(root: pathlib.Path, which: str) -> str:
    """Per-kernel figures of one decode step from rocprofv3 CSVs: kernel-trace durations,
    FETCH_SIZE and WRITE_SIZE scaled by what they read for a 256 MiB copy, the L2 hit rate."""
    import csv
    from collections import defaultdict

    sys.path.insert(0, str(ROOT / "muyo-llm_amd"))
    import muyo_hip as mh

    shape = dict(mh.QWEN25_05B if which == "05b" else mh.QWEN25_7B)
    position = 1024 if which == "05b" else 2040

    def rows(sub: str, suffix: str):
        files = sorted((root / sub).rglob(f"*{suffix}"))
        if not files:
            raise SystemExit(f"no *{suffix} under {root / sub}")
        with open(files[0], newline="") as fh:
            return sorted(csv.DictReader(fh), key=lambda r: int(r["Dispatch_Id"]))

    def classify(records):
        kinds, previous = {}, None
        for r in records:
            k = step_kind(r["Kernel_Name"], previous)
            if k is not None:
                kinds[int(r["Dispatch_Id"])] = k
                previous = k
        return kinds

    def counter_means(sub: str, names):
        recs = rows(sub, "counter_collection.csv")
        kinds = classify(recs)
        acc = defaultdict(lambda: defaultdict(list))
        for r in recs:
            k = kinds.get(int(r["Dispatch_Id"]))
            if k is not None and r["Counter_Name"] in names:
                acc[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
        return {k: {n: sum(v) / len(v) for n, v in d.items()} for k, d in acc.items()}

    def copy_mean(sub: str, name: str) -> float:
        vals = [float(r["Counter_Value"]) for r in rows(sub, "counter_collection.csv")
                if "copyBuffer" in r["Kernel_Name"] and r["Counter_Name"] == name]
        return sum(vals) / len(vals)

    copy_kib = 2 * 4 * 64 * 1024 * 1024 / 2 / 1024  # 256 MiB read, 256 MiB written
    fetch_scale = copy_kib / copy_mean("copy_fetch", "FETCH_SIZE")
    write_scale = copy_kib / copy_mean("copy_write", "WRITE_SIZE")

    trace = rows("trace", "kernel_trace.csv")
    kinds = classify(trace)
    durations = defaultdict(list)
    for r in trace:
        k = kinds.get(int(r["Dispatch_Id"]))
        if k is not None:
            durations[k].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    fetch = counter_means("fetch", {"FETCH_SIZE"})
    write = counter_means("write", {"WRITE_SIZE"})
    hits = counter_means("hit", {"TCC_HIT_sum", "TCC_MISS_sum"})
    steps = len(durations["lm_head"])
    per_step = {"embed": 1, "qkv": shape["layers"], "attention": shape["layers"], "merge": shape["layers"],
                "o_proj": shape["layers"], "lm_head": 1}
    for kind in ("GATE_UP", "DOWN", "FFN"):
        per_step[kind.lower()] = sum(kind in layer_kinds(shape, layer) for layer in range(shape["layers"]))
    lines = [f"fetch scale {fetch_scale:.4f}, write scale {write_scale:.4f} (256 MiB copy); {steps} steps",
             "",
             "| kernel | launches/step | avg µs | µs/step | share | algorithmic bytes | counter bytes | "
             "counter/alg | GB/s (alg) | % of 8 TB/s | L2 hit rate |",
             "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    total = sum(per_step[k] * sum(v) / len(v) for k, v in durations.items())
    for k in ("embed", "qkv", "attention", "merge", "o_proj", "ffn", "gate_up", "down", "lm_head"):
        if k not in durations:
            continue
        us = sum(durations[k]) / len(durations[k])
        alg = kernel_bytes(shape, k, position) if k != "embed" else kernel_bytes(shape, k, 0)
        got = (fetch.get(k, {}).get("FETCH_SIZE", 0.0) * fetch_scale + write.get(k, {}).get("WRITE_SIZE", 0.0)
               * write_scale) * 1024
        hit = hits.get(k, {})
        rate = hit.get("TCC_HIT_sum", 0.0) / max(1.0, hit.get("TCC_HIT_sum", 0.0) + hit.get("TCC_MISS_sum", 0.0))
        gbs = alg / (us * 1e-6) / 1e9
        lines.append(f"| {k} | {per_step[k]} | {us:.2f} | {per_step[k] * us:.1f} | {100 * per_step[k] * us / total:.1f} % "
                     f"| {alg:,} | {got:,.0f} | {got / alg:.3f} | {gbs:,.0f} | {100 * gbs / HBM_PEAK_GBS:.1f} | {rate:.3f} |")
    lines.append(f"| step (sum of kernels) | | | {total:.1f} | | | | | | | |")
    return "\n".join(lines)


def summarize_ops(root: pathlib.Path) -> str:
    """Per-launcher figures of the per-op suite from rocprofv3 CSVs of `--ops-only` runs kept under
    root (trace/, fetch/, write/, hit/, copy_fetch/, copy_write/, and ops.json, the trace run's
    JSON line): kernel-trace durations, FETCH_SIZE and WRITE_SIZE scaled by what they read for a
    256 MiB copy, the L2 hit rate. The suite runs its launchers in a fixed order, each launch
    eagerly once and then from a replayed hipGraph; the fills between them are left out."""
    import csv
    from collections import defaultdict

    ops = json.loads((root / "ops.json").read_text())["kernels"]
    names = list(ops)

    def rows(sub: str, suffix: str):
        files = sorted((root / sub).rglob(f"*{suffix}"))
        if not files:
            raise SystemExit(f"no *{suffix} under {root / sub}")
        with open(files[0], newline="") as fh:
            return sorted(csv.DictReader(fh), key=lambda r: int(r["Dispatch_Id"]))

    def segment(records):
        """Dispatch id -> op name: runs of one (kernel, grid) between fills, in suite order."""
        runs, last = [], None
        for r in records:
            kname = r["Kernel_Name"]
            if "FillNormal" in kname or kname.startswith("void at::native") or kname.startswith("at::native"):
                continue
            key = (kname, r.get("Grid_Size_X") or r.get("Grid_Size"))
            if key != last:
                runs.append([])
                last = key
            runs[-1].append(int(r["Dispatch_Id"]))
        if len(runs) != len(names):
            raise SystemExit(f"{len(runs)} launcher runs in the trace, {len(names)} ops in ops.json")
        return {d: name for name, ids in zip(names, runs) for d in ids}

    def counter_means(sub: str, counters):
        recs = rows(sub, "counter_collection.csv")
        # One record per (dispatch, counter): segment on the distinct dispatches.
        seen, firsts = set(), []
        for r in recs:
            if r["Dispatch_Id"] not in seen:
                seen.add(r["Dispatch_Id"])
                firsts.append(r)
        which = segment(firsts)
        acc = defaultdict(lambda: defaultdict(list))
        for r in recs:
            name = which.get(int(r["Dispatch_Id"]))
            if name is not None and r["Counter_Name"] in counters:
                acc[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
        return {n: {c: sum(v) / len(v) for c, v in d.items()} for n, d in acc.items()}

    def copy_mean(sub: str, name: str) -> float:
        vals = [float(r["Counter_Value"]) for r in rows(sub, "counter_collection.csv")
                if "copyBuffer" in r["Kernel_Name"] and r["Counter_Name"] == name]
        return sum(vals) / len(vals)

    copy_kib = 2 * 4 * 64 * 1024 * 1024 / 2 / 1024  # 256 MiB read, 256 MiB written
    fetch_scale = copy_kib / copy_mean("copy_fetch", "FETCH_SIZE")
    write_scale = copy_kib / copy_mean("copy_write", "WRITE_SIZE")
    trace = rows("trace", "kernel_trace.csv")
    which = segment(trace)
    durations = defaultdict(list)
    for r in trace:
        name = which.get(int(r["Dispatch_Id"]))
        if name is not None:
            durations[name].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    fetch = counter_means("fetch", {"FETCH_SIZE"})
    write = counter_means("write", {"WRITE_SIZE"})
    hits = counter_means("hit", {"TCC_HIT_sum", "TCC_MISS_sum"})
    lines = [f"fetch scale {fetch_scale:.4f}, write scale {write_scale:.4f} (256 MiB copy)",
             "",
             "| launcher | dispatches | avg µs | algorithmic bytes | counter bytes | counter/alg | GB/s (alg) | "
             "% of 8 TB/s | L2 hit rate | copies rotated |",
             "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for name in names:
        us = sum(durations[name]) / len(durations[name])
        alg = ops[name]["bytes_per_launch"]
        got = (fetch.get(name, {}).get("FETCH_SIZE", 0.0) * fetch_scale + write.get(name, {}).get("WRITE_SIZE", 0.0)
               * write_scale) * 1024
        hit = hits.get(name, {})
        rate = hit.get("TCC_HIT_sum", 0.0) / max(1.0, hit.get("TCC_HIT_sum", 0.0) + hit.get("TCC_MISS_sum", 0.0))
        gbs = alg / (us * 1e-6) / 1e9
        lines.append(f"| {name} | {len(durations[name])} | {us:.2f} | {alg:,} | {got:,.0f} | {got / alg:.3f} | "
                     f"{gbs:,.0f} | {100 * gbs / HBM_PEAK_GBS:.1f} | {rate:.3f} | {ops[name]['rotated_copies']} |")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--position", type=int, default=1024)
    ap.add_argument("--cpu-samples", type=int, default=10, help="timed CPU-baseline steps per variant (median)")
    ap.add_argument("--no-ops", action="store_true", help="skip the per-op launcher suite")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-7b", action="store_true", help="skip the 7B-shape secondary figure")
    ap.add_argument("--floor", choices=["05b", "7b"],
                    help="only the step beside its streaming floor (a chain of pure-read kernels with the step's "
                         "launch count and bytes) and the per-phase kernels beside pure streams of their bytes")
    ap.add_argument("--launch-floor", choices=["05b", "7b"],
                    help="only the kernel-boundary measurements (muyo-llm_amd/launch_floor): hipGraph and raw AQL "
                         "chains of empty kernels by fence scope, and the step's launch sequence as pure streams and "
                         "with activation hand-offs under each fence and coherence scheme")
    ap.add_argument("--kernel-only", choices=["lm_head", "copy", "step_05b", "step_7b"],
                    help="only launch one kernel back to back, or whole decode steps kernel by kernel "
                         "(0.5B shape from cache row 1024, 7B shape from row 2040), for rocprofv3")
    ap.add_argument("--summarize-counters", metavar="DIR",
                    help="print the per-kernel table of a step's rocprofv3 runs kept under DIR "
                         "(trace/, fetch/, write/, hit/, copy_fetch/, copy_write/) and exit")
    ap.add_argument("--shape", choices=["05b", "7b"], default="05b", help="shape for --summarize-counters")
    ap.add_argument("--summarize-ops", metavar="DIR",
                    help="print the per-launcher table of the per-op suite's rocprofv3 runs kept under DIR "
                         "(trace/, fetch/, write/, hit/, copy_fetch/, copy_write/, ops.json) and exit")
    ap.add_argument("--launches", type=int, default=20, help="launches for --kernel-only")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the batched-prefill figures (2048-token prompts, 0.5B and 7B shapes)")
    ap.add_argument("--ops-only", action="store_true",
                    help="only the per-op launcher suite (element-wise and reduction set, GEMV suite), for rocprofv3")
    args = ap.parse_args()

    if args.summarize_counters:
        print(summarize_counters(pathlib.Path(args.summarize_counters), args.shape), flush=True)
        return 0
    if args.summarize_ops:
        print(summarize_ops(pathlib.Path(args.summarize_ops)), flush=True)
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); the decode "
              "path is single-GPU by design and multi-GPU figures are not produced.", file=sys.stderr)
        return 2

    import muyo_hip as mh

    if args.launch_floor:
        print(json.dumps(launch_floor_report(mh, args.launch_floor)), flush=True)
        return 0

    import torch

    torch.cuda.set_device(0)
    mh.load()
    if args.kernel_only:
        print(json.dumps(kernel_only(mh, torch, args.kernel_only, args.launches)), flush=True)
        return 0
    if args.floor:
        print(json.dumps(floor_report(mh, torch, args.floor)), flush=True)
        return 0
    if args.ops_only:
        print(json.dumps({"kernels": time_ops(mh, torch, reps=3)}), flush=True)
        return 0
    shape = dict(mh.QWEN25_05B)
    seed = 20261201
    if args.prefill_only:
        lines = {"qwen2.5-0.5b-shape-prefill": prefill_line(mh, torch, shape, 2048, 5, seed, None)}
        if not args.no_7b:
            lines["qwen2.5-7b-shape-prefill"] = prefill_line(mh, torch, dict(mh.QWEN25_7B), 2048, 3, seed + 7, None)
        print(json.dumps(lines), flush=True)
        return 0

    ms, positions, launches, ids, median_ms = time_decode(mh, torch, shape, args.position, args.steps, args.warmup,
                                                          seed)
    total_bytes = sum(step_bytes(shape, p) for p in positions)
    value = total_bytes / (ms * 1e-3 * args.steps) / 1e9

    kern = time_kernels(mh, torch, shape, seed, rounds=64)
    # Each kernel kind of the step, graph-replayed over the 24 layers at the timed window's middle
    # row: the roofline kernel's share of the step comes from these, not from a profile.
    phases = time_phases(mh, torch, shape, positions[len(positions) // 2], seed)
    ops = {} if args.no_ops else time_ops(mh, torch)
    lm_gbs = lm_head_bytes(shape) / (kern["lm_head_ms"] * 1e-3) / 1e9
    assert ffn_fused(shape) and kern["roofline_kind"] == "FFN", kern["roofline_kind"]
    assert launches == len(chain_bytes_of(shape, positions[0])), launches
    ffn_gbs = ffn_bytes(shape) / (kern["roofline_ms"] * 1e-3) / 1e9
    ffn_layers = len(kind_layers(shape)["FFN"])

    secondary = {}
    # The same decode with the device sampler after every step (the reference's sampling options
    # at common settings plus a repetition penalty): its cost per token over greedy.
    sampling = dict(temperature=0.7, top_k=40, top_p=0.95, repeat_penalty=1.1, repeat_last_n=64, seed=seed)
    ms_s, _, launches_s, _, _ = time_decode(mh, torch, shape, args.position, args.steps, args.warmup, seed,
                                            sampling)
    secondary["qwen2.5-0.5b-shape-sampled"] = {
        "sampler": sampling, "tok_per_s": round(1000.0 / ms_s, 1), "ms_per_step": round(ms_s, 5),
        "sampler_ms_per_token": round(ms_s - ms, 5), "launches_per_step": launches_s,
    }
    # Batched prefill of a 2048-token prompt, against feeding it one decode step per token (the
    # reference's feedToken loop) at this run's decode rate.
    secondary["qwen2.5-0.5b-shape-prefill"] = prefill_line(mh, torch, shape, 2048, 5, seed, ms)
    if not args.no_7b:
        shape7 = dict(mh.QWEN25_7B)
        steps7 = 16
        ms7, pos7, _, _, median7 = time_decode(mh, torch, shape7, 2048 - steps7 // 2, steps7, 4, seed + 7)
        bytes7 = sum(step_bytes(shape7, p) for p in pos7)
        gbs7 = bytes7 / (ms7 * 1e-3 * steps7) / 1e9
        secondary["qwen2.5-7b-shape"] = {
            "GB/s": round(gbs7, 1), "pct_of_peak": round(100 * gbs7 / HBM_PEAK_GBS, 1),
            "tok_per_s": round(1000.0 / ms7, 1), "ms_per_step": round(ms7, 4), "ms_per_step_median": round(median7, 4),
            "positions": f"{pos7[0]}..{pos7[-1]}", "bytes_per_step": bytes7 // steps7,
        }
        secondary["qwen2.5-7b-shape-prefill"] = prefill_line(mh, torch, shape7, 2048, 3, seed + 7, ms7)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "ms_per_step_median": round(median_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "qwen2.5-0.5b-shape greedy decode step, fp16 weights + fp16 KV cache, f32 accumulate",
            "layers": shape["layers"], "hidden": shape["hidden"], "ffn": shape["ffn"], "heads": shape["heads"],
            "kv_heads": shape["kv_heads"], "head_dim": shape["head_dim"], "vocab": shape["vocab"],
            "max_seq": shape["max_seq"], "positions": f"{positions[0]}..{positions[-1]}",
            "weights_dtype": "f16", "launches_per_step": launches,
        },
        "tok_per_s": round(1000.0 / ms, 1),
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "bytes_per_step": total_bytes // args.steps,
        "roofline": {
            "kernel": "FfnFusedKernel (ffn_norm + gate/up 2x4864x896 + swiglu + down 896x4864 from transposed "
                      "weights, added into the hidden state's partial vectors)",
            "bound": "hbm",
            "achieved": round(ffn_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(ffn_gbs / HBM_PEAK_GBS, 4),
            "traffic": FFN_TRAFFIC_BYTES,
            "l2_hit_rate": FFN_L2_HIT_RATE,
            "traffic_source": FFN_COUNTER_SOURCE,
            "launch_ms": round(kern["roofline_ms"], 5),
            "bytes_per_launch": ffn_bytes(shape),
            "share_of_step": round(phases["ffn"] * ffn_layers / (ms * 1000.0), 3),
            "note": f"rotated over the {ffn_layers} fused layers' weights "
                    f"({ffn_layers * ffn_bytes(shape) / 1e6:.0f} MB > MALL)",
        },
        "kernels": {
            "lm_head": {"GB/s": round(lm_gbs, 1), "launch_ms": round(kern["lm_head_ms"], 5),
                        "bytes_per_launch": lm_head_bytes(shape), "frac": round(lm_gbs / HBM_PEAK_GBS, 4)},
            **ops,
        },
        "phases_us": {k: round(v, 2) for k, v in phases.items()},
        "secondary": secondary,
        "greedy_ids_head": ids[:8],
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(shape, args.position, max(10, args.cpu_samples), seed)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
