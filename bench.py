#!/usr/bin/env python3
"""Decode-step benchmark on one MI355X.

Workload: one greedy decode step of a Qwen2.5-0.5B-shaped model (24 layers, hidden 896, ffn
4864, 14/2 heads, head_dim 64, tied vocab 151936), fp16 weights N(0, 0.02) from the portable
seeded generator, fp16 KV cache pre-filled with N(0, 1), steps centred on cache position 1024.
A "step" is one token: embed -> 24 x (norm+QKV+rope+append, attention, o_proj+residual,
norm+gate/up+swiglu, down+residual) -> norm + LM head + argmax, replayed as one hipGraph with the
greedy id fed back on the device. Inputs are resident in HBM before the timed region.

value = algorithmic HBM bytes of the timed steps / time (GB/s): every weight once as fp16, the KV
rows 0..p read once as fp16, the appended rows written, activations as f32 once per kernel that
reads or writes them. tok/s is reported beside it.

roofline: the LM-head kernel (rms_norm prologue + 151936 x 896 fp16 GEMV + argmax; the largest
single launch, 272 MB, bigger than the 256 MB MALL), timed alone with HIP events on its stream.

cpu_baseline: the CPU oracle's decode step (oracle/, a C restatement of the reference's CPU
path) on one host core, over a bounded sample of steps of the same workload.
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
# HBM bytes per LM-head launch from rocprofv3 FETCH_SIZE / WRITE_SIZE, each scaled by what the
# counter reads for a 256 MiB device copy (profiles/lm_head_0.5b_pmc.md), and the L2 hit rate
# (TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum)) of the same runs.
LM_HEAD_TRAFFIC_BYTES = 273_149_422
LM_HEAD_L2_HIT_RATE = 0.105


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


def time_decode(mh, torch, shape, position, steps, warmup, seed):
    """Returns (ms per step, positions timed, decoder launches per step)."""
    stream = torch.cuda.current_stream()
    start = max(1, position - steps // 2 - warmup)
    dec = mh.Decoder(mh.qwen2_config(**shape))
    try:
        dec.fill_random(seed)
        dec.fill_kv_random(start, seed + 1)
        token = 9707
        dec.generate_async(token, start, warmup, stream.cuda_stream)
        torch.cuda.synchronize()
        warm_ids = dec.generated_ids(warmup)
        first = start + warmup
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        begin.record(stream)
        dec.generate_async(warm_ids[-1], first, steps, stream.cuda_stream)
        end.record(stream)
        torch.cuda.synchronize()
        ms = begin.elapsed_time(end) / steps
        ids = dec.generated_ids(steps)
        launches = dec.launches_per_step()
    finally:
        dec.close()
    return ms, list(range(first, first + steps)), launches, ids


def time_kernels(mh, torch, shape, seed, rounds):
    """Per-launch ms of the LM-head kernel and of the gate/up kernel rotated over all layers."""
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
        torch.cuda.synchronize()
        b.record(stream)
        for _ in range(rounds):
            dec.enqueue_kernel("LM_HEAD", 0, s)
        e.record(stream)
        torch.cuda.synchronize()
        out["lm_head_ms"] = b.elapsed_time(e) / rounds
        for layer in range(shape["layers"]):
            dec.enqueue_kernel("GATE_UP", layer, s)
        torch.cuda.synchronize()
        b.record(stream)
        for _ in range(max(1, rounds // 4)):
            for layer in range(shape["layers"]):
                dec.enqueue_kernel("GATE_UP", layer, s)
        e.record(stream)
        torch.cuda.synchronize()
        out["gate_up_ms"] = b.elapsed_time(e) / (max(1, rounds // 4) * shape["layers"])
    finally:
        dec.close()
    return out


def cpu_baseline(shape, position, seconds, seed):
    """The CPU oracle's decode step on one core over a bounded sample (TEST INFRASTRUCTURE path)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    oracle.set_threads(min(16, os.cpu_count() or 1))
    model = oracle.Model(**shape)
    model.fill_random(seed)
    model.fill_kv_random(position, seed + 1)
    oracle.set_threads(1)
    token, done, t0 = 9707, 0, time.perf_counter()
    positions = []
    while True:
        token, _, _ = model.step(token, position + done)
        positions.append(position + done)
        done += 1
        if time.perf_counter() - t0 >= seconds or position + done >= shape["max_seq"]:
            break
    elapsed = time.perf_counter() - t0
    total = sum(step_bytes(shape, p) for p in positions)
    return {
        "value": round(total / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{done} decode steps of the same 0.5B-shape workload at cache rows {positions[0]}..{positions[-1]} "
                  f"({elapsed:.1f} s, {done / elapsed:.3f} tok/s, double-accumulating C oracle, -O2, 1 thread)",
        "tok_per_s": round(done / elapsed, 4),
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
    else:
        raise ValueError(which)
    ms = b.elapsed_time(e) / launches
    return {"kernel": which, "launches": launches, "avg_ms": round(ms, 5), "bytes_per_launch": nbytes,
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--position", type=int, default=1024)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-7b", action="store_true", help="skip the 7B-shape secondary figure")
    ap.add_argument("--kernel-only", choices=["lm_head", "copy"],
                    help="only launch one kernel back to back (for rocprofv3 traces and counters)")
    ap.add_argument("--launches", type=int, default=20, help="launches for --kernel-only")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); the decode "
              "path is single-GPU by design and multi-GPU figures are not produced.", file=sys.stderr)
        return 2

    import torch

    import muyo_hip as mh

    torch.cuda.set_device(0)
    mh.load()
    if args.kernel_only:
        print(json.dumps(kernel_only(mh, torch, args.kernel_only, args.launches)), flush=True)
        return 0
    shape = dict(mh.QWEN25_05B)
    seed = 20261201

    ms, positions, launches, ids = time_decode(mh, torch, shape, args.position, args.steps, args.warmup, seed)
    total_bytes = sum(step_bytes(shape, p) for p in positions)
    value = total_bytes / (ms * 1e-3 * args.steps) / 1e9

    kern = time_kernels(mh, torch, shape, seed, rounds=64)
    lm_gbs = lm_head_bytes(shape) / (kern["lm_head_ms"] * 1e-3) / 1e9
    gu_gbs = gate_up_bytes(shape) / (kern["gate_up_ms"] * 1e-3) / 1e9

    secondary = {}
    if not args.no_7b:
        shape7 = dict(mh.QWEN25_7B)
        steps7 = 16
        ms7, pos7, _, _ = time_decode(mh, torch, shape7, 2048 - steps7 // 2, steps7, 4, seed + 7)
        bytes7 = sum(step_bytes(shape7, p) for p in pos7)
        gbs7 = bytes7 / (ms7 * 1e-3 * steps7) / 1e9
        secondary["qwen2.5-7b-shape"] = {
            "GB/s": round(gbs7, 1), "pct_of_peak": round(100 * gbs7 / HBM_PEAK_GBS, 1),
            "tok_per_s": round(1000.0 / ms7, 1), "ms_per_step": round(ms7, 4),
            "positions": f"{pos7[0]}..{pos7[-1]}", "bytes_per_step": bytes7 // steps7,
        }

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
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
            "kernel": "FusedMatVec<16,8,1,true,NormStage,LmHeadEpi> (final norm + tied LM head 151936x896 + argmax)",
            "bound": "hbm",
            "achieved": round(lm_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(lm_gbs / HBM_PEAK_GBS, 4),
            "traffic": LM_HEAD_TRAFFIC_BYTES,
            "l2_hit_rate": LM_HEAD_L2_HIT_RATE,
            "launch_ms": round(kern["lm_head_ms"], 5),
            "bytes_per_launch": lm_head_bytes(shape),
        },
        "kernels": {
            "gate_up_swiglu": {"GB/s": round(gu_gbs, 1), "launch_ms": round(kern["gate_up_ms"], 5),
                               "bytes_per_launch": gate_up_bytes(shape),
                               "note": "rotated over the 24 layers' weights (420 MB > MALL)"},
        },
        "secondary": secondary,
        "greedy_ids_head": ids[:8],
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(shape, args.position, args.cpu_seconds, seed)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
