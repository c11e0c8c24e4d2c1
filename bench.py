#!/usr/bin/env python3
"""Benchmark: E8-D4 fused decode matvec on synthetic Llama-2-7B layers, one MI355X.

Workload (batch 1): the seven quantized Linears of
every one of Llama-2-7B's 32 decoder layers — q/k/v/o 4096x4096, gate/up
11008x4096, down 4096x11008 — E8-D4 codebook at radius 1.75, 0.1% critical
blocks, seeded synthetic indices and scales.  One step = one token's worth of
quantized-Linear work: 224 launches over 32 distinct layers (1.66 GB of
algorithmic bytes, far above the 256 MB MALL, so the bytes come from HBM).
The step is captured once in a HIP graph and replayed.

Reported: ``value`` = algorithmic GB/s over the timed steps (inputs resident
in HBM), ``roofline`` for the matvec kernel (algorithmic bytes per launch over
its average launch duration measured with HIP events on the launch stream),
and ``cpu_baseline`` = the reference CPU path (dequantize_layer restatement +
fp32 matmul) on one q_proj layer, timed on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "dequant-matvec GB/s (% HBM peak); tok/s synthetic Llama-2-7B bs=1"
HBM_PEAK_GBS = 8000.0
LLAMA2_7B = [("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
             ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]


def algo_bytes(out, inp, B, nnz, bias=False, n_groups=0):
    """Algorithmic bytes of one decode call, each operand counted once:
    Q 2MN + S 2GN + CSR (16+4)nnz + 4(M+1) + g 2out + h 2in + bias + x 2B·in + y 2B·out."""
    M = out // 8
    return (2 * M * inp + 2 * n_groups * inp + 20 * nnz + 4 * (M + 1) + 2 * out + 2 * inp
            + (2 * out if bias else 0) + 2 * B * inp + 2 * B * out)


def cpu_baseline(seed=1000):
    """Reference CPU path on one Llama-2-7B q_proj at B=1: the per-column
    dequantize_layer restatement (algorithms/eptq.py:406-471) + fp32 matmul."""
    import torch
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer, make_x
    from oracle.dequant import dequantize_layer_torch_loop

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    qd = make_layer(4096, 4096, seed=seed, percmask=0.001)
    x = make_x(1, 4096, seed=seed + 1)
    tab = E8D4Quantizer(radius=1.75).flat_table().numpy()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        W = dequantize_layer_torch_loop(qd.Q.numpy(), qd.g.numpy(), qd.h.numpy(), qd.O.numpy(),
                                        tab, "e8_d4")
        y = torch.matmul(x.float(), W.float().T)
        times.append(time.perf_counter() - t0)
    del y
    t = statistics.median(times)
    nbytes = algo_bytes(4096, 4096, 1, qd.O.shape[0])
    return {"value": round(nbytes / t / 1e9, 6), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"one q_proj 4096x4096 B=1 (E8-D4 r=1.75, p=0.001): per-column "
                      f"dequantize_layer + fp32 torch.matmul, median of 3 = {t:.3f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the quantized Linear is a single-GPU kernel; sharding is a design note).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from eptq_amd.kernels import _lib
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer, make_x

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B = args.batch
    codes = E8D4Quantizer(radius=1.75).flat_table().half().to(dev)

    def csr(Q):
        rows, cols = (Q == 32767).nonzero(as_tuple=True)
        counts = torch.bincount(rows, minlength=Q.shape[0])
        rp = torch.cat([torch.zeros(1, dtype=torch.int32, device=dev), counts.cumsum(0).to(torch.int32)])
        return cols.to(torch.int32), rp

    t0 = time.time()
    layers = []
    for li in range(args.layers):
        for idx, (name, out, inp) in enumerate(LLAMA2_7B):
            qd = make_layer(out, inp, seed=1000 + 10 * li + idx, percmask=0.001, device=dev)
            ocol, orp = csr(qd.Q)
            layers.append(dict(name=name, out=out, inp=inp, Q=qd.Q, g=qd.g, h=qd.h,
                               O=qd.O, O_col=ocol, O_row_ptr=orp, nnz=int(qd.O.shape[0])))
    xs = {inp: make_x(B, inp, seed=7 + inp, device=dev) for inp in {l["inp"] for l in layers}}
    ys = {out: torch.empty((B, out), dtype=torch.float16, device=dev) for out in {l["out"] for l in layers}}
    torch.cuda.synchronize()
    print(f"# generated {len(layers)} layers in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    step_bytes = sum(algo_bytes(l["out"], l["inp"], B, l["nnz"]) for l in layers)

    def launch(l, stream):
        _lib.forward_into("e8_d4", l["Q"], codes, l["g"], l["h"], xs[l["inp"]], l["O"],
                          l["O_col"], l["O_row_ptr"], None, None, ys[l["out"]], stream)

    def run_step(stream):
        for l in layers:
            launch(l, stream)

    # Per-launch kernel durations with HIP events on the launch stream.
    cur = torch.cuda.current_stream()
    run_step(cur.cuda_stream)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in layers]
    per_launch = [0.0] * len(layers)
    reps = 3
    for _ in range(reps):
        for i, l in enumerate(layers):
            evs[i][0].record(cur)
            launch(l, cur.cuda_stream)
            evs[i][1].record(cur)
        torch.cuda.synchronize()
        for i in range(len(layers)):
            per_launch[i] += evs[i][0].elapsed_time(evs[i][1]) / reps
    kern_ms = sum(per_launch)
    per_shape = {}
    for i, l in enumerate(layers):
        d = per_shape.setdefault(l["name"], {"shape": f"{l['out']}x{l['inp']}", "us": 0.0, "n": 0, "bytes": 0})
        d["us"] += per_launch[i] * 1e3
        d["n"] += 1
        d["bytes"] += algo_bytes(l["out"], l["inp"], B, l["nnz"])
    for d in per_shape.values():
        d["gbs"] = round(d["bytes"] / (d["us"] * 1e-6) / 1e9, 1)
        d["us"] = round(d["us"] / d["n"], 3)
        del d["bytes"], d["n"]

    # Capture one step in a graph and replay it.
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        run_step(side.cuda_stream)
    cur.wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run_step(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    value = step_bytes / (ms * 1e-3) / 1e9

    achieved = step_bytes / (kern_ms * 1e-3) / 1e9
    rec = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "llama2_7b_decoder_linears_decode", "batch": B,
                   "layers": args.layers, "linears_per_step": len(layers),
                   "codebook": "e8_d4", "radius": 1.75, "percmask": 0.001,
                   "algorithmic_bytes_per_step": step_bytes, "hip_graph": True},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_matvec<E8D4,BT=1>",
                     "avg_launch_us": round(kern_ms * 1e3 / len(layers), 3),
                     "algorithmic_bytes_per_launch": round(step_bytes / len(layers))},
        "per_shape": per_shape,
    }
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline()
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
