#!/usr/bin/env python3
"""Benchmark: E8-D4 fused decode matvec on synthetic Llama-2-7B layers, one MI355X.

Workload (``config.workload`` = llama2_7b_decoder_linears_decode; benchmark
configuration 1 at batch 1): the seven quantized Linears of each of
Llama-2-7B's 32 decoder layers — q/k/v/o 4096x4096, gate/up 11008x4096, down
4096x11008 — E8-D4 codebook at radius 1.75, 0.1% critical blocks, seeded
synthetic indices and scales, generated on the GPU.  One step = one token's
quantized-Linear work over 224 distinct layers (1.66 GB of algorithmic bytes,
far above the 256 MB MALL, so the bytes stream from HBM), launched as a
decode step does: per decoder layer q|k|v and gate|up as multi-layer launches
(each layer with its own scales) and o, down alone — 128 launches.  The step
is captured once in a HIP graph and replayed ``--steps`` times; the same 224
Linears as 224 separate launches are reported beside it.

JSON fields beyond the driver contract:

* ``roofline`` — the decode kernel: algorithmic bytes per launch (mean over
  the 128 launches) over the mean launch duration, which is the HIP-event time
  of the timed graph replays (recorded on the stream the graph is launched
  on) divided by the launches they hold; every launch in the step is this
  kernel.  ``per_shape`` times each shape's 32 launches back to back with
  events around the group and the queue backed up by a device sleep.  ``traffic`` = HBM bytes
  per launch from two ``rocprofv3 --pmc`` passes (FETCH_SIZE, WRITE_SIZE) over
  one step, each scaled by the same counter's reading for a 512 MiB device
  copy; the passes run as child processes before this process touches the GPU.
* ``e2e`` — tokens/s of the synthetic Llama-2-7B (every decoder Linear a
  synthetic E8-D4 layer, benchmark configuration 4): 128-token prompt, greedy
  decode, graph-captured step, prefill untimed, batch 1 and 8.
* ``decode_batches`` — the decode-step Linear units (q|k|v, o, gate|up,
  down) of Llama-2-7B at batch 1 and 8 (benchmark configuration 1) and of
  Llama-3-8B with S_group qb=128 at batch 1, 4 and 16 (configuration 2), one
  launch each with the decode workspace: microseconds and algorithmic GB/s.
  Batches of 3..16 run the matrix-core decode kernel.
* ``prefill`` — the Llama-2-13B shapes at 2048 tokens (benchmark
  configuration 3): ``fused`` (the dequantize-into-LDS MFMA GEMM, which the
  C ABI and the module forward run) and, as a yardstick only,
  ``dequant_library_gemm`` (the bit-exact dequantization kernel into an fp16
  W, then torch's library fp16 GEMM; no product path runs it); TFLOP/s and
  fraction of the 2.5 PFLOP/s fp16 dense MFMA peak.
* ``dequant`` — the bit-exact dequantizer (``eptq_e8d4_dequant``, fp16 W of
  ``dequantize_layer``) on the Llama-2-7B shapes: algorithmic GB/s (index
  and scale reads plus the W write) and fraction of HBM peak.
* ``config0`` — benchmark configuration 0, the E8-lattice Linear at OPT-125m
  fc1 shape (3072x768) with bias at batch 1: microseconds per launch over
  distinct copies, algorithmic GB/s and fraction of HBM peak.
* ``cpu_baseline`` — the reference CPU path (per-column ``dequantize_layer``
  restatement + fp32 ``torch.matmul``) on a 4096x4096 and an 11008x4096
  Linear at batch 1, dequant and matmul timed separately (median of 5), on
  this host's cores.  ``--cpu-configs`` adds ``cpu_configs``: the same
  per layer and batch of configurations 0-3.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import shutil
import signal
import statistics
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "dequant-matvec GB/s (% HBM peak); tok/s synthetic Llama-2-7B bs=1"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
LLAMA2_7B = [("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
             ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]
LLAMA2_13B = [("qkvo", 5120, 5120), ("gate_up", 13824, 5120), ("down", 5120, 13824)]
DECODE_KERNEL = "k_decode_e8d4"
CALIB_BYTES = 512 << 20


def algo_bytes(out, inp, B, nnz, bias=False, n_groups=0):
    """Algorithmic bytes of one decode call, each operand counted once:
    Q 2MN + S 2GN + CSR (16+4)nnz + 4(M+1) + g 2out + h 2in + bias + x 2B·in + y 2B·out."""
    M = out // 8
    return (2 * M * inp + 2 * n_groups * inp + 20 * nnz + 4 * (M + 1) + 2 * out + 2 * inp
            + (2 * out if bias else 0) + 2 * B * inp + 2 * B * out)


# ---------------------------------------------------------------------------
# Workload
# ---------------------------------------------------------------------------

def make_workload(torch, dev, n_layers, B):
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer, make_x

    codes = E8D4Quantizer(radius=1.75).flat_table().half().to(dev)

    def csr(Q):
        rows, cols = (Q == 32767).nonzero(as_tuple=True)
        counts = torch.bincount(rows, minlength=Q.shape[0])
        rp = torch.cat([torch.zeros(1, dtype=torch.int32, device=dev), counts.cumsum(0).to(torch.int32)])
        return cols.to(torch.int32), rp

    layers = []
    for li in range(n_layers):
        for idx, (name, out, inp) in enumerate(LLAMA2_7B):
            qd = make_layer(out, inp, seed=1000 + 10 * li + idx, percmask=0.001, device=dev)
            ocol, orp = csr(qd.Q)
            layers.append(dict(name=name, out=out, inp=inp, Q=qd.Q, g=qd.g, h=qd.h,
                               O=qd.O, O_col=ocol, O_row_ptr=orp, nnz=int(qd.O.shape[0])))
    xs = {inp: make_x(B, inp, seed=7 + inp, device=dev) for inp in {l["inp"] for l in layers}}
    ys = {out: torch.empty((B, out), dtype=torch.float16, device=dev) for out in {l["out"] for l in layers}}
    return codes, layers, xs, ys


def make_launcher(codes, xs, ys):
    """Return launch(layer, stream) with argument pointers resolved once per layer."""
    from eptq_amd.kernels import _lib
    lib = _lib.load()
    fn = lib.eptq_e8d4_forward

    def p(t):
        return None if t is None or t.numel() == 0 else t.data_ptr()

    def launch(l, stream):
        args = l.get("_args")
        if args is None:
            x, y = xs[l["inp"]], ys[l["out"]]
            args = (p(l["Q"]), p(codes), _lib.EPTQ_F16, p(l["g"]), p(l["h"]), p(x), _lib.EPTQ_F16,
                    p(l["O"]), p(l["O_col"]), p(l["O_row_ptr"]), None, None, 0,
                    int(l["Q"].shape[0]), int(l["Q"].shape[1]), int(x.shape[0]), p(y))
            l["_args"] = args
        rc = fn(*args, stream)
        if rc:
            _lib.check(rc, "eptq_e8d4_forward")

    return launch


def make_units(torch, codes, layers, xs, B):
    """The launches of a decode step: per decoder layer q|k|v and gate|up as
    multi-layer launches (each layer keeps its own scales), o and down alone.
    Returns [(launch(stream), [layers])]."""
    from eptq_amd.kernels import _lib
    lib = _lib.load()
    units, i = [], 0
    # Split-K workspace of the matrix-core decode (batches of 3..16); the
    # launches of a step run one after another on one stream.
    from eptq_amd.kernels import decode_workspace
    work = decode_workspace(codes.device)
    while i < len(layers):
        name = layers[i]["name"]
        grp = layers[i:i + 3] if name == "q" else layers[i:i + 2] if name == "gate" else layers[i:i + 1]
        i += len(grp)
        arr = (_lib.EptqLayer * len(grp))()
        off = 0
        for k, l in enumerate(grp):
            arr[k] = _lib.EptqLayer(l["Q"].data_ptr(), l["g"].data_ptr(), l["h"].data_ptr(),
                                    l["O"].data_ptr() if l["nnz"] else None,
                                    l["O_col"].data_ptr() if l["nnz"] else None,
                                    l["O_row_ptr"].data_ptr(), None, None, 0, l["Q"].shape[0], off)
            off += l["out"]
        x = xs[grp[0]["inp"]]
        y = torch.empty((B, off), dtype=torch.float16, device=x.device)

        def run(stream, arr=arr, n=len(grp), x=x, y=y, off=off, N=grp[0]["inp"]):
            rc = lib.eptq_e8d4_forward_multi(n, arr, codes.data_ptr(), _lib.EPTQ_F16, x.data_ptr(),
                                             _lib.EPTQ_F16, N, B, y.data_ptr(), off, work.data_ptr(),
                                             work.numel(), stream)
            if rc:
                _lib.check(rc, "eptq_e8d4_forward_multi")
        units.append((run, grp, arr, y))
    return units


def event_timed(torch, fns, stream, sleep_cycles=20_000_000):
    """GPU duration (ms) of each of ``fns`` launched back to back on ``stream``.

    Consecutive launches are separated by timing events; a device sleep ahead
    of them keeps the queue backed up so that host-side launch overhead falls
    outside the brackets.  Returns (durations, backed_up)."""
    n = len(fns)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    backed = False
    for _ in range(4):
        with torch.cuda.stream(stream):
            torch.cuda._sleep(sleep_cycles)
            guard = torch.cuda.Event()
            guard.record(stream)
            evs[0].record(stream)
            for i, f in enumerate(fns):
                f()
                evs[i + 1].record(stream)
            backed = not guard.query()
        torch.cuda.synchronize()
        if backed:
            break
        sleep_cycles *= 4
    return [evs[i].elapsed_time(evs[i + 1]) for i in range(n)], backed


# ---------------------------------------------------------------------------
# HBM traffic from rocprofv3 counters (child processes, before GPU init here)
# ---------------------------------------------------------------------------

def traffic_probe(args):
    """Child of ``rocprofv3 --pmc``: one 512 MiB calibration copy, then one
    eager step of the decode workload."""
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    codes, layers, xs, ys = make_workload(torch, dev, args.layers, args.batch)
    src = torch.ones(CALIB_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    units = make_units(torch, codes, layers, xs, args.batch)
    s = torch.cuda.current_stream().cuda_stream
    for u in units:
        u[0](s)
    torch.cuda.synchronize()
    print("probe done", flush=True)


def _pmc_pass(counter, args, tmp):
    rocprof = shutil.which("rocprofv3")
    if rocprof is None:
        raise RuntimeError("rocprofv3 not found")
    out = os.path.join(tmp, counter)
    cmd = [rocprof, "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "p", "--",
           sys.executable, "-u", os.path.abspath(__file__), "--probe-traffic",
           "--layers", str(args.layers), "--batch", str(args.batch)]
    proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                            start_new_session=True, text=True)
    try:
        log, _ = proc.communicate(timeout=args.pmc_timeout)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        proc.communicate()
        raise RuntimeError(f"rocprofv3 --pmc {counter} timed out")
    if proc.returncode != 0 and "probe done" not in log:
        raise RuntimeError(f"rocprofv3 --pmc {counter} exited {proc.returncode}: {log[-400:]}")
    files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise RuntimeError(f"no counter_collection.csv from the {counter} pass")
    per_dispatch = {}
    with open(files[0], newline="") as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            key = row["Dispatch_Id"]
            d = per_dispatch.setdefault(key, {"name": row["Kernel_Name"], "v": 0.0})
            d["v"] += float(row["Counter_Value"])
    calib = [d["v"] for d in per_dispatch.values() if "copyBuffer" in d["name"]]
    dec = [d["v"] for d in per_dispatch.values() if DECODE_KERNEL in d["name"]]
    if not calib or not dec:
        raise RuntimeError(f"{counter}: calibration copy or decode dispatches missing")
    kib_copy = max(calib)
    factor = CALIB_BYTES / (kib_copy * 1024.0)
    return {"counter": counter, "copy_kib": kib_copy, "factor": round(factor, 4),
            "decode_dispatches": len(dec),
            "bytes_per_launch": statistics.fmean(dec) * 1024.0 * factor}


def measure_traffic(args):
    tmp = tempfile.mkdtemp(prefix="eptq_pmc_")
    try:
        fetch = _pmc_pass("FETCH_SIZE", args, tmp)
        write = _pmc_pass("WRITE_SIZE", args, tmp)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return {"bytes_per_launch": fetch["bytes_per_launch"] + write["bytes_per_launch"],
            "fetch": fetch, "write": write}


# ---------------------------------------------------------------------------
# Side measurements
# ---------------------------------------------------------------------------

def _cpu_threads():
    import torch
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return torch.get_num_threads()


def _median_runs(fn, runs=5):
    """Wall-clock seconds of ``fn``: one warmup call, then the median of ``runs``."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _cpu_dequant_matmul(qd, xs, kind, tab, runs=5):
    """Reference CPU path on one layer: seconds of the per-column
    ``dequantize_layer`` restatement (algorithms/eptq.py:406-471) and, for
    each x of ``xs``, of y = x.float() @ W.float().T (+ bias); each the
    median of ``runs`` after one warmup."""
    import torch
    from oracle.dequant import dequantize_layer_torch_loop
    S = None if qd.S_group is None else qd.S_group.numpy()
    args = (qd.Q.numpy(), qd.g.numpy(), qd.h.numpy(), qd.O.numpy(), tab, kind, S)
    t_dq = _median_runs(lambda: dequantize_layer_torch_loop(*args), runs)
    Wf = dequantize_layer_torch_loop(*args).float()
    bf = None if qd.bias is None else qd.bias.float()
    t_mm = []
    for x in xs:
        xf = x.float()

        def mm():
            y = torch.matmul(xf, Wf.T)
            return y if bf is None else y + bf
        t_mm.append(_median_runs(mm, runs))
    return t_dq, t_mm


def cpu_baseline(seed=1000, runs=5):
    """Reference CPU path (per-column ``dequantize_layer`` restatement +
    fp32 ``torch.matmul``) on a bounded sample of the benchmark workload: the
    seven Linears of one Llama-2-7B decoder layer (1/32 of a step) at batch
    1, on all of this host's cores (about 20 s with the warm-up runs)."""
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer, make_x

    cores = _cpu_threads()
    tab = E8D4Quantizer(radius=1.75).flat_table().numpy()
    t_dq = t_mm = 0.0
    nbytes = 0
    for idx, (_, out, inp) in enumerate(LLAMA2_7B):
        qd = make_layer(out, inp, seed=seed + idx, percmask=0.001)
        a, b = _cpu_dequant_matmul(qd, [make_x(1, inp, seed=seed + 100 + idx)], "e8_d4", tab, runs)
        t_dq, t_mm = t_dq + a, t_mm + b[0]
        nbytes += algo_bytes(out, inp, 1, int(qd.O.shape[0]))
        del qd
    t = t_dq + t_mm
    return {"value": round(nbytes / t / 1e9, 6), "unit": "GB/s", "cores": cores, "kind": "port",
            "dequant_s": round(t_dq, 4), "matmul_s": round(t_mm, 5),
            "sample": f"the seven Linears of one Llama-2-7B decoder layer (q/k/v/o 4096x4096, gate/up "
                      f"11008x4096, down 4096x11008; E8-D4 r=1.75, p=0.001) at B=1: per-column "
                      f"dequantize_layer restatement, then fp32 torch.matmul, each timed separately, "
                      f"median of {runs} after one warmup; {t:.2f} s for {nbytes} algorithmic bytes"}


def cpu_configs(seed=2000, runs=5):
    """The reference CPU path per layer and batch of benchmark configurations
    0-3 (BASELINE's CPU plan): dequant and matmul timed separately, median of
    ``runs`` after one warmup, all host cores."""
    from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
    from eptq_amd.synthetic import make_layer, make_x

    cores = _cpu_threads()
    e8d4 = E8D4Quantizer(radius=1.75).flat_table().numpy()
    e8 = E8LatticeQuantizer(radius=1.6).flat_table().numpy()
    cases = [("0", "e8_lattice", e8, 3072, 768, None, 0.002, True, (1,))]
    cases += [("1", "e8_d4", e8d4, o, i, None, 0.001, False, (1, 8))
              for o, i in ((4096, 4096), (11008, 4096), (4096, 11008))]
    cases += [("2", "e8_d4", e8d4, o, i, LLAMA3_8B_QB, 0.002, False, (1, 4, 16))
              for o, i in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336))]
    cases += [("3", "e8_d4", e8d4, o, i, None, 0.002, False, (2048,)) for _, o, i in LLAMA2_13B]
    rows = []
    for k, (cfg, kind, tab, out, inp, qb, p, bias, batches) in enumerate(cases):
        qd = make_layer(out, inp, seed=seed + k, percmask=p, qb_size=qb, bias=bias)
        nnz = int(qd.O.shape[0])
        ng = 0 if qd.S_group is None else int(qd.S_group.shape[0])
        t_dq, t_mms = _cpu_dequant_matmul(qd, [make_x(B, inp, seed=seed + 50 + B) for B in batches], kind, tab,
                                          runs)
        for B, t_mm in zip(batches, t_mms):
            row = {"config": cfg, "shape": f"{out}x{inp}", "B": B, "dequant_s": round(t_dq, 4),
                   "matmul_s": round(t_mm, 5), "total_s": round(t_dq + t_mm, 4)}
            if cfg == "3":
                row["tflops"] = round(2.0 * B * out * inp / (t_dq + t_mm) / 1e12, 4)
            else:
                row["gbs"] = round(algo_bytes(out, inp, B, nnz, bias=bias, n_groups=ng) / (t_dq + t_mm) / 1e9, 6)
            rows.append(row)
            print(f"# cpu config {cfg} {out}x{inp} B={B}: dequant {t_dq:.3f} s, matmul {t_mm * 1e3:.2f} ms",
                  file=sys.stderr, flush=True)
    return {"cores": cores, "kind": "port", "runs": runs, "rows": rows}


def e2e_decode(torch, dev, batches=(1, 8), new_tokens=256, prompt_len=128):
    """Synthetic Llama-2-7B greedy decode tok/s (prefill untimed)."""
    from eptq_amd.llama import LLAMA2_7B as CFG, GraphDecoder, build_synthetic
    model = build_synthetic(CFG, device=dev, percmask=0.002)
    res = {}
    for B in batches:
        dec = GraphDecoder(model, B, prompt_len + new_tokens, device=dev)
        gen = torch.Generator(device=dev).manual_seed(11)
        prompt = torch.randint(0, CFG.vocab, (B, prompt_len), generator=gen, device=dev)
        dec.prefill(prompt)
        dec.capture()
        best = None
        for _ in range(2):
            torch.cuda.synchronize()
            tp = time.perf_counter()
            dec.prefill(prompt)
            torch.cuda.synchronize()
            prefill_s = time.perf_counter() - tp
            t0 = time.perf_counter()
            for _ in range(new_tokens - 1):
                dec.step()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            if best is None or dt < best[0]:
                best = (dt, prefill_s)
        dt, prefill_s = best
        res[f"b{B}"] = {"tok_s": round(B * (new_tokens - 1) / dt, 1),
                        "tok_s_per_seq": round((new_tokens - 1) / dt, 1),
                        "ms_per_token_step": round(dt / (new_tokens - 1) * 1e3, 3),
                        "prefill_ms": round(prefill_s * 1e3, 2)}
        del dec
    del model
    torch.cuda.empty_cache()
    res["config"] = {"model": "llama-2-7b (random init)", "prompt_len": prompt_len,
                     "new_tokens": new_tokens, "codebook": "e8_d4", "radius": 1.75,
                     "percmask": 0.002, "lm_head": "fp16", "hip_graph": True,
                     "timing": "(new_tokens-1) decode steps after an untimed prefill, best of 2"}
    return res


LLAMA3_8B_QB = 128


def decode_batches(torch, dev, stream_bytes=576 << 20):
    """Decode-step Linear units at the batch sizes of configurations 1 and 2:
    synthetic Llama-2-7B (B = 1, 8) and Llama-3-8B with S_group qb=128
    (B = 1, 4, 16).  Each unit is one eptq_e8d4_forward_multi launch with the
    decode workspace (q|k|v and gate|up as multi-layer launches).  Every unit
    is built as enough distinct copies (different seeds) to exceed
    ``stream_bytes`` of indices (over 512 MB, twice the 256 MB MALL), and the copies are
    launched back to back with HIP events around the whole group, as a decode
    step streams distinct layers.  B = 1..2 run the vector decode kernel,
    3..16 the matrix-core one."""
    from eptq_amd.kernels import _lib, decode_workspace
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer, make_x

    codes = E8D4Quantizer(radius=1.75).flat_table().half().to(dev)
    lib = _lib.load()
    work = decode_workspace(dev)
    stream = torch.cuda.current_stream()
    models = {
        "llama2_7b": (None, 0.001, (1, 8), [("q|k|v", [(4096, 4096)] * 3), ("o", [(4096, 4096)]),
                                            ("gate|up", [(11008, 4096)] * 2), ("down", [(4096, 11008)])]),
        "llama3_8b_qb128": (LLAMA3_8B_QB, 0.002, (1, 4, 16),
                            [("q|k|v", [(4096, 4096), (1024, 4096), (1024, 4096)]), ("o", [(4096, 4096)]),
                             ("gate|up", [(14336, 4096)] * 2), ("down", [(4096, 14336)])]),
    }
    out = {}
    for mname, (qb, p, batches, units) in models.items():
        res = {}
        for ui, (uname, shapes) in enumerate(units):
            ubytes = sum(o // 8 * i * 2 for o, i in shapes)
            copies = []
            for c in range(-(-stream_bytes // ubytes)):
                keep = []
                for k, (o, i) in enumerate(shapes):
                    qd = make_layer(o, i, seed=5000 + 1000 * c + 37 * ui + k, percmask=p, qb_size=qb, device=dev)
                    r_, c_ = (qd.Q == 32767).nonzero(as_tuple=True)
                    rp = torch.cat([torch.zeros(1, dtype=torch.int32, device=dev),
                                    torch.bincount(r_, minlength=qd.Q.shape[0]).cumsum(0).to(torch.int32)])
                    keep.append((qd, c_.to(torch.int32), rp))
                arr = (_lib.EptqLayer * len(keep))()
                off = 0
                for k, (qd, oc, rp) in enumerate(keep):
                    ng = 0 if qd.S_group is None else int(qd.S_group.shape[0])
                    arr[k] = _lib.EptqLayer(qd.Q.data_ptr(), qd.g.data_ptr(), qd.h.data_ptr(),
                                            qd.O.data_ptr() if qd.O.numel() else None,
                                            oc.data_ptr() if oc.numel() else None, rp.data_ptr(), None,
                                            None if qd.S_group is None else qd.S_group.data_ptr(), ng,
                                            qd.Q.shape[0], off)
                    off += 8 * qd.Q.shape[0]
                copies.append((keep, arr))
            N = shapes[0][1]
            width = sum(o for o, _ in shapes)
            # Llama-3 runs in bf16 (HF default): its units also with bf16 x and y.
            for B, bf in [(B, False) for B in batches] + ([(B, True) for B in batches] if qb else []):
                x = make_x(B, N, seed=B, device=dev)
                if bf:
                    x = x.bfloat16()
                y = torch.empty((B, width), dtype=x.dtype, device=dev)
                xdt = _lib.EPTQ_BF16 if bf else _lib.EPTQ_F16

                def f():
                    for keep, arr in copies:
                        rc = lib.eptq_e8d4_forward_multi(len(keep), arr, codes.data_ptr(), _lib.EPTQ_F16,
                                                         x.data_ptr(), xdt, N, B, y.data_ptr(), width,
                                                         work.data_ptr(), work.numel(), stream.cuda_stream)
                        if rc:
                            _lib.check(rc, "eptq_e8d4_forward_multi")
                f()
                d, _ = event_timed(torch, [f, f, f], stream)
                us = statistics.median(d) * 1e3 / len(copies)
                nbytes = sum(algo_bytes(8 * qd.Q.shape[0], qd.Q.shape[1], B, int(qd.O.shape[0]),
                                        n_groups=0 if qd.S_group is None else int(qd.S_group.shape[0]))
                             for qd, _, _ in copies[0][0])
                res[f"{uname} B={B}" + (" bf16" if bf else "")] = {
                    "shape": " + ".join(f"{o}x{i}" for o, i in shapes), "us": round(us, 2),
                    "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                    "kernel": "k_decode_mfma" if B >= 3 else DECODE_KERNEL}
                del x, y
            del copies
            torch.cuda.empty_cache()
        out[mname] = res
    out["note"] = ("per launch: HIP events around %d MB+ of distinct copies of the unit launched back to "
                   "back (median of 3); gbs = algorithmic bytes (indices, S_group, CSR, scales, x, y) / time"
                   % (stream_bytes >> 20))
    return out


def config0(torch, dev, copies=1024, reps=3):
    """Benchmark configuration 0: the E8-lattice Linear at OPT-125m fc1 shape
    (out 3072, in 768) with bias, batch 1, radius 1.6, 0.2% critical blocks.
    ``copies`` distinct layers (over 512 MB of indices, past the MALL) are
    launched back to back through ``eptq_e8_forward`` with HIP events around
    the group and the queue backed up by a device sleep; microseconds per
    launch, algorithmic GB/s and fraction of HBM peak.  The layer is small
    enough that the launch's fixed cost dominates."""
    from eptq_amd.kernels import _lib
    from eptq_amd.quantizers import E8LatticeQuantizer
    from eptq_amd.synthetic import make_layer, make_x

    codes = E8LatticeQuantizer(radius=1.6).flat_table().half().to(dev)
    out_f, in_f = 3072, 768
    stream = torch.cuda.current_stream()
    x = make_x(1, in_f, seed=9, device=dev)
    y = torch.empty((1, out_f), dtype=torch.float16, device=dev)
    layers = []
    for c in range(copies):
        qd = make_layer(out_f, in_f, seed=9000 + c, percmask=0.002, bias=True, device=dev)
        rows, cols = (qd.Q == 32767).nonzero(as_tuple=True)
        rp = torch.cat([torch.zeros(1, dtype=torch.int32, device=dev),
                        torch.bincount(rows, minlength=qd.Q.shape[0]).cumsum(0).to(torch.int32)])
        layers.append((qd, cols.to(torch.int32), rp))

    def f():
        for qd, oc, rp in layers:
            _lib.forward_into("e8_lattice", qd.Q, codes, qd.g, qd.h, x, qd.O, oc, rp, qd.bias, None,
                              y, stream.cuda_stream)
    f()
    d, backed = event_timed(torch, [f] * reps, stream)
    us = statistics.median(d) * 1e3 / copies
    nbytes = statistics.mean(algo_bytes(out_f, in_f, 1, int(qd.O.shape[0]), bias=True) for qd, _, _ in layers)
    gbs = nbytes / (us * 1e-6) / 1e9
    res = {"shape": f"{out_f}x{in_f}", "B": 1, "codebook": "e8_lattice", "radius": 1.6, "percmask": 0.002,
           "bias": True, "us": round(us, 3), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "algorithmic_bytes": round(nbytes), "kernel": "k_matvec<E8>", "copies": copies,
           "events_backed_up": backed}
    del layers
    torch.cuda.empty_cache()
    return res


def dequant_layers(torch, dev, reps=10):
    """Bit-exact dequantization (``eptq_e8d4_dequant``: the fp16 W of the
    reference's ``dequantize_layer``) of the Llama-2-7B Linear shapes.
    Algorithmic bytes: Q, g, h and the CSR (16-byte O rows, 4-byte columns,
    row pointers) read once, W (2 bytes per weight) written once; HBM
    roofline (the write of W dominates: 16x the index bytes)."""
    from eptq_amd.kernels import dequant
    from eptq_amd.kernels.linear import EPTQLinear
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer

    q = E8D4Quantizer(radius=1.75)
    stream = torch.cuda.current_stream()
    out = {}
    for idx, (name, o, i) in enumerate((("4096x4096", 4096, 4096), ("11008x4096", 11008, 4096),
                                        ("4096x11008", 4096, 11008))):
        lin = EPTQLinear.from_quantized_data(make_layer(o, i, seed=4000 + idx, percmask=0.001, device=dev),
                                             q, "e8_d4").to(dev)
        args = ("e8_d4", lin.Q, lin._table_f32.to(dev), lin.g, lin.h, lin.O_vals, lin.O_col, lin.O_row_ptr)
        M, N, nnz = lin.Q.shape[0], lin.Q.shape[1], lin.O_col.numel()
        nbytes = 2 * M * N + 2 * 8 * M + 2 * N + 20 * nnz + 4 * (M + 1) + 2 * 8 * M * N
        dequant(*args)
        d, _ = event_timed(torch, [lambda: dequant(*args)] * reps, stream)
        us = statistics.median(d) * 1e3
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": nbytes}
        del lin
    return out


def prefill_gemm(torch, dev, T=2048, reps=10):
    from eptq_amd.kernels import _lib
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer, make_x

    from eptq_amd.kernels import dequant, f16_gemm

    codes32 = E8D4Quantizer(radius=1.75).flat_table().float().to(dev)
    codes = codes32.half()
    stream = torch.cuda.current_stream()
    out = {}
    for idx, (name, o, i) in enumerate(LLAMA2_13B):
        qd = make_layer(o, i, seed=3000 + idx, percmask=0.002, device=dev)
        rows, cols = (qd.Q == 32767).nonzero(as_tuple=True)
        rp = torch.cat([torch.zeros(1, dtype=torch.int32, device=dev),
                        torch.bincount(rows, minlength=qd.Q.shape[0]).cumsum(0).to(torch.int32)])
        cols = cols.to(torch.int32)
        x = make_x(T, i, seed=3100 + idx, device=dev)
        y = torch.empty((T, o), dtype=torch.float16, device=dev)

        def f():
            _lib.forward_into("e8_d4", qd.Q, codes, qd.g, qd.h, x, qd.O, cols, rp, None, None,
                              y, stream.cuda_stream)
        layer = dict(Q=qd.Q, g=qd.g, h=qd.h, O_vals=qd.O, O_col=cols, O_row_ptr=rp)

        def f2():
            # Comparison only (no product path runs it): the bit-exact W of
            # this library's dequantizer, then torch's fp16 GEMM (hipBLASLt).
            W = dequant("e8_d4", layer["Q"], codes32, layer["g"], layer["h"], layer["O_vals"],
                        layer["O_col"], layer["O_row_ptr"])
            torch.nn.functional.linear(x, W)

        def f3():
            # The two-pass prefill of this library: the same W, then its own
            # LDS-DMA GEMM (eptq_f16_gemm).
            W = dequant("e8_d4", layer["Q"], codes32, layer["g"], layer["h"], layer["O_vals"],
                        layer["O_col"], layer["O_row_ptr"])
            f16_gemm(W, x)
        row = {"shape": f"{o}x{i}", "tokens": T}
        for key, fn in (("fused", f), ("dequant_library_gemm", f2), ("two_pass", f3)):
            fn()
            d, _ = event_timed(torch, [fn] * reps, stream)
            us = statistics.median(d) * 1e3
            tflops = 2.0 * T * o * i / (us * 1e-6) / 1e12
            row[key] = {"us": round(us, 1), "tflops": round(tflops, 1),
                        "frac_mfma_f16": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
        out[name] = row
        del qd, x, y
    return out


# ---------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc passes")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--no-batches", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-dequant", action="store_true")
    ap.add_argument("--no-config0", action="store_true")
    ap.add_argument("--cpu-configs", action="store_true",
                    help="also time the reference CPU path per layer and batch of configurations 0-3 (minutes)")
    ap.add_argument("--pmc-timeout", type=int, default=240)
    ap.add_argument("--probe-traffic", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the quantized Linear is a single-GPU kernel; how it would shard is a design note).",
              file=sys.stderr)
        sys.exit(2)
    if args.probe_traffic:
        traffic_probe(args)
        return

    traffic, traffic_note = None, None
    if not args.no_traffic:
        try:
            traffic = measure_traffic(args)
        except Exception as e:  # counters are evidence, not the measurement itself
            traffic_note = f"unavailable: {e}"
        print(f"# traffic: {traffic if traffic else traffic_note}", file=sys.stderr, flush=True)

    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B = args.batch
    t0 = time.time()
    codes, layers, xs, ys = make_workload(torch, dev, args.layers, B)
    torch.cuda.synchronize()
    print(f"# generated {len(layers)} layers in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    step_bytes = sum(algo_bytes(l["out"], l["inp"], B, l["nnz"]) for l in layers)
    launch = make_launcher(codes, xs, ys)

    cur = torch.cuda.current_stream()
    for l in layers:
        launch(l, cur.cuda_stream)
    torch.cuda.synchronize()

    # Per-shape kernel durations: the launches of each shape back to back on
    # the launch stream, HIP events around each group, host overhead hidden
    # behind a device sleep.
    names = [n for n, _, _ in LLAMA2_7B]
    groups = {n: [l for l in layers if l["name"] == n] for n in names}
    fns = [(lambda g=groups[n]: [launch(l, cur.cuda_stream) for l in g]) for n in names]
    reps = 3
    group_ms = [0.0] * len(names)
    all_backed = True
    for _ in range(reps):
        d, backed = event_timed(torch, fns, cur)
        all_backed &= backed
        for i, v in enumerate(d):
            group_ms[i] += v / reps
    per_shape = {}
    for i, n in enumerate(names):
        g = groups[n]
        nbytes = sum(algo_bytes(l["out"], l["inp"], B, l["nnz"]) for l in g)
        per_shape[n] = {"shape": f"{g[0]['out']}x{g[0]['inp']}",
                        "us": round(group_ms[i] * 1e3 / len(g), 3),
                        "gbs": round(nbytes / (group_ms[i] * 1e-3) / 1e9, 1)}

    def graph_ms(issue):
        """HIP-graph one step (issue(stream) launches it), replay, time with events."""
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            issue(side.cuda_stream)
        cur.wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            issue(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            g.replay()
        end.record()
        torch.cuda.synchronize()
        del g
        return start.elapsed_time(end) / args.steps

    # Reference point: every Linear as its own launch (224 per step).
    ms_separate = graph_ms(lambda st: [launch(l, st) for l in layers])
    # The timed region: the step as a decode step runs it (q|k|v and gate|up
    # as multi-layer launches: 128 launches), captured in a graph, replayed.
    units = make_units(torch, codes, layers, xs, B)
    ms = graph_ms(lambda st: [u[0](st) for u in units])
    value = step_bytes / (ms * 1e-3) / 1e9

    n = len(units)
    bytes_per_launch = step_bytes / n
    avg_us = ms * 1e3 / n
    achieved = bytes_per_launch / (avg_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": round(traffic["bytes_per_launch"]) if traffic else None,
                "kernel": f"{DECODE_KERNEL} (B={B})", "avg_launch_us": round(avg_us, 3),
                "avg_launch_us_source": "HIP events around the timed graph replays / launches",
                "algorithmic_bytes_per_launch": round(bytes_per_launch),
                "launches": n, "per_shape_events_backed_up": all_backed}
    if traffic:
        roofline["traffic_detail"] = {
            "fetch_factor": traffic["fetch"]["factor"], "write_factor": traffic["write"]["factor"],
            "fetch_bytes_per_launch": round(traffic["fetch"]["bytes_per_launch"]),
            "write_bytes_per_launch": round(traffic["write"]["bytes_per_launch"]),
            "calibration": f"{CALIB_BYTES} B device copy (copyBuffer) per counter"}
    else:
        roofline["traffic_note"] = traffic_note or "skipped (--no-traffic)"

    for l in layers:
        l.clear()
    del layers, xs, ys, units
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    rec = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "llama2_7b_decoder_linears_decode", "batch": B,
                   "layers": args.layers, "linears_per_step": 7 * args.layers, "launches_per_step": n,
                   "grouping": "q|k|v and gate|up as multi-layer launches, o and down alone",
                   "codebook": "e8_d4", "radius": 1.75, "percmask": 0.001,
                   "algorithmic_bytes_per_step": step_bytes, "hip_graph": True},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "roofline": roofline,
        "per_shape": per_shape,
        "separate_launches": {"launches_per_step": len(LLAMA2_7B) * args.layers,
                              "ms_per_step": round(ms_separate, 5),
                              "gbs": round(step_bytes / (ms_separate * 1e-3) / 1e9, 2)},
    }
    if not args.no_batches:
        rec["decode_batches"] = decode_batches(torch, dev)
    if not args.no_e2e:
        rec["e2e"] = e2e_decode(torch, dev)
        print(f"# e2e: {rec['e2e']}", file=sys.stderr, flush=True)
    if not args.no_prefill:
        rec["prefill"] = prefill_gemm(torch, dev)
        print(f"# prefill: {rec['prefill']}", file=sys.stderr, flush=True)
    if not args.no_dequant:
        rec["dequant"] = dequant_layers(torch, dev)
        print(f"# dequant: {rec['dequant']}", file=sys.stderr, flush=True)
    if not args.no_config0:
        rec["config0"] = config0(torch, dev)
        print(f"# config0: {rec['config0']}", file=sys.stderr, flush=True)
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline()
    if args.cpu_configs:
        rec["cpu_configs"] = cpu_configs()
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
