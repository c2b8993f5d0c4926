"""Benchmark of the HIP sampler on one MI355X.

A step is one tms_sample_batch call over the resident batch (config 2 of the
survey by default: B=64 rows x V=128256 fp32 logits, repetition/frequency/
presence penalties over 256-id windows, a grammar bitmask, T=0.7, top-k 40,
top-p 0.95, min-p 0.05).  W warm-up steps, then K timed steps captured in a
HIP graph and replayed once, bracketed by device synchronisation; HIP events
on the launch stream time the region.  Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--config 2|3|5] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM = 8.0e12
METRIC = "sampled rows/sec and HBM GB/s (% of peak) at B=64, V=128256, fp32 logits"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=[2, 3, 5])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--eager", action="store_true", help="time eager launches, no graph")
    return ap.parse_args()


def workload(cfg):
    from tensormark_amd import workloads

    if cfg == 2:
        w = workloads.cfg2(with_mask=True)
        B, V = w["logits"].shape
        bytes_ = w["logits"].nbytes + w["recent"].nbytes + w["mask"].nbytes
        name = "cfg2: B=64 V=128256 fp32, penalties + grammar mask + top-k 40 + top-p 0.95 + min-p 0.05"
        return w, "f32", bytes_, name
    if cfg == 3:
        w = workloads.cfg3()
        bytes_ = w["logits"].nbytes + w["mask"].nbytes
        return w, "f16", bytes_, "cfg3: B=128 V=151936 fp16, grammar mask (0.3%), top-p 0.9"
    w = workloads.cfg5()
    w["logits"] = workloads.to_bf16_bits(w["logits"])
    B = w["logits"].shape[0]
    bytes_ = w["logits"].nbytes + w["recent"].nbytes + B * 4
    return w, "bf16", bytes_, "cfg5: B=1024 V=256000 bf16, 50% greedy, top-k 100 + top-p 0.98"


def cpu_baseline(w, cfg):
    """The reference's own tmsample.h (oracle/_ref), timed on this host."""
    import oracle

    ref = oracle.reference()
    if ref is None or cfg != 2:
        return None
    x = w["logits"]
    threads = max(1, min(16, os.cpu_count() or 1))
    t0 = time.perf_counter()
    dt, _ = ref.bench(x, 0.7, 40, 0.95, recent=w["recent"], window=256, penalty=1.1,
                      mask=w["mask"], threads=threads, reps=1)
    reps = max(1, min(200, int(2.0 / max(dt, 1e-4))))
    dt, _ = ref.bench(x, 0.7, 40, 0.95, recent=w["recent"], window=256, penalty=1.1,
                      mask=w["mask"], threads=threads, reps=reps)
    wall = time.perf_counter() - t0
    B = x.shape[0]
    return {
        "value": round(B / dt, 1),
        "unit": "rows/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"the reference tmsample.h (mask -> apply_repeat_penalty 1.1/256 -> "
                   f"sample T=0.7 k=40 p=0.95) over the same {B} x {x.shape[1]} fp32 rows, "
                   f"best of {reps} passes, {threads} threads, {wall:.1f} s wall; "
                   f"frequency/presence/min-p are absent from the reference"),
    }


def traffic_from_profiles(cfg):
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    try:
        d = json.load(open(p))
        return d.get(f"cfg{cfg}")
    except Exception:
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              f"(rows are independent; a batch split across GPUs needs no exchange)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from tensormark_amd import Sampler

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    w, dt_name, algo_bytes, name = workload(args.config)
    x_np = w["logits"]
    B, V = x_np.shape
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt_name]
    if dt_name == "bf16":
        x = torch.from_numpy(x_np.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        x = torch.from_numpy(x_np).to(dev)
    recent = None if w.get("recent") is None else torch.from_numpy(w["recent"]).to(dev)
    mask = None if w.get("mask") is None else torch.from_numpy(w["mask"].view(np.int32)).to(dev)
    s = Sampler(B, V)
    params = s.params_tensor(w["params"])
    out = {
        "tokens": torch.empty(B, dtype=torch.int32, device=dev),
        "status": torch.empty(B, dtype=torch.int32, device=dev),
        "keep": torch.empty(B, dtype=torch.int32, device=dev),
    }
    stream = torch.cuda.Stream(device=dev)
    import ctypes

    a = s.make_args(x, params, recent=recent, mask=mask, out=out)
    ap = ctypes.byref(a)
    sp = ctypes.c_void_p(stream.cuda_stream)
    fn = s.lib.tms_sample_batch
    h = s.handle

    def launch():
        rc = fn(h, ap, sp)
        if rc != 0:
            raise RuntimeError(f"tms_sample_batch returned {rc}")

    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            launch()
    torch.cuda.synchronize()
    st = out["status"].cpu().numpy()
    assert (st == 0).all(), f"row status {st}"

    graph = None
    if not args.eager:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(args.steps):
                launch()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()   # one untimed replay: graph upload
        torch.cuda.synchronize()

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        if graph is not None:
            graph.replay()
        else:
            for _ in range(args.steps):
                launch()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    rows_per_s = B / (ms * 1e-3)
    achieved = algo_bytes / (ms * 1e-3)
    cpu = None if args.no_cpu else cpu_baseline(w, args.config)
    line = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"f32": "f32", "f16": "f16", "bf16": "bf16"}[dt_name] + " logits, f64 softmax tail",
        "data": "synthetic (seeded numpy; no model)",
        "config": {"workload": name, "batch": B, "vocab": V, "launch": "graph" if graph else "eager",
                   "wall_s": round(wall, 4)},
        "hbm_gbps": round(achieved / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved / 1e9, 1),
            "peak": PEAK_HBM / 1e9,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM, 4),
            "traffic": traffic_from_profiles(args.config),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    s.close()


if __name__ == "__main__":
    main()
