"""Benchmark of the HIP sampler on one MI355X.

A step is one tms_sample_batch call over the resident batch (config 2 of the
survey by default: B=64 rows x V=128256 fp32 logits, repetition/frequency/
presence penalties over 256-id windows, a grammar bitmask, T=0.7, top-k 40,
top-p 0.95, min-p 0.05).  W warm-up steps, then K timed steps captured in a
HIP graph and replayed once, bracketed by device synchronisation; HIP events
on the launch stream time the region.  Prints one JSON line.

The inputs are resident in HBM before the timed region starts.  The chip's
256 MB last-level cache (MALL) would hold one config-2 batch (34 MB) between
launches, so the bench keeps enough copies of the batch to stream at least
768 MB and rotates through them, launch by launch: every launch reads its
batch from HBM, not from the cache (--no-rotate times the cache-resident case).

    python bench.py [--steps K] [--warmup W] [--config 2|3|4|5] [--no-cpu] [--no-rotate]
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
    ap.add_argument("--config", type=int, default=2, choices=[2, 3, 4, 5])
    ap.add_argument("--no-rotate", action="store_true",
                    help="reuse one input batch (cache-resident after the first launch)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--eager", action="store_true", help="time eager launches, no graph")
    ap.add_argument("--general", action="store_true",
                    help="pass no row-kind hint (the general kernel for every batch)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="first run 3 plain device copies of MIB MiB (a known-size kernel that "
                         "calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def workload(cfg):
    from tensormark_amd import workloads

    if cfg == 2:
        w = workloads.cfg2(with_mask=True)
        B, V = w["logits"].shape
        bytes_ = w["logits"].nbytes + w["recent"].nbytes + w["mask"].nbytes
        name = "cfg2: B=64 V=128256 fp32, penalties + grammar mask + top-k 40 + top-p 0.95 + min-p 0.05"
        return w, "f32", bytes_, name
    if cfg == 4:
        w = workloads.cfg4()
        bytes_ = w["target"].nbytes + w["draft"].nbytes + w["tokens"].nbytes
        return w, "f32", bytes_, ("cfg4: speculative verify B=32 x k=8 drafts, V=32000 fp32, "
                                  "accept/reject + residual or bonus draw")
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
    reps = max(1, min(5000, int(10.0 / max(dt, 1e-4))))   # about 10 s of host work
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


def traffic_from_profiles(cfg, general=False):
    """HBM bytes per launch measured with rocprofv3 (profiles/traffic.json), or None."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    try:
        d = json.load(open(p))
        return d.get(f"cfg{cfg}" + ("_general" if general else ""))
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
    from tensormark_amd.sampler import ROWS_ANY, row_kinds_of

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    w, dt_name, algo_bytes, name = workload(args.config)
    import ctypes

    if args.calib_copy > 0:
        n = args.calib_copy * 2**20 // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    stream = torch.cuda.Stream(device=dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    n_sets = 1 if args.no_rotate else max(1, -(-768 * 2**20 // algo_bytes))

    def up(a_np, view=None):
        t = torch.from_numpy(np.ascontiguousarray(a_np if view is None else a_np.view(view)))
        return t.to(dev)

    keep = []   # device buffers the argument records point at
    if args.config == 4:
        from tensormark_amd.sampler import SpecArgs

        B, k1, V = w["target"].shape
        s = Sampler(B, V)
        params = s.params_tensor(w["params"])
        tg0, dr0, tok = up(w["target"]), up(w["draft"]), up(w["tokens"])
        out = {n: torch.empty(B, dtype=torch.int32, device=dev)
               for n in ("accepted", "token", "status")}
        recs = []
        for i in range(n_sets):
            tg, dr = (tg0, dr0) if i == 0 else (tg0.clone(), dr0.clone())
            keep += [tg, dr]
            a = SpecArgs()
            a.target_logits, a.draft_logits = tg.data_ptr(), dr.data_ptr()
            a.dtype, a.batch, a.k, a.vocab = 0, B, k1 - 1, V
            a.draft_tokens, a.params = tok.data_ptr(), params.data_ptr()
            a.draws = None
            a.out_accepted = out["accepted"].data_ptr()
            a.out_token = out["token"].data_ptr()
            a.out_status = out["status"].data_ptr()
            recs.append(a)
        fn = s.lib.tms_spec_verify
    else:
        x_np = w["logits"]
        B, V = x_np.shape
        x0 = up(x_np, np.int16).view(torch.bfloat16) if dt_name == "bf16" else up(x_np)
        recent = None if w.get("recent") is None else up(w["recent"])
        mask0 = None if w.get("mask") is None else up(w["mask"], np.int32)
        s = Sampler(B, V)
        params = s.params_tensor(w["params"])
        # the caller's row-kind hint, from the host-side parameters
        kinds = ROWS_ANY if args.general else row_kinds_of(w["params"])
        out = {n: torch.empty(B, dtype=torch.int32, device=dev) for n in ("tokens", "status", "keep")}
        recs = []
        for i in range(n_sets):
            x = x0 if i == 0 else x0.clone()
            mask = mask0 if (i == 0 or mask0 is None) else mask0.clone()
            rc = recent if (i == 0 or recent is None) else recent.clone()
            keep += [x, mask, rc]
            recs.append(s.make_args(x, params, recent=rc, mask=mask, out=out, row_kinds=kinds))
        fn = s.lib.tms_sample_batch
    ptrs = [ctypes.byref(a) for a in recs]
    h = s.handle
    counter = [0]

    def launch():
        rc = fn(h, ptrs[counter[0] % n_sets], sp)
        counter[0] += 1
        if rc != 0:
            raise RuntimeError(f"launch returned {rc}")

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
    rows_per_s = B / (ms * 1e-3)   # config 4: sequences verified per second
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
        "dtype": "f32",
        "data": "synthetic (seeded numpy; no model)",
        "config": {"workload": name, "batch": B, "vocab": V, "launch": "graph" if graph else "eager",
                   "input_sets": n_sets, "hbm_resident_bytes": n_sets * algo_bytes,
                   "wall_s": round(wall, 4)},
        "hbm_gbps": round(achieved / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved / 1e9, 1),
            "peak": PEAK_HBM / 1e9,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM, 4),
            "traffic": traffic_from_profiles(args.config, args.general),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    s.close()


if __name__ == "__main__":
    main()
