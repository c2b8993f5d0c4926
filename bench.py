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

roofline.traffic is the sampler's HBM bytes per launch measured in the same
run: before this process touches the GPU it runs itself twice under
rocprofv3 (--pmc FETCH_SIZE, then --pmc WRITE_SIZE, 22 eager launches each),
and scales each counter by what it reads for a 256 MiB device copy of known
size (--no-traffic skips this).  The CPU baseline is the reference's own
tmsample.h (oracle/_ref) on the host's threads, median pass, with a one-thread
figure beside it.

    python bench.py [--steps K] [--warmup W] [--config 2|3|4|5] [--no-cpu] [--no-traffic]
                    [--no-rotate]
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
# BASELINE.json's metric is quoted on config 2; the other configs are named the
# same way for their own shapes.
METRICS = {
    1: "sampled rows/sec at B=1, V=32000, fp32 logits (single-row latency)",
    2: "sampled rows/sec and HBM GB/s (% of peak) at B=64, V=128256, fp32 logits",
    3: "sampled rows/sec and HBM GB/s (% of peak) at B=128, V=151936, fp16 logits",
    4: "verified sequences/sec and HBM GB/s (% of peak) at B=32, k=8, V=32000, fp32 logits",
    5: "sampled rows/sec and HBM GB/s (% of peak) at B=1024, V=256000, bf16 logits",
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--no-rotate", action="store_true",
                    help="reuse one input batch (cache-resident after the first launch)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--eager", action="store_true", help="time eager launches, no graph")
    ap.add_argument("--general", action="store_true",
                    help="pass no row-kind hint (the general kernel for every batch)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the in-run HBM traffic measurement (two rocprofv3 counter passes)")
    ap.add_argument("--rotate-mb", type=int, default=768, metavar="MB",
                    help="HBM-resident input copies to rotate through, in MB in all (default 768: "
                         "above the 256 MB MALL)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="first run 3 plain device copies of MIB MiB (a known-size kernel that "
                         "calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def workload(cfg):
    from tensormark_amd import workloads

    if cfg == 1:
        w = workloads.cfg1()
        bytes_ = w["logits"].nbytes + w["recent"].nbytes
        return w, "f32", bytes_, ("cfg1: B=1 V=32000 fp32, repetition 1.1/64 + top-k 40 + top-p 0.95, "
                                  "one row a call")
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


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(run, budget=10.0):
    """(median pass seconds, passes): one pass to size, then passes for
    about `budget` seconds of host work (median taken by the callee)."""
    dt = run(1)
    reps = max(3, min(5000, int(budget / max(dt, 1e-4))))
    return run(reps), reps


def cpu_baseline(w, cfg):
    """The reference's own tmsample.h (oracle/_ref) on this host for configs
    2, 3 and 5: rows dealt to a thread pool, the median pass of about 10 s of
    work, and a one-thread figure beside it.  Config 4 has no reference
    implementation: the oracle's C restatement of the verify rule is timed
    instead, one thread (kind "port")."""
    import oracle

    nproc = os.cpu_count() or 1
    # the GPU box's CPU share is 16 threads (OMP_NUM_THREADS there), whatever nproc shows
    threads = max(1, min(nproc, int(os.environ.get("OMP_NUM_THREADS", "16") or 16), 16))
    t0 = time.perf_counter()
    if cfg == 4:
        orc = oracle.oracle()
        tg, dr, tok, prm = w["target"], w["draft"], w["tokens"], w["params"]
        B, k = tok.shape
        words = np.zeros((B, k + 1, 2), np.uint32)
        for b in range(B):
            for i in range(k + 1):
                words[b, i] = orc.row_words(int(prm["seed"][b]), int(prm["offset"][b]), i)

        def run(reps):
            ts = []
            for _ in range(reps):
                a = time.perf_counter()
                for b in range(B):
                    orc.spec_verify_seq(tg[b], dr[b], tok[b], float(prm["temperature"][b]), words[b])
                ts.append(time.perf_counter() - a)
            return float(np.median(ts))

        dt, reps = _timed(run)
        return {"value": round(B / dt, 1), "unit": "sequences/s", "cores": 1, "kind": "port",
                "cpu": cpu_model(), "nproc": nproc,
                "sample": (f"the oracle's C restatement (tmo_spec_verify_seq; the reference has no "
                           f"stochastic verify) over the same {B} sequences x {k} drafts, V="
                           f"{tg.shape[2]}, one thread, median of {reps} passes; "
                           f"{time.perf_counter() - t0:.1f} s wall")}
    ref = oracle.reference()
    if ref is None:
        return None
    if cfg == 1:
        x = w["logits"]
        groups = [(x, dict(recent=w["recent"], window=64, penalty=1.1), (0.8, 40, 0.95, False))]
        what = "apply_repeat_penalty 1.1/64 -> sample T=0.8 k=40 p=0.95, one row"
    elif cfg == 2:
        x = w["logits"]
        groups = [(x, dict(recent=w["recent"], window=256, penalty=1.1, mask=w["mask"]),
                   (0.7, 40, 0.95, False))]
        what = "mask -> apply_repeat_penalty 1.1/256 -> sample T=0.7 k=40 p=0.95"
    elif cfg == 3:
        x = w["logits"].astype(np.float32)   # fp16 widened before the timed region
        groups = [(x, dict(mask=w["mask"]), (1.0, x.shape[1], 0.9, False))]
        what = "fp16 rows widened beforehand; mask -> sample T=1.0 k=V p=0.9"
    else:
        from tensormark_amd import workloads

        x = workloads.bf16_bits_to_f32(w["logits"])   # bf16 widened before the timed region
        g = np.asarray(w["params"]["greedy"]) != 0
        rec = w["recent"]
        groups = []
        for sel, greedy in ((~g, False), (g, True)):
            groups.append((np.ascontiguousarray(x[sel]),
                           dict(recent=np.ascontiguousarray(rec[sel]), window=512, penalty=1.05),
                           (1.2, 100, 0.98, greedy)))
        what = ("bf16 rows widened beforehand; apply_repeat_penalty 1.05/512 -> sample T=1.2 k=100 "
                "p=0.98 on the sampled half, greedy on the other half (two pools, times added)")
    B, V = x.shape

    def run_all(thr, rows=None):
        def run(reps):
            tot = 0.0
            for xx, kw, (T, k, p, gr) in groups:
                kk = dict(kw)
                xs = xx if rows is None else xx[:rows]
                if rows is not None:
                    for key in ("recent", "mask"):
                        if kk.get(key) is not None:
                            kk[key] = kk[key][:rows]
                d, _ = ref.bench(xs, T, k, p, threads=thr, reps=reps, greedy=gr, **kk)
                tot += d
            return tot
        return run

    if B == 1:
        threads = 1   # one row: one thread does all of it
    dt, reps = _timed(run_all(threads))
    # the one-thread figure: up to 16 rows of each group, median of enough
    # passes for about 3 s of work
    n1 = min(B, 16)
    dt1, reps1 = _timed(run_all(1, rows=n1), budget=3.0)
    n1 *= len(groups)
    return {
        "value": round(B / dt, 1),
        "unit": "rows/s",
        "cores": threads,
        "kind": "reference",
        "one_core": round(n1 / dt1, 1),
        "cpu": cpu_model(),
        "nproc": nproc,
        "sample": (f"the reference tmsample.h compiled -O3 ({what}) over the same {B} x {V} rows, "
                   f"rows dealt to {threads} threads (the GPU box's CPU share; nproc {nproc}), "
                   f"median of {reps} passes; one_core: {n1} rows on 1 thread, median of {reps1} passes; "
                   f"{time.perf_counter() - t0:.1f} s wall in all; frequency/presence/min-p are "
                   f"absent from the reference"),
    }


def verify(w, cfg, out):
    """The last timed launch's outputs against the oracle's answer for the
    same inputs (every row): tokens, keep counts and status (configs 1-3, 5),
    accepted lengths, tokens and status (config 4).  Returns (ok, note)."""
    import oracle

    orc = oracle.oracle()
    got = {k: v.cpu().numpy() for k, v in out.items()}
    if cfg == 4:
        tg, dr, tok, prm = w["target"], w["draft"], w["tokens"], w["params"]
        B, k = tok.shape
        bad = 0
        for b in range(B):
            words = np.array([orc.row_words(int(prm["seed"][b]), int(prm["offset"][b]), i)
                              for i in range(k + 1)], np.uint32)
            st, acc, t = orc.spec_verify_seq(tg[b], dr[b], tok[b], float(prm["temperature"][b]), words)
            bad += int(got["accepted"][b] != acc or got["token"][b] != t or got["status"][b] != st)
        return bad == 0, f"{B - bad} of {B} sequences equal the oracle's (accepted length, token)"
    x = w["logits"]
    if cfg == 3:
        x = x.astype(np.float32)
    elif cfg == 5:
        from tensormark_amd import workloads

        x = workloads.bf16_bits_to_f32(x)
    want = orc.sample_batch(x, w["params"], recent=w.get("recent"), mask=w.get("mask"))
    ok = ((got["tokens"] == want["tokens"]) & (got["keep"] == want["keep"]) &
          (got["status"] == want["status"]))
    return bool(ok.all()), f"{int(ok.sum())} of {len(ok)} rows equal the oracle's (token, keep, status)"


def measure_traffic(args):
    """HBM bytes per launch of the sampler, measured in this run: two child
    runs of this script under rocprofv3 (FETCH_SIZE, then WRITE_SIZE; one
    counter pass each), each with a device copy of 256 MiB first whose
    counters calibrate the bytes.  The children rotate over 64 MB of input
    copies, twice the L2 caches' 32 MB, so every launch misses L2 (the
    counters count what L2 fetches, MALL hits included) while the copies'
    set-up stays short under the profiler.  Returns (bytes, note) or (None,
    reason)."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if prof is None:
        return None, "rocprofv3 not found"
    steps, warm, mib = 20, 2, 256
    vals = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        out = tempfile.mkdtemp(prefix="tms_traffic_", dir="/tmp")
        cmd = [prof, "--pmc", ctr, "--output-format", "csv", "-d", out, "-o", "p", "--",
               sys.executable, os.path.abspath(__file__), "--config", str(args.config),
               "--steps", str(steps), "--warmup", str(warm), "--no-cpu", "--eager",
               "--no-traffic", "--calib-copy", str(mib), "--rotate-mb", "64"] + \
            (["--general"] if args.general else [])
        env = dict(os.environ, TMPDIR="/tmp")
        try:
            r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True, timeout=300)
        except subprocess.TimeoutExpired:
            return None, f"rocprofv3 {ctr} pass timed out"
        files = [os.path.join(d, f) for d, _, fs in os.walk(out) for f in fs
                 if f.endswith("counter_collection.csv")]
        if r.returncode != 0 or not files:
            return None, f"rocprofv3 {ctr} pass failed (rc {r.returncode})"
        copy, tms = [], []
        for row in csv.DictReader(open(files[0])):
            if row.get("Counter_Name") != ctr:
                continue
            v = float(row["Counter_Value"])
            name = row["Kernel_Name"]
            if "copyBuffer" in name:
                copy.append((int(row["Dispatch_Id"]), v))
            elif "tms::" in name or "_ZN3tms" in name:
                tms.append(v)
        shutil.rmtree(out, ignore_errors=True)
        if len(copy) < 3 or not tms:
            return None, f"rocprofv3 {ctr} pass: no copy or sampler dispatches"
        # the calibration copies are the run's first three copy dispatches
        # (before any input upload)
        cal = sorted(v for _, v in sorted(copy)[:3])[1]
        known_kib = mib * 1024.0   # the copy reads mib MiB and writes mib MiB
        factor = known_kib / cal
        vals[ctr] = (sum(tms) / (steps + warm), factor)
    fetch, ff = vals["FETCH_SIZE"]
    write, fw = vals["WRITE_SIZE"]
    nbytes = int(round((fetch * ff + write * fw) * 1024.0))
    note = (f"rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE in this run ({steps + warm} eager launches "
            f"each): {fetch:.1f} KiB x {ff:.3f} read + {write:.1f} KiB x {fw:.3f} written per launch, "
            f"factors from a {mib} MiB device copy")
    return nbytes, note


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              f"(rows are independent; a batch split across GPUs needs no exchange)",
              file=sys.stderr)
        sys.exit(2)
    # The traffic passes run as child processes before this one touches the GPU.
    traffic, traffic_note = (None, "not measured (--no-traffic)") if args.no_traffic \
        else measure_traffic(args)
    import torch

    from tensormark_amd import Sampler
    from tensormark_amd.sampler import ROWS_ANY, ROWS_SPARSE_MASK, mask_is_sparse, row_kinds_of

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
    n_sets = 1 if args.no_rotate else max(1, -(-args.rotate_mb * 2**20 // algo_bytes))

    def up(a_np, view=None):
        t = torch.from_numpy(np.ascontiguousarray(a_np if view is None else a_np.view(view)))
        return t.to(dev)

    keep = []   # device buffers the argument records point at
    kinds_name = None
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
        # the caller's row-kind hint, from the host-side parameters and masks
        # (a grammar engine knows how many ids each mask allows)
        if args.general:
            kinds = ROWS_ANY
        elif w.get("mask") is not None and mask_is_sparse(w["mask"]):
            kinds = ROWS_SPARSE_MASK
        else:
            kinds = row_kinds_of(w["params"])
        kinds_name = {0: "any", 1: "topk", 2: "sparse_mask"}[kinds]
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
    verified, verify_note = (None, "not checked (--no-cpu)") if args.no_cpu else verify(w, args.config, out)
    line = {
        "metric": METRICS[args.config],
        "value": round(rows_per_s, 1),
        "unit": "sequences/s" if args.config == 4 else "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt_name,
        "data": "synthetic (seeded numpy; no model)",
        "config": {"workload": name, "batch": B, "vocab": V, "launch": "graph" if graph else "eager",
                   "row_kinds": kinds_name,
                   "input_sets": n_sets, "hbm_resident_bytes": n_sets * algo_bytes,
                   "wall_s": round(wall, 4)},
        "hbm_gbps": round(achieved / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved / 1e9, 1),
            "peak": PEAK_HBM / 1e9,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
        },
        "cpu_baseline": cpu,
        "verified": verified,
        "verify_note": verify_note,
    }
    print(json.dumps(line), flush=True)
    s.close()


if __name__ == "__main__":
    main()
