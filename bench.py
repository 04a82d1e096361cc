#!/usr/bin/env python3
"""Benchmark of the logits-to-token stage on one MI355X.

Headline workload (the metric's configuration): one CBv2 decode sampling step
over B=64 rows of V=151,936 bf16 logits (N(0,3^2) plus a per-row Zipf(1.1)
log-prior), 2048-token Zipf output histories feeding presence 0.5 and
frequency 0.3 penalties, T=0.8, top-k 50, top-p 0.95, min-p 0.05, one uniform
per row.  A "step" is one lsamp_sample call over that batch.

* value: steps/s of whole steps replayed from a HIP graph.  The graph holds
  `--copies` steps over distinct copies of the input (16 x 19.4 MB, more than
  the 256 MB Infinity Cache holds), so each step reads its logits from HBM.
* kernel times: an eager pass with the library's per-kernel timing hook (HIP
  events on the launch stream, queue kept full by a leading GPU sleep).
* roofline: algorithmic bytes of one step / average launch duration of the
  step's kernel (fused mode: the one kernel, timed by HIP events around the
  graph replays on its stream; split mode: both kernels from the eager hook),
  against 8 TB/s; `traffic` is the HBM bytes per launch measured with
  rocprofv3 FETCH_SIZE / WRITE_SIZE and calibrated on a copy of known size.
* cpu_baseline: the oracle (the reference op sequence restated in C: full
  sorts, dense penalty tensors) timed on the host's cores on whole steps.

Usage: python bench.py [--gpus 1] [--steps 1600] [--warmup 160]

Exactly `--steps` steps are timed after exactly `--warmup` untimed ones: the
graph of `--copies` steps is replayed as often as it fits, and a graph of
the first `steps % copies` steps runs the rest.

`--path c1 | c3 | c4 | c5` measures the other configurations of the metric
(one JSON line each, same shape, with roofline and cpu_baseline):
* c1: one mlx-lm row of 151,936 fp32 logits, repetition 1.1 over 20, T=0.7,
  top-p 0.9 (latency-bound: also the synchronized single-launch latency);
* c3: the continuous-batching mixed step, 256 rows of 262,144 bf16 logits;
* c4: the grammar-constrained step, 64 rows of 151,936 fp32 logits with
  bitmasks (0.1% .. 100% and an EOS-only row), repetition 1.1 over 20;
* c5: textbook speculative verification (RESIDUAL) of 32 sequences x 4
  positions, target [32,4,V] and draft [32,3,V] bf16, T=0.8, top-p 0.95.

`--path top2 | logprobs | commit` measures one of the stage's other entry
points on the same batch instead (one JSON line of the same shape; the
headline line is the default `--path sample`):
* top2: lsamp_top2 over the 64 x 151,936 bf16 logits;
* logprobs: lsamp_logprobs of the sampled tokens and the top 20;
* commit: lsamp_commit of one token per row into the device penalty table
  built from the workload's histories (repetition window 64 on, counts on);
* masks: lsamp_mask_assemble of the grammar-constrained batch (64 rows of
  151,936 tokens; allowed sets of density 0.1%, 2%, 30%, 100% and one EOS-only
  row): the steady state where every row's mask is cached (value), and every
  row built from its allowed ids (the `miss` field); eager calls, since the
  host staging cannot be captured;
* verify: lsamp_verify (EXACT mode) of 32 sequences x 4 positions of 151,936
  bf16 target logits, T=0.8, top-p 0.95; with --penalties, presence 0.5 and
  frequency 0.3 over 2,048-token confirmed outputs and the window's drafts.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "mlx-swift-lm_amd"))

METRIC = "sampling steps/s + µs/step at B=64 V=151,936; achieved HBM GB/s vs 8 TB/s"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1600)
    ap.add_argument("--warmup", type=int, default=160)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--kernel-steps", type=int, default=512)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="time budget of each CPU baseline figure (all threads, one thread)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic", default=os.path.join(REPO, "profiles", "traffic_c2.json"),
                    help="measured HBM traffic per launch (rocprofv3 --pmc summary)")
    ap.add_argument("--probe", action="store_true",
                    help="counter-collection run: one copy kernel of --probe-copy-mib MiB "
                         "(the calibration), then --probe-steps eager steps; no timing")
    ap.add_argument("--probe-copy-mib", type=int, default=256)
    ap.add_argument("--probe-steps", type=int, default=32)
    ap.add_argument("--path", default="sample",
                    choices=["sample", "c1", "c3", "c4", "c5", "top2", "logprobs", "commit",
                             "verify", "masks", "step"])
    ap.add_argument("--penalties", action="store_true",
                    help="--path verify: penalty-aware windows")
    ap.add_argument("--top-k", type=int, default=20,
                    help="--path logprobs / step: top_k of the log-probabilities")
    ap.add_argument("--step-config", default="c2", choices=["c2", "c3", "c4"],
                    help="--path step: the headline batch (with a commit), or the mixed (c3) "
                         "or grammar-constrained fp32 (c4) batch (draw only), which take the "
                         "fused sampling kernel")
    return ap.parse_args()


def sample_kernel_name(launch):
    """The kernel(s) one sampling step launched (lsamp_launch_info.fused:
    2 the one-pass top-k kernel, 1 the fused kernel, 0 the two-kernel split)."""
    return {4: "k_fused", 3: "k_topk", 2: "k_topk", 1: "k_fused"}.get(launch["fused"],
                                                                       "k_stats+k_select")


def graph_runner(launches, stream):
    """`launches`: callables, each enqueueing one step on `stream`.  Returns
    run(n), which enqueues exactly n steps: a graph of all of them replayed
    n // len(launches) times, then a graph of the first n % len(launches)."""
    import torch
    R = len(launches)
    graphs = {}

    def graph_of(k):
        if k not in graphs:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for f in launches[:k]:
                    f()
            torch.cuda.synchronize()
            graphs[k] = g
        return graphs[k]

    def prepare(*counts):
        for n in counts:
            if n >= R:
                graph_of(R)
            if n % R:
                graph_of(n % R)

    def run(n):
        full, rem = divmod(n, R)
        with torch.cuda.stream(stream):
            for _ in range(full):
                graph_of(R).replay()
            if rem:
                graph_of(rem).replay()

    run.prepare = prepare
    return run


def time_steps(run, stream, steps, warmup):
    """Warm-up, then exactly `steps` steps bracketed by synchronizations;
    (wall seconds, HIP-event milliseconds on `stream`)."""
    import torch
    run.prepare(steps, warmup)
    run(warmup)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    run(steps)
    e1.record(stream)
    torch.cuda.synchronize()
    return time.perf_counter() - t0, e0.elapsed_time(e1)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline_of(step, rows, seconds, unit="steps/s", per_step=1.0):
    """The oracle as the CPU baseline: step(threads, nrows) runs one whole step
    on the first nrows rows.  Median of up to 20 timed runs after up to 3
    warm-ups, each figure bounded by `seconds`: with every thread of the box's
    share (min(16, nproc)) over all rows, and with one thread over as many
    rows as fit the budget (scaled to the whole step).  value = per_step /
    median seconds of a whole step."""
    nproc = os.cpu_count() or 1
    threads = max(1, min(16, nproc))

    def figure(th, nrows):
        t0 = time.perf_counter()
        step(th, nrows)
        first = time.perf_counter() - t0
        warm = 0 if first * 4 > seconds else 2
        for _ in range(warm):
            step(th, nrows)
        ts, t_all = [], time.perf_counter()
        while len(ts) < 20 and (time.perf_counter() - t_all) < seconds or len(ts) < 3:
            t0 = time.perf_counter()
            step(th, nrows)
            ts.append(time.perf_counter() - t0)
        med = sorted(ts)[len(ts) // 2]
        return med * rows / nrows, len(ts), warm + 1

    t_all, n_all, w_all = figure(threads, rows)
    # one thread: enough rows for about a second per run
    per_row = t_all * threads / rows
    n1 = int(max(1, min(rows, 1.0 / max(per_row, 1e-6))))
    t_one, n_one, w_one = figure(1, n1)
    return {"value": per_step / t_all, "unit": unit, "cores": threads, "kind": "port",
            "nproc": nproc, "host": cpu_model(),
            "sample": f"median of {n_all} whole steps ({rows} rows) after {w_all} warm-up(s), "
                      f"rows over {threads} threads; ms/step {1e3 * t_all:.2f}",
            "one_thread": {"value": per_step / t_one, "unit": unit,
                           "sample": f"median of {n_one} runs over {n1} of {rows} rows after "
                                     f"{w_one} warm-up(s), scaled to the step; "
                                     f"ms/step {1e3 * t_one:.2f}"}}


def bench_aux(args):
    """One JSON line for lsamp_top2 / lsamp_logprobs / lsamp_commit on the
    headline batch: launches per second from a HIP graph of `--copies`
    launches over distinct input copies, the launch duration from HIP events
    on the launch stream, and the oracle timed on the host as the baseline."""
    import numpy as np
    import torch

    from lsamp import _ffi, workloads as W
    from lsamp.api import Context, PenaltyTable
    from lsamp.history import Cbv2RowState

    if args.path == "verify":
        return bench_verify(args)
    if args.path == "masks":
        return bench_masks(args)
    if args.path in ("c1", "c3", "c4"):
        return bench_config(args, int(args.path[1]))
    if args.path == "c5":
        return bench_c5(args)
    if args.path == "step":
        return bench_step(args)
    cfg = W.config2()
    B, V, R = cfg["rows"], cfg["vocab"], args.copies
    steps, warm = args.steps, args.warmup
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(11)
    ctx = Context(0, max_rows=B, max_vocab=V)
    base = torch.from_numpy(cfg["logits"].view(np.int16)).view(torch.bfloat16)
    copies = torch.empty((R, B, V), dtype=torch.bfloat16, device=dev)
    for i in range(R):
        copies[i].copy_(base)
        if i:
            idx = torch.from_numpy(rng.integers(0, V, B)).to(dev)
            copies[i, torch.arange(B, device=dev), idx] = 0.0
    tokens = torch.from_numpy(rng.integers(0, V, (R, B)).astype(np.int32)).to(dev)
    if args.path == "top2":
        preps = [ctx.prepare_top2(copies[i]) for i in range(R)]
        launch = preps[0].launch
        alg = B * V * 2 + B * 2 * 8
        unit_name, kernel = "top-2 rows/s", "k_rank"
    elif args.path == "logprobs":
        preps = [ctx.prepare_logprobs(copies[i], tokens=tokens[i], top_k=args.top_k)
                 for i in range(R)]
        alg = B * V * 2 + B * 4 + B * 4 + B * args.top_k * 8 + B * 4
        unit_name, kernel = "log-prob rows/s", "k_rank"
    else:
        # the workload's output histories, as a device table with room to grow
        states = []
        for r in range(B):
            e = cfg["entries"][cfg["row_ptr"][r]:cfg["row_ptr"][r + 1]]
            hist = np.repeat(e["token"], e["count"])
            states.append(Cbv2RowState(prompt=[], output=rng.permutation(hist), repetition_window=64,
                                       repetition_on=True, counts_on=True, vocab=V))
        cap = max(len(st.entries()) for st in states) + steps + warm + 2 * R + 16
        table = PenaltyTable(states, capacity=cap, window_capacity=64)
        # tokens to commit: drawn from each row's own history (mostly repeats)
        for r in range(B):
            e = cfg["entries"][cfg["row_ptr"][r]:cfg["row_ptr"][r + 1]]
            tokens[:, r] = torch.from_numpy(rng.choice(e["token"], R).astype(np.int32)).to(dev)

        class _Commit:
            def __init__(self, i):
                self.i = i

            def launch(self, stream=None):
                table.commit(ctx, tokens[self.i], V, stream)
        preps = [_Commit(i) for i in range(R)]
        n_ent = int(table.row_len.sum().item())
        alg = n_ent * 16 + B * (4 * 8 + 64 * 4)
        unit_name, kernel = "commit rows/s", "k_commit"
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for p in preps:
            p.launch(stream.cuda_stream)
    torch.cuda.synchronize()
    run = graph_runner([(lambda p=p: p.launch(stream.cuda_stream)) for p in preps], stream)
    wall_s, ev_ms = time_steps(run, stream, steps, warm)
    launch_us = 1e3 * ev_ms / steps
    achieved = alg / (launch_us * 1e-6) / 1e9
    out = {
        "metric": f"{unit_name} at B={B} V={V} (lsamp_{args.path})",
        "value": B * steps / wall_s, "unit": "rows/s", "n_gpus": 1, "steps": steps,
        "warmup": warm, "ms_per_step": 1e3 * wall_s / steps, "us_per_launch": launch_us,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u32" if args.path != "logprobs" else "f32", "data": "synthetic",
        "config": {"workload": f"lsamp_{args.path} B={B} V={V} bf16" +
                   (f" top_k={args.top_k}" if args.path == "logprobs" else ""),
                   "input_copies": R},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes": alg,
                     "kernel": kernel, "launch_us": launch_us},
        "cpu_baseline": None,
    }
    if not args.no_cpu and args.path != "commit":
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O
        kw = dict(dtype=_ffi.DTYPE_BF16, k=2 if args.path == "top2" else args.top_k,
                  raw_values=args.path == "top2",
                  tokens=None if args.path == "top2" else tokens[0].cpu().numpy())
        n, t0 = 0, time.perf_counter()
        while True:
            O.rank(cfg["logits"], **kw)
            n += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds and n >= 3:
                break
        out["cpu_baseline"] = {"value": B * n / el, "unit": "rows/s", "cores": 1, "kind": "port",
                               "sample": f"{n} whole batches of {B} rows in {el:.1f} s, one thread"}
    ctx.close()
    print(json.dumps(out))
    return 0


def bench_step(args):
    """One JSON line for lsamp_step on the headline batch (CBv2DefaultSampler.
    sample: draw, penalty commit into a device table, raw log-probabilities
    of the drawn tokens and the top --top-k): steps/s from a HIP graph of
    `--copies` steps over distinct input copies, with and without the
    log-probabilities, so the line shows what they cost.  The draw reads the
    headline batch's penalty entries and the commit writes a table built from
    the same histories: replaying fixed logits through a table that the draw
    also read would pile penalties onto the drawn tokens step after step and
    grow every row's history without bound, a workload no decode loop has."""
    import numpy as np
    import torch

    from lsamp import workloads as W
    from lsamp.api import Context, PenaltyTable
    from lsamp.history import Cbv2RowState

    if args.step_config != "c2":
        return bench_step_fused(args)
    cfg = W.config2()
    B, V, R = cfg["rows"], cfg["vocab"], args.copies
    steps, warm = args.steps, args.warmup
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(12)
    ctx = Context(0, max_rows=B, max_vocab=V)
    base = torch.from_numpy(cfg["logits"].view(np.int16)).view(torch.bfloat16)
    copies = torch.empty((R, B, V), dtype=torch.bfloat16, device=dev)
    for i in range(R):
        copies[i].copy_(base)
        if i:
            idx = torch.from_numpy(rng.integers(0, V, B)).to(dev)
            copies[i, torch.arange(B, device=dev), idx] = 0.0
    u = torch.from_numpy(cfg["uniforms"]).to(dev)

    def table():
        states = []
        for r in range(B):
            e = cfg["entries"][cfg["row_ptr"][r]:cfg["row_ptr"][r + 1]]
            hist = np.repeat(e["token"], e["count"])
            states.append(Cbv2RowState(prompt=[], output=np.random.default_rng(r).permutation(hist),
                                       repetition_window=64, repetition_on=False, counts_on=True,
                                       vocab=V))
        cap = max(len(st.entries()) for st in states) + steps + warm + 2 * R + 64
        return PenaltyTable(states, capacity=cap, window_capacity=64)

    stream = torch.cuda.Stream(device=dev)
    res = {}
    for k in (args.top_k, -1):
        t = table()
        preps = [ctx.prepare_step(copies[i], cfg["params"], table=t, uniforms=u, logprobs_top_k=k,
                                  draw_from_table=False, row_ptr=cfg["row_ptr"],
                                  entries=cfg["entries"])
                 for i in range(R)]
        with torch.cuda.stream(stream):
            for p in preps:
                p.launch(stream.cuda_stream)
        torch.cuda.synchronize()
        launch = ctx.last_launch()
        run = graph_runner([(lambda p=p: p.launch(stream.cuda_stream)) for p in preps], stream)
        wall_s, ev_ms = time_steps(run, stream, steps, warm)
        res[k] = (wall_s, 1e3 * ev_ms / steps, launch)
        del preps, run, t
        torch.cuda.synchronize()
    wall_s, us, launch = res[args.top_k]
    wall0, us0, launch0 = res[-1]
    kinds = {3: "k_topk with raw log-probabilities + k_commit", 2: "k_topk + k_commit + k_rank"}
    out = {
        "metric": f"decode steps/s with raw log-probabilities (top {args.top_k}) at B={B} V={V} "
                  "(lsamp_step)",
        "value": steps / wall_s, "unit": "steps/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": 1e3 * wall_s / steps, "us_per_step_events": us,
        "us_per_step_without_logprobs": us0, "logprob_cost_ratio": us / us0,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["workload"] + f" + commit + log-probs top {args.top_k}",
                   "input_copies": R,
                   "kernels": kinds.get(launch["fused"], sample_kernel_name(launch)) ,
                   "kernels_without_logprobs": sample_kernel_name(launch0) + " + k_commit"},
        "roofline": None, "cpu_baseline": None,
    }
    ctx.close()
    print(json.dumps(out))
    return 0


def bench_step_fused(args):
    """lsamp_step (draw + raw log-probabilities, no commit) on the mixed
    (c3) or grammar-constrained fp32 (c4) batch, whose rows take the fused
    sampling kernel: with the log-probabilities it ranks the raw logits in
    its own pass (launch kind 4), so the line's ratio is what they cost in
    that pass; `lsamp_logprobs` alone on the same batch is timed beside it
    (the second pass the step no longer makes)."""
    import numpy as np
    import torch

    from lsamp import _ffi, workloads as W
    from lsamp.api import Context

    n = int(args.step_config[1])
    cfg = W.WORKLOADS[n]()
    B, V = cfg["rows"], cfg["vocab"]
    R = args.copies if n != 3 else min(args.copies, 4)
    steps, warm = args.steps, args.warmup
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(30 + n)
    if cfg["dtype"] == _ffi.DTYPE_F32:
        base = torch.from_numpy(np.ascontiguousarray(cfg["logits"], np.float32))
        tdt = torch.float32
    else:
        base = torch.from_numpy(cfg["logits"].view(np.int16)).view(torch.bfloat16)
        tdt = torch.bfloat16
    copies = torch.empty((R, B, V), dtype=tdt, device=dev)
    for i in range(R):
        copies[i].copy_(base)
        if i:
            idx = torch.from_numpy(rng.integers(0, V, B)).to(dev)
            copies[i, torch.arange(B, device=dev), idx] = 0.0
    ctx = Context(0, max_rows=B, max_vocab=V)
    assert cfg["semantics"] == _ffi.SEM_CBV2  # (lsamp_step is the CBv2 step)
    kw = dict(row_ptr=cfg.get("row_ptr"), entries=cfg.get("entries"), uniforms=cfg["uniforms"])
    if cfg.get("bitmask") is not None:
        kw.update(bitmask=cfg["bitmask"], mask_bits=cfg["mask_bits"],
                  mask_tail=cfg.get("mask_tail", 0))
    stream = torch.cuda.Stream(device=dev)
    res = {}
    for k in (args.top_k, -1):
        preps = [ctx.prepare_step(copies[i], cfg["params"], logprobs_top_k=k, **kw)
                 for i in range(R)]
        with torch.cuda.stream(stream):
            for p in preps:
                p.launch(stream.cuda_stream)
        torch.cuda.synchronize()
        launch = ctx.last_launch()
        run = graph_runner([(lambda p=p: p.launch(stream.cuda_stream)) for p in preps], stream)
        wall_s, ev_ms = time_steps(run, stream, steps, warm)
        res[k] = (wall_s, 1e3 * ev_ms / steps, launch)
        del preps, run
        torch.cuda.synchronize()
    # the second pass alone (lsamp_logprobs), which the step no longer makes
    tok = torch.zeros(B, dtype=torch.int32, device=dev)
    lps = [ctx.prepare_logprobs(copies[i], tokens=tok, top_k=args.top_k) for i in range(R)]
    with torch.cuda.stream(stream):
        for p in lps:
            p.launch(stream.cuda_stream)
    torch.cuda.synchronize()
    run = graph_runner([(lambda p=p: p.launch(stream.cuda_stream)) for p in lps], stream)
    _, ev_lp = time_steps(run, stream, steps, warm)
    wall_s, us, launch = res[args.top_k]
    wall0, us0, launch0 = res[-1]
    out = {
        "metric": f"sampling steps/s with raw log-probabilities (top {args.top_k}) at B={B} V={V} "
                  "(lsamp_step, fused sampling kernel)",
        "value": steps / wall_s, "unit": "steps/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": 1e3 * wall_s / steps, "us_per_step_events": us,
        "us_per_step_without_logprobs": us0, "logprob_cost_ratio": us / us0,
        "us_second_pass_lsamp_logprobs": 1e3 * ev_lp / steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["workload"] + f" + log-probs top {args.top_k} (no commit)",
                   "input_copies": R, "launch": launch, "launch_without_logprobs": launch0,
                   "kernels": sample_kernel_name(launch) +
                   (" with raw log-probabilities" if launch["fused"] == 4 else " + k_rank")},
        "roofline": None, "cpu_baseline": None,
    }
    ctx.close()
    print(json.dumps(out))
    return 0


def bench_masks(args):
    """lsamp_mask_assemble on the grammar-constrained batch: per-call duration
    from HIP events on the launch stream (descriptor copy + assembly) and
    calls per second by the host clock, for the all-cached and all-built
    steps; the oracle's assembly timed on the host as the baseline."""
    import numpy as np
    import torch

    from lsamp.api import Context
    from lsamp.constraint import ConstraintMasks, MaskPlan

    B, V = 64, 151936
    rng = np.random.default_rng(4)
    cm = ConstraintMasks(B, V)
    words = cm.words
    dens = [0.001, 0.02, 0.3, 1.0]
    sets = [np.sort(rng.choice(V, max(1, int(V * dens[r % 4])), replace=False)).astype(np.int32)
            for r in range(B - 1)] + [np.array([151645], np.int32)]
    ptr = np.concatenate([[0], np.cumsum([len(x) for x in sets])]).astype(np.int32)
    ids = np.concatenate(sets)
    src = np.arange(B, dtype=np.int32)
    miss = MaskPlan(src, np.ones(B, np.uint8), ptr, ids)
    hit = MaskPlan(src, np.zeros(B, np.uint8), np.zeros(B + 1, np.int32), np.zeros(0, np.int32))
    ctx = Context(0, max_rows=B, max_vocab=V)
    dev = torch.device("cuda", 0)
    pool = torch.zeros((cm.pool_rows, words), dtype=torch.int32, device=dev)
    outs = [torch.empty((B, words), dtype=torch.int32, device=dev) for _ in range(2)]
    stream = torch.cuda.Stream(device=dev)
    res = {}
    for name, plan in (("miss", miss), ("hit", hit)):
        for i in range(args.warmup):
            ctx.assemble_masks(plan, pool, V, out=outs[i & 1], stream=stream.cuda_stream)
        torch.cuda.synchronize()
        n = args.steps
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(n):
            ctx.assemble_masks(plan, pool, V, out=outs[i & 1], stream=stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        res[name] = (n, wall, 1e3 * e0.elapsed_time(e1) / n)
    row_bytes = words * 4
    alg_hit = B * 2 * row_bytes + B * 5
    alg_miss = 4 * len(ids) + B * 2 * row_bytes + B * 9
    n, wall, us = res["hit"]
    achieved = alg_hit / (us * 1e-6) / 1e9
    nm, wallm, usm = res["miss"]
    out = {
        "metric": f"grammar bitmask steps/s at B={B} V={V} (lsamp_mask_assemble)",
        "value": n / wall, "unit": "steps/s", "n_gpus": 1, "steps": n, "warmup": args.warmup,
        "ms_per_step": 1e3 * wall / n, "us_per_launch": us, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u32", "data": "synthetic",
        "config": {"workload": f"grammar masks B={B} V={V} densities 0.1/2/30/100% + EOS-only, "
                               "every row cached"},
        "miss": {"steps_per_s": nm / wallm, "us_per_launch": usm, "ids": int(len(ids)),
                 "algorithmic_bytes": alg_miss,
                 "achieved_GBps": alg_miss / (usm * 1e-6) / 1e9},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes": alg_hit,
                     "kernel": "k_mask_assemble (+ descriptor copy)", "launch_us": us},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O
        opool = np.zeros((cm.pool_rows, words), np.uint32)
        O.assemble_masks(miss, opool, V)   # fills the cache rows (untimed)
        k, t0 = 0, time.perf_counter()
        while True:
            O.assemble_masks(hit, opool, V)
            k += 1
            el = time.perf_counter() - t0
            if el >= min(args.cpu_seconds, 5.0) and k >= 3:
                break
        out["cpu_baseline"] = {"value": k / el, "unit": "steps/s", "cores": 1, "kind": "port",
                               "sample": f"{k} all-cached assemblies of the same batch in "
                                         f"{el:.1f} s, one thread"}
    ctx.close()
    print(json.dumps(out))
    return 0


def tokens_check(baseline, gpu_tokens, seen):
    """Compare the GPU's tokens for the workload's own input copy with the
    oracle's from the baseline's whole-step runs; the result goes into the
    baseline object and the caller's exit status."""
    import numpy as np

    want = seen.get("tokens")
    if want is None:
        baseline["tokens_match"] = None
        return True
    got = np.asarray(gpu_tokens)
    bad = np.flatnonzero(got != want)
    baseline["tokens_match"] = bool(bad.size == 0)
    if bad.size:
        baseline["tokens_mismatch_rows"] = bad[:8].tolist()
    return bad.size == 0


def cpu_baseline(cfg, seconds, gpu_tokens):
    """The oracle on whole steps of the headline workload (cpu_baseline_of),
    and its tokens checked against the GPU's (tokens_check)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    seen = {}

    def step(threads, nrows):
        rp = cfg["row_ptr"]
        res = O.sample(semantics=cfg["semantics"], logits=cfg["logits"][:nrows],
                       dtype=cfg["dtype"], params=cfg["params"][:nrows],
                       row_ptr=rp[:nrows + 1] - rp[0], entries=cfg["entries"][rp[0]:rp[nrows]],
                       uniforms=cfg["uniforms"][:nrows], threads=threads)
        if nrows == cfg["rows"]:
            seen["tokens"] = res["tokens"]

    base = cpu_baseline_of(step, cfg["rows"], seconds)
    return base, tokens_check(base, gpu_tokens, seen)


def bench_config(args, n):
    """Configuration 1, 3 or 4 of the metric: steps/s from HIP-graph replays
    over `--copies` distinct input copies (c1: a single row, so copies are
    cheap), the step duration from HIP events on the launch stream, and the
    oracle on the same workload as the CPU baseline."""
    import numpy as np
    import torch

    from lsamp import _ffi, workloads as W
    from lsamp.api import Context

    cfg = W.WORKLOADS[n]()
    B, V = cfg["rows"], cfg["vocab"]
    R = args.copies if n != 3 else min(args.copies, 4)  # c3 copies are 134 MB each
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(100 + n)
    if cfg["dtype"] == _ffi.DTYPE_F32:
        base = torch.from_numpy(np.ascontiguousarray(cfg["logits"], np.float32))
        tdt = torch.float32
    else:
        base = torch.from_numpy(cfg["logits"].view(np.int16)).view(torch.bfloat16)
        tdt = torch.bfloat16
    copies = torch.empty((R, B, V), dtype=tdt, device=dev)
    for i in range(R):
        copies[i].copy_(base)
        if i:  # one perturbed token per row: no two copies share every line
            idx = torch.from_numpy(rng.integers(0, V, B)).to(dev)
            copies[i, torch.arange(B, device=dev), idx] = 0.0
    ctx = Context(0, max_rows=B, max_vocab=V)
    kw = dict(semantics=cfg["semantics"], row_ptr=cfg.get("row_ptr"), entries=cfg.get("entries"),
              uniforms=cfg["uniforms"])
    if cfg.get("bitmask") is not None:
        kw.update(bitmask=cfg["bitmask"], mask_bits=cfg["mask_bits"], mask_tail=cfg.get("mask_tail", 0))
    preps = [ctx.prepare_sample(copies[i], cfg["params"], **kw) for i in range(R)]
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for p in preps:
            p.launch(stream.cuda_stream)
    torch.cuda.synchronize()
    run = graph_runner([(lambda p=p: p.launch(stream.cuda_stream)) for p in preps], stream)
    wall_s, ev_ms = time_steps(run, stream, args.steps, args.warmup)
    launch = ctx.last_launch()
    step_us = 1e3 * ev_ms / args.steps
    alg = W.algorithmic_bytes(cfg)
    achieved = alg / (step_us * 1e-6) / 1e9
    out = {
        "metric": METRIC.replace("B=64 V=151,936", f"B={B} V={V:,}"),
        "value": args.steps / wall_s, "unit": "steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1e3 * wall_s / args.steps,
        "us_per_step_events": step_us, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": cfg["workload"], "rows": B, "vocab": V,
                   "logits_dtype": "fp32" if cfg["dtype"] == _ffi.DTYPE_F32 else "bf16",
                   "semantics": "mlx-lm" if cfg["semantics"] == _ffi.SEM_MLXLM else "CBv2",
                   "input_copies": R},
        "launch": launch,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes": alg,
                     "kernel": sample_kernel_name(launch),
                     "launch_us": step_us},
        "cpu_baseline": None,
    }
    if n == 1:
        # single-launch latency: each launch waited for before the next
        lat = []
        for i in range(max(20, min(args.steps, 200))):
            t0 = time.perf_counter()
            preps[i % R].launch(stream.cuda_stream)
            stream.synchronize()
            lat.append(time.perf_counter() - t0)
        out["single_launch_us"] = 1e6 * sorted(lat)[len(lat) // 2]
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O

        seen = {}

        def step(threads, nrows):
            r = slice(0, nrows)
            rp = cfg.get("row_ptr")
            kw2 = {}
            if rp is not None:
                kw2["row_ptr"] = rp[:nrows + 1] - rp[0]
                kw2["entries"] = cfg["entries"][rp[0]:rp[nrows]]
            if cfg.get("bitmask") is not None:
                kw2.update(bitmask=cfg["bitmask"][r], mask_bits=cfg["mask_bits"],
                           mask_tail=cfg.get("mask_tail", 0))
            res = O.sample(semantics=cfg["semantics"], logits=cfg["logits"][r],
                           dtype=cfg["dtype"], params=cfg["params"][r],
                           uniforms=cfg["uniforms"][r], threads=threads, **kw2)
            if nrows == B:
                seen["tokens"] = res["tokens"]

        out["cpu_baseline"] = cpu_baseline_of(step, B, args.cpu_seconds)
        ok = tokens_check(out["cpu_baseline"], preps[0].tokens.cpu().numpy(), seen)
        out["tokens_match"] = out["cpu_baseline"]["tokens_match"]
    ctx.close()
    print(json.dumps(out))
    return 0 if args.no_cpu or ok else 1


def bench_c5(args):
    """Configuration 5: textbook speculative verification (lsamp_verify,
    RESIDUAL) of 32 sequences x 4 positions with draft logits.  The drafts
    are the draft rows' own draws (lsamp_sample with the draft uniforms,
    outside the timed region)."""
    import numpy as np
    import torch

    from lsamp import _ffi, workloads as W
    from lsamp.api import Context

    cfg = W.config5()
    S, Wn, V = cfg["sequences"], cfg["window"], cfg["vocab"]
    D = Wn - 1
    R = min(args.copies, 4)
    dev = torch.device("cuda", 0)
    ctx = Context(0, max_rows=S * (2 * Wn - 1), max_vocab=V)
    tgt = torch.from_numpy(cfg["target"].view(np.int16)).view(torch.bfloat16)
    dft = torch.from_numpy(cfg["draft"].view(np.int16)).view(torch.bfloat16)
    tc = torch.empty((R, S, Wn, V), dtype=torch.bfloat16, device=dev)
    dc = torch.empty((R, S, D, V), dtype=torch.bfloat16, device=dev)
    for i in range(R):
        tc[i].copy_(tgt)
        dc[i].copy_(dft)
    drafts = ctx.sample(dc[0].reshape(S * D, V), np.repeat(cfg["params"], D),
                        semantics=_ffi.SEM_CBV2,
                        uniforms=cfg["draft_uniforms"].reshape(-1))["tokens"].reshape(S, D)
    torch.cuda.synchronize()
    preps = [ctx.prepare_verify(tc[i], dc[i], drafts, cfg["params"], cfg["uniforms"],
                                mode=_ffi.VERIFY_RESIDUAL) for i in range(R)]
    stream = torch.cuda.Stream(device=dev)
    for p_ in preps:
        p_.launch(stream.cuda_stream)
    torch.cuda.synchronize()
    run = graph_runner([(lambda p=p_: p.launch(stream.cuda_stream)) for p_ in preps], stream)
    wall_s, ev_ms = time_steps(run, stream, args.steps, args.warmup)
    us = 1e3 * ev_ms / args.steps
    alg = W.algorithmic_bytes(cfg)
    achieved = alg / (us * 1e-6) / 1e9
    out = {
        "metric": f"MTP verify windows/s at S={S} W={Wn} V={V:,} (lsamp_verify RESIDUAL); "
                  "achieved HBM GB/s vs 8 TB/s",
        "value": args.steps / wall_s, "unit": "verifies/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1e3 * wall_s / args.steps, "us_per_launch": us,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["workload"] + " RESIDUAL, draft [S,W-1,V] bf16",
                   "input_copies": R},
        "launch": ctx.last_launch(),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes": alg,
                     "kernel": "k_fused + k_verify_finish", "launch_us": us},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O
        dnp = drafts.cpu().numpy()
        seen = {}

        def step(threads, nseq):
            res = O.verify(mode=_ffi.VERIFY_RESIDUAL, target=cfg["target"][:nseq],
                           draft=cfg["draft"][:nseq], draft_tokens=dnp[:nseq],
                           dtype=_ffi.DTYPE_BF16, params=cfg["params"][:nseq],
                           uniforms=cfg["uniforms"][:nseq], threads=threads)
            if nseq == S:
                seen["tokens"] = res["tokens"].reshape(-1)

        out["cpu_baseline"] = cpu_baseline_of(step, S, args.cpu_seconds, unit="verifies/s")
        ok = tokens_check(out["cpu_baseline"], preps[0].tokens.cpu().numpy().reshape(-1), seen)
        out["tokens_match"] = out["cpu_baseline"]["tokens_match"]
    ctx.close()
    print(json.dumps(out))
    return 0 if args.no_cpu or ok else 1


def bench_verify(args):
    """lsamp_verify on the MTP verify configuration, HIP-graph timed."""
    import numpy as np
    import torch

    from lsamp import _ffi, workloads as W
    from lsamp.api import Context
    from lsamp.history import Cbv2RowState, csr

    cfg = W.config5()
    S, Wn, V = cfg["sequences"], cfg["window"], cfg["vocab"]
    R = 4
    steps, warm = args.steps, args.warmup
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(13)
    ctx = Context(0, max_rows=S * (2 * Wn - 1), max_vocab=V)
    base = torch.from_numpy(cfg["target"].view(np.int16)).view(torch.bfloat16)
    copies = torch.empty((R, S, Wn, V), dtype=torch.bfloat16, device=dev)
    for i in range(R):
        copies[i].copy_(base)
    drafts = rng.integers(0, V, (S, Wn - 1)).astype(np.int32)
    params = cfg["params"]
    kw = {}
    alg = S * Wn * V * 2 + S * Wn * 12
    if args.penalties:
        p = W.resolve_cbv2(temperature=0.8, top_p=0.95, presence_penalty=0.5,
                           frequency_penalty=0.3, vocab=V)
        params = W._params([p] * S)
        cdf = W._zipf_cdf(1.1, V)
        ents = []
        for s in range(S):
            hist = rng.permutation(V)[W.zipf_ranks(rng, 1.1, V, 2048, cdf)]
            ents.append(Cbv2RowState(prompt=[], output=hist, repetition_window=64,
                                     repetition_on=False, counts_on=True, vocab=V).entries())
        rp, en = csr(ents)
        kw = dict(penalty_row_ptr=rp, penalty_entries=en)
        alg += len(en) * 16 * (1 + Wn)
    preps = [ctx.prepare_verify(copies[i], None, drafts, params, cfg["uniforms"],
                                mode=_ffi.VERIFY_EXACT, **kw) for i in range(R)]
    stream = torch.cuda.Stream(device=dev)
    for p_ in preps:
        p_.launch(stream.cuda_stream)
    torch.cuda.synchronize()
    run = graph_runner([(lambda p=p_: p.launch(stream.cuda_stream)) for p_ in preps], stream)
    wall_s, ev_ms = time_steps(run, stream, steps, warm)
    us = 1e3 * ev_ms / steps
    achieved = alg / (us * 1e-6) / 1e9
    out = {
        "metric": f"MTP verify windows/s at S={S} W={Wn} V={V} (lsamp_verify EXACT"
                  + (", penalties)" if args.penalties else ")"),
        "value": steps / wall_s, "unit": "verifies/s", "n_gpus": 1, "steps": steps,
        "warmup": warm, "ms_per_step": 1e3 * wall_s / steps, "us_per_launch": us,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["workload"] + (" pres0.5 freq0.3 2048-token outputs"
                                                  if args.penalties else ""),
                   "input_copies": R},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes": alg,
                     "kernel": "k_window_entries + k_fused + k_verify_finish" if args.penalties
                     else "k_fused + k_verify_finish", "launch_us": us},
        "cpu_baseline": None,
    }
    ctx.close()
    print(json.dumps(out))
    return 0


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one GPU only: the sampling stage is row-parallel and needs no "
              "collective; multi-GPU runs are not part of this build.", file=sys.stderr)
        return 2
    if args.path != "sample":
        return bench_aux(args)
    import numpy as np
    import torch

    from lsamp import _ffi, workloads as W
    from lsamp.api import Context

    cfg = W.config2()
    B, V, R = cfg["rows"], cfg["vocab"], args.copies
    steps, warm = args.steps, args.warmup
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(7)
    base = torch.from_numpy(cfg["logits"].view(np.int16)).view(torch.bfloat16)
    # R copies in HBM: copy 0 is the workload itself, the others perturb
    # one random token per row so no two copies share cache lines' contents
    copies = torch.empty((R, B, V), dtype=torch.bfloat16, device=dev)
    for i in range(R):
        copies[i].copy_(base)
        if i:
            idx = torch.from_numpy(rng.integers(0, V, B)).to(dev)
            copies[i, torch.arange(B, device=dev), idx] = 0.0
    uniforms = torch.from_numpy(rng.random((R, B), dtype=np.float32)).to(dev)
    uniforms[0] = torch.from_numpy(cfg["uniforms"]).to(dev)
    ctx = Context(0, max_rows=B, max_vocab=V)
    preps = [ctx.prepare_sample(copies[i], cfg["params"], semantics=cfg["semantics"],
                                row_ptr=cfg["row_ptr"], entries=cfg["entries"],
                                uniforms=uniforms[i]) for i in range(R)]
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for p in preps:
            p.launch()
    torch.cuda.synchronize()

    if args.probe:
        # a plain device-to-device copy of known size calibrates the traffic
        # counters; then eager steps, each reading a distinct input copy
        n = args.probe_copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for i in range(args.probe_steps):
                preps[i % R].launch()
        torch.cuda.synchronize()
        print(json.dumps({"probe": True, "copy_bytes": n, "steps": args.probe_steps,
                          "launch": ctx.last_launch(),
                          "algorithmic_bytes": W.algorithmic_bytes(cfg)}))
        ctx.close()
        return 0

    # warm-up, then exactly `steps` steps (graphs over the input copies)
    run = graph_runner([(lambda p=p: p.launch()) for p in preps], stream)
    wall_s, ev_ms = time_steps(run, stream, steps, warm)
    us_step = 1e6 * wall_s / steps

    # per-kernel durations: eager launches with the timing hook, queue kept full
    kn = min(args.kernel_steps, 4096)
    ctx.set_timing(True)
    with torch.cuda.stream(stream):
        torch.cuda._sleep(50_000_000)
        for i in range(kn):
            preps[i % R].launch()
    torch.cuda.synchronize()
    k1_ms, k2_ms, n_timed = ctx.read_timing()
    ctx.set_timing(False)
    launch = ctx.last_launch()
    k1_us = 1e3 * k1_ms / n_timed
    k2_us = 1e3 * k2_ms / n_timed
    # eager launches, each bracketed by the library's timing-hook events: a
    # per-launch figure that includes the hook's own event overhead, outside
    # the timed region (the roofline uses the timed region's events)
    if launch["fused"]:
        dom_name = sample_kernel_name(launch)
        eager_hook_us = {dom_name: k1_us, "timed_calls": n_timed}
        dom_us = k1_us
    else:
        eager_hook_us = {"k_stats": k1_us, "k_select": k2_us, "timed_calls": n_timed}
        dom_name, dom_us = "k_stats+k_select", k1_us + k2_us

    # the tokens of the copy that is the workload itself (checked against
    # the oracle in the CPU-baseline leg)
    tok0 = preps[0].tokens.cpu().numpy()

    alg_bytes = W.algorithmic_bytes(cfg)
    # The timed region is back-to-back launches of the step on one stream
    # (HIP events on that stream bracket it); in fused mode a step is exactly
    # one launch of the dominant kernel, so its average launch duration is the
    # events' time per step.  (The eager hook's per-launch figure above also
    # counts each launch's own event overhead.)
    launch_us = 1e3 * ev_ms / steps if launch["fused"] else dom_us
    achieved = alg_bytes / (launch_us * 1e-6) / 1e9
    traffic = None
    if args.traffic and os.path.exists(args.traffic):
        with open(args.traffic) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": steps / wall_s,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": 1e3 * wall_s / steps,
        "us_per_step": us_step,
        "us_per_step_events": 1e3 * ev_ms / steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "rows": B, "vocab": V, "logits_dtype": "bf16",
                   "semantics": "CBv2", "input_copies": R, "graph_steps_per_replay": R},
        "eager_hook_us": eager_hook_us,
        "launch": launch,
        "step_effective_GBps": alg_bytes / (us_step * 1e-6) / 1e9,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "algorithmic_bytes": alg_bytes, "kernel": dom_name, "launch_us": launch_us},
        "tokens_copy0_head": tok0[:4].tolist(),
    }
    ok = True
    if not args.no_cpu:
        out["cpu_baseline"], ok = cpu_baseline(cfg, args.cpu_seconds, tok0)
        out["tokens_match"] = out["cpu_baseline"]["tokens_match"]
    else:
        out["cpu_baseline"] = None
    ctx.close()
    print(json.dumps(out))
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
