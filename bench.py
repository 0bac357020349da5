#!/usr/bin/env python3
"""Benchmark of the gfx950 routing chain (one MI355X).

Headline: chain_from_tokens at T=4096, E=64, K=256, N=128 (FP32). After
--warmup untimed chains, exactly --steps chains run in at most 20 batches;
each batch is one HIP-event span divided by its size (reference runner
semantics, benchmarks/core/runner.cpp:218-236, 283-411) and value = T / p50
of the batch means. Each fused launch and each stage operator is also timed
alone, 50 back-to-back calls recorded into one HIP graph (no host submission
between them), and priced against its roofline with the algorithmic work
model (minimum unique traffic / GEMM flops). Extras measured in the same run:
the Mixtral-shaped grouped GEMM + permute + unpermute (C4, aligned and
non-aligned; permute / unpermute warm and cold), the fine-grained chain (C5),
the histogram-scan stress (C3, with the launch floor beside it), chain graphs
of 1 / 10 / 50 chains against direct calls. The CPU baseline is the reference
CPU oracle chain restated in oracle/ (single thread), timed on the host on the
same headline workload.

Runner mode (`--suite NAME` or `--operator NAME` with `--param key=value ...`,
`--variant`, `--cache-mode warm|cold_scrub`, `--samples`, `--kernel-repeats`,
`--profile-once`; reference benchmarks/benchmark_main.cpp:16-33) times any
shape and prints one record of the same form.

Prints one JSON line. `--gpus N` with N > 1 exits with a message: this build
runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, vendor peak
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix, vendor peak
RIDGE = FP32_MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)  # flop/byte


SUITES = ("chain_from_tokens", "chain_from_logits", "chain_from_route_ids")
OPERATORS = ("dense_gemm", "topk_gate", "histogram", "exclusive_scan", "histogram_exclusive_scan",
             "token_permute", "grouped_gemm", "unpermute")


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed calls before timing (default 20; runner mode: 5, the reference runner's)")
    ap.add_argument("--quick", action="store_true",
                    help="no CPU baseline and no extras unless --only names them (then without their CPU samples)")
    ap.add_argument("--only", default="", help="comma list of extras to run: c1,c2,c3,c4,c4u,c5,route,trace")
    ap.add_argument("--route-trace", default="", help="replay every frame of this .rrtrace file (extras.route_trace)")
    ap.add_argument("--profile", default="", choices=["", "headline", "c4", "c3", "c5"],
                    help="profiler driver: a fixed number of launches of one case, no timing, "
                         "no JSON line (for rocprofv3 --pmc / --kernel-trace runs)")
    # shape-generic runner (reference benchmarks/benchmark_main.cpp:16-33)
    ap.add_argument("--suite", choices=SUITES, help="runner mode: time one chain entry at --param shapes")
    ap.add_argument("--operator", choices=OPERATORS, help="runner mode: time one operator at --param shapes")
    ap.add_argument("--param", action="extend", nargs="+", default=[], metavar="KEY=VALUE",
                    help="T, E, K, N, top_k, distribution, zipf_s, tie_fraction, seed "
                         "(one or more pairs per flag, the flag repeatable)")
    ap.add_argument("--variant", default="auto", choices=["auto", "naive", "optimized"])
    ap.add_argument("--cache-mode", default="warm", choices=["warm", "cold_scrub"])
    ap.add_argument("--cache-scrub-bytes", type=int, default=512 << 20,
                    help="runner mode, cold_scrub: bytes written before every warmup call and sample")
    ap.add_argument("--samples", type=int, default=10, help="runner mode: timed samples")
    ap.add_argument("--kernel-repeats", type=int, default=1,
                    help="runner mode: calls per sample (the sample is their span divided by the count)")
    ap.add_argument("--profile-once", action="store_true",
                    help="runner mode: warm up, then enqueue one call without timing and print nothing")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="phase times of the headline chain's expert launch, read from the instrumentation "
                         "build (RR_LIBRARY=raggedroute_amd/libraggedroute_amd_stamps.so)")
    ap.add_argument("--phase-stamps-out", default="",
                    help="--phase-stamps: also save the launch's raw stamps (workgroups x 8 waves x slots, "
                         "int64 .npy) to this file")
    return ap.parse_args(argv)


# ------------------------------------------------------------------ work model

def work_model(t, e, k, n, active=None, sorted_route=False):
    """Algorithmic bytes / flops per stage (FP32 = 4 bytes, R = 2T)."""
    r = 2 * t
    active = e if active is None else active
    return {
        "dense_gemm": (4 * (t * k + k * e + t * e), 2.0 * t * k * e),
        "topk_gate": (4 * t * e + 8 * r, 0.0),
        "histogram": (4 * r + 4 * e, 0.0),
        "exclusive_scan": (4 * e + 4 * (e + 1), 0.0),
        "histogram_scan": (4 * r + 4 * e + 4 * (e + 1), 0.0),
        "token_permute": (4 * t * k + 4 * r * k + 4 * r + 4 * (e + 1) + 4 * r + (4 * r if sorted_route else 0), 0.0),
        "grouped_gemm": (4 * (r * k + active * k * n + r * n) + 4 * (e + 1), 2.0 * r * k * n),
        "unpermute": (4 * r * n + 4 * t * n + 8 * r, 3.0 * t * n),
    }


def fused_work_model(t, e, k, n, active=None):
    """Algorithmic bytes / flops of the fused chain's launches (unique HBM
    traffic: every input read once, every output written once)."""
    r = 2 * t
    active = e if active is None else active
    gate = (4 * (t * k + k * e + t * e) + 16 * t + 4 * t * n, 2.0 * t * k * e)
    prep = (4 * r + 4 * e + 4 * (e + 1) + 4 * e + 8 * r, 0.0)
    gemm = (4 * (t * k + active * k * n + r * k + r * n + t * n) + 8 * r + 4 * (e + 1),
            2.0 * r * k * n + 2.0 * r * n)
    return {
        # x, router weights in; logits, ids, weights out; y zeroed
        "router_gate": gate,
        "gate": (gate[0] - 4 * (t * k + k * e) + 0, 0.0),
        # ids in; counts, offsets, cursors, route_pos, sorted_route out
        "route_prep": prep,
        # x, active expert weights, sorted_route, route weights, offsets in;
        # x_permuted, y_permuted, y out (y += w * y_permuted)
        "expert_gemm": gemm,
        # both in one launch: ids in instead of sorted_route
        "route_prep_expert_gemm": (prep[0] + gemm[0] - 8 * r, gemm[1]),
    }


def roofline(name, nbytes, flops, seconds):
    ai = flops / nbytes if nbytes else 0.0
    if flops and ai > RIDGE:
        achieved = flops / seconds / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 3), "peak": FP32_MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4)}
    achieved = nbytes / seconds / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4)}


# ------------------------------------------------------------------- harness

class Chain:
    """Device buffers + per-stage argument structs of one chain workload."""

    def __init__(self, cfg, inputs, device, with_inverse=False):
        import torch
        import raggedroute_amd as rr
        self.rr, self.torch, self.cfg = rr, torch, cfg
        t, e, k, n = cfg.tokens, cfg.experts, cfg.hidden, cfg.output
        i32 = dict(dtype=torch.int32, device=device)
        self.x, self.we = inputs["x"], inputs["expert_weights"]
        self.wr = inputs.get("router_weights")
        self.logits = inputs["logits"] if "logits" in inputs else torch.empty(t, e, device=device)
        self.ids = torch.empty(t, 2, **i32)
        self.w = torch.empty(t, 2, device=device)
        self.counts = torch.empty(e, **i32)
        self.offsets = torch.empty(e + 1, **i32)
        self.xp = torch.empty(2 * t, k, device=device)
        self.pos = torch.empty(2 * t, **i32)
        self.inv = torch.empty(2 * t, **i32) if with_inverse else None
        self.yp = torch.empty(2 * t, n, device=device)
        self.y = torch.empty(t, n, device=device)
        ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
        self.stream = torch.cuda.current_stream(device).cuda_stream
        # chain workspace: E cursor words (also the token_permute workspace)
        # followed by the fused path's sorted_route scratch
        ws_words = rr.get_chain_workspace_size(rr.ChainArgs(tokens=t, experts=e)) // 4
        self.workspace = torch.empty(ws_words, **i32)
        self.cursors = self.workspace[:e]
        self.ctx = rr.RuntimeContext(stream=self.stream, workspace=self.workspace.data_ptr(),
                                     workspace_bytes=ws_words * 4,
                                     architecture=int(rr.DeviceArchitecture.kGfx950))
        self.chain_args = rr.ChainArgs(
            x=ptr(self.x), router_weights=ptr(self.wr), logits=ptr(self.logits), expert_ids=ptr(self.ids),
            route_weights=ptr(self.w), counts=ptr(self.counts), offsets=ptr(self.offsets),
            x_permuted=ptr(self.xp), route_pos=ptr(self.pos), sorted_route=ptr(self.inv),
            expert_weights=ptr(self.we), y_permuted=ptr(self.yp), y=ptr(self.y),
            tokens=t, experts=e, hidden=k, output=n)
        cv, mv = rr.cview, rr.mview
        self.stage_args = {
            "dense_gemm": (rr.dense_gemm, rr.DenseGemmArgs(a=cv(ptr(self.x)), b=cv(ptr(self.wr)),
                                                           c=mv(ptr(self.logits)), m=t, n=e, k=k)),
            "topk_gate": (rr.topk_gate, rr.TopKGateArgs(logits=cv(ptr(self.logits)), expert_ids=ptr(self.ids),
                                                        weights=mv(ptr(self.w)), tokens=t, experts=e)),
            "histogram": (rr.histogram, rr.HistogramArgs(
                expert_ids=ptr(self.ids), counts=ptr(self.counts), route_pairs=2 * t, experts=e)),
            "exclusive_scan": (rr.exclusive_scan, rr.ExclusiveScanArgs(
                counts=ptr(self.counts), offsets=ptr(self.offsets), experts=e)),
            "histogram_scan": (rr.histogram_exclusive_scan, rr.HistogramExclusiveScanArgs(
                expert_ids=ptr(self.ids), counts=ptr(self.counts), offsets=ptr(self.offsets),
                route_pairs=2 * t, experts=e)),
            "token_permute": (rr.token_permute, rr.TokenPermuteArgs(
                x=cv(ptr(self.x)), expert_ids=ptr(self.ids), offsets=ptr(self.offsets), x_permuted=mv(ptr(self.xp)),
                route_pos=ptr(self.pos), sorted_route=ptr(self.inv), tokens=t, experts=e, top_k=2, hidden=k)),
            "grouped_gemm": (rr.grouped_gemm, rr.GroupedGemmArgs(
                x_permuted=cv(ptr(self.xp)), expert_weights=cv(ptr(self.we)), offsets=ptr(self.offsets),
                y_permuted=mv(ptr(self.yp)), experts=e, hidden=k, output=n, max_expert_tokens=2 * t)),
            "unpermute": (rr.unpermute, rr.UnpermuteArgs(
                y_permuted=cv(ptr(self.yp)), route_pos=ptr(self.pos), route_weights=cv(ptr(self.w)),
                y=mv(ptr(self.y)), tokens=t, top_k=2, output=n)),
        }
        if not cfg.from_tokens:
            del self.stage_args["dense_gemm"]

    def ctx_on(self, stream):
        """The chain's context on another HIP stream (handle)."""
        return self.rr.RuntimeContext(stream=stream, workspace=self.ctx.workspace,
                                      workspace_bytes=self.ctx.workspace_bytes,
                                      architecture=self.ctx.architecture)

    def chain(self, stream=None):
        fn = self.rr.chain_from_tokens if self.cfg.from_tokens else self.rr.chain_from_logits
        status = fn(self.chain_args, self.ctx if stream is None else self.ctx_on(stream))
        if not status.ok():
            raise RuntimeError(status.message)

    def fused_launch(self, index, stream=None):
        ctx = self.ctx if stream is None else self.ctx_on(stream)
        status = self.rr.chain_fused_launch(self.chain_args, ctx, self.cfg.from_tokens, index)
        if not status.ok():
            raise RuntimeError(f"fused launch {index}: {status.message}")

    def stage(self, name, stream=None):
        fn, args = self.stage_args[name]
        status = fn(args, self.ctx if stream is None else self.ctx_on(stream))
        if not status.ok():
            raise RuntimeError(f"{name}: {status.message}")


def settle(torch, fn, busy_s=0.03, probe=10):
    """Untimed back-to-back calls of `fn` until the GPU has run them for about
    `busy_s` (the per-call time from `probe` calls): launches reach their
    steady-state rate only after about 20 ms of continuous load (see
    SETTLE_CHAINS)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(probe):
        fn()
    torch.cuda.synchronize()
    per = max((time.perf_counter() - t0) / probe, 1e-6)
    for _ in range(int(busy_s / per)):
        fn()
    torch.cuda.synchronize()


def time_loop(torch, fn, reps, warmup=3):
    """Average seconds per call of `fn` over `reps` back-to-back launches,
    bracketed by HIP events on the current stream (host-submitted: use for
    calls long enough that the GPU never waits for the host)."""
    for _ in range(warmup):
        fn()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3 / reps


def graph_time(torch, device, call, n=50, replays=4):
    """Average seconds per call: `n` calls recorded back to back into one HIP
    graph (torch.cuda.CUDAGraph) and the graph replayed `replays` times between
    HIP events. No host submission sits between the calls, so short kernels
    are timed at the GPU's rate. `call(stream)` enqueues one call on the HIP
    stream handle it is given (kernels only: no memset or allocation)."""
    stream = torch.cuda.Stream(device)
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(n):
            call(stream.cuda_stream)
    graph.replay()  # (first replay uploads)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    stop.record()
    stop.synchronize()
    del graph
    return start.elapsed_time(stop) / 1e3 / (replays * n)


def percentile(values, q):
    """Linear interpolation between closest ranks (reference runner.cpp:42-50)."""
    v = sorted(values)
    if len(v) == 1:
        return v[0]
    pos = q * (len(v) - 1)
    lo = int(pos)
    hi = min(lo + 1, len(v) - 1)
    return v[lo] + (v[hi] - v[lo]) * (pos - lo)


def sample_stats(seconds):
    mean = statistics.fmean(seconds)
    cv = statistics.pstdev(seconds) / mean if mean > 0 else 0.0
    return {"samples": len(seconds), "p50_us": round(percentile(seconds, 0.5) * 1e6, 2),
            "p95_us": round(percentile(seconds, 0.95) * 1e6, 2), "cv": round(cv, 4)}


MIN_BATCH = 10      # chains per timed sample (the reference runner's kernel_repeats role)
# Untimed back-to-back chains before the first timed sample, counting
# --warmup, and again before the per-launch and per-stage timings. The chain
# reaches its steady state only after about 20 ms of continuous load (measured
# on MI355X, p50 of 20 batches of 10 after N chains: N = 50 20.2-20.4 us, 200
# 20.0, 500 19.6, 1000 19.3, 2000-8000 19.3; after 0.5 s idle, 50 chains give
# 20.4 us again).
SETTLE_CHAINS = 1500


def batch_sizes(steps, samples=20, min_batch=MIN_BATCH):
    """`steps` calls split into at most `samples` batches of at least
    `min_batch` calls each (one batch when steps < min_batch), sizes differing
    by at most one and summing to exactly `steps`. Each batch carries one
    timing event, so its cost per call does not grow as --steps shrinks
    (the reference runner's fixed kernel_repeats per sample,
    benchmarks/core/runner.cpp:350-370)."""
    n = max(1, min(samples, steps // min_batch))
    return [steps // n + (1 if i < steps % n else 0) for i in range(n)]


class Marks:
    """Timing-only HIP events, created through the HIP runtime the process has
    already loaded, with hipEventDisableSystemFence: recording one then skips
    the system-scope cache writeback and invalidate of a default event, which
    costs about 1.6 us of GPU time per event on MI355X (measured between
    back-to-back headline chains: 26.8 us per chain with default events,
    25.0 us with these, 23.9 us with no event in between)."""

    DISABLE_SYSTEM_FENCE = 0x20000000
    _hip = None

    def __init__(self, count):
        if Marks._hip is None:
            path = next(line.split()[-1] for line in Path("/proc/self/maps").read_text().splitlines()
                        if "libamdhip64" in line)
            Marks._hip = ctypes.CDLL(path)
        self.events = []
        for _ in range(count):
            ev = ctypes.c_void_p()
            rc = Marks._hip.hipEventCreateWithFlags(ctypes.byref(ev), ctypes.c_uint(self.DISABLE_SYSTEM_FENCE))
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            self.events.append(ev)

    def record(self, i, stream):
        if Marks._hip.hipEventRecord(self.events[i], ctypes.c_void_p(stream)) != 0:
            raise RuntimeError("hipEventRecord failed")

    def synchronize(self, i):
        if Marks._hip.hipEventSynchronize(self.events[i]) != 0:
            raise RuntimeError("hipEventSynchronize failed")

    def seconds(self, i, j):
        ms = ctypes.c_float()
        if Marks._hip.hipEventElapsedTime(ctypes.byref(ms), self.events[i], self.events[j]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value / 1e3

    def __del__(self):
        for ev in self.events:
            Marks._hip.hipEventDestroy(ev)


def batch_means(torch, fn, samples=20, repeats=10, sizes=None, stream=None):
    """Reference runner semantics (runner.cpp:218-236, 283-411): each sample is
    the event span of a batch of back-to-back calls divided by the batch size.
    The batches run back to back too, separated only by timing-only events
    (Marks), with one host synchronisation at the end; a short device spin
    first lets the host queue the work ahead of the first event."""
    sizes = sizes or [repeats] * samples
    stream = torch.cuda.current_stream().cuda_stream if stream is None else stream
    marks = Marks(len(sizes) + 1)
    torch.cuda.synchronize()
    torch.cuda._sleep(200_000)  # ~0.1 ms of GPU time, before the first event
    marks.record(0, stream)
    for i, reps in enumerate(sizes):
        for _ in range(reps):
            fn()
        marks.record(i + 1, stream)
    marks.synchronize(len(sizes))
    return [marks.seconds(i, i + 1) / reps for i, reps in enumerate(sizes)]


def cold_spans(torch, ch, device, samples, scrub_mib=512, call=None):
    """Single calls (a chain by default), each after a scrub of scrub_mib MiB
    written through the caches (rr_launch_cache_scrub): the chain's working set
    (~60 MB) and C4's x (134 MB) otherwise stay in the 256 MB Infinity Cache
    between calls. The scrub also keeps the GPU busy while the host queues the
    timed call."""
    call = call or ch.chain
    scrub = torch.empty(scrub_mib << 18, dtype=torch.int32, device=device)
    out = []
    for _ in range(samples):
        assert ch.rr.ops.launch_cache_scrub(scrub.data_ptr(), scrub.numel(), ch.stream) == 0
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(); call(); b.record()
        b.synchronize()
        out.append(a.elapsed_time(b) / 1e3)
    del scrub
    return out


def graph_report(torch, device, ch, reps=200):
    """The chain replayed from captured graphs (rr_chain_graph_*) against
    direct calls: GPU time per chain (events over back-to-back launches on one
    stream) and host time to submit one chain (no synchronisation inside the
    loop), for graphs of 1, 10 and 50 chains (a sequence graph: one
    hipGraphLaunch replays them all). Each form is first settled (settle) so
    that all of them are timed at the steady-state clock."""
    rr = ch.rr
    stream = torch.cuda.Stream(device)
    ctx = ch.ctx_on(stream.cuda_stream)
    entry = rr.CHAIN_FROM_TOKENS if ch.cfg.from_tokens else rr.CHAIN_FROM_LOGITS
    fn = rr.chain_from_tokens if ch.cfg.from_tokens else rr.chain_from_logits

    def direct():
        status = fn(ch.chain_args, ctx)
        assert status.ok(), status.message

    def submit_us(call, per_call, n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            call()
        elapsed = time.perf_counter() - t0
        torch.cuda.synchronize()
        return round(elapsed / (n * per_call) * 1e6, 2)

    out = {}
    with torch.cuda.stream(stream):
        settle(torch, direct)
        out["direct_us"] = round(time_loop(torch, direct, reps, warmup=10) * 1e6, 2)
        out["direct_submit_us"] = submit_us(direct, 1, reps)
        for chains in (1, 10, 50):
            with rr.ChainGraph(entry, [ch.chain_args] * chains if chains > 1 else ch.chain_args, ctx) as graph:
                def replay():
                    status = graph.launch(stream.cuda_stream)
                    assert status.ok(), status.message
                n = max(4, reps // chains)
                key = f"graph{chains}"
                settle(torch, replay, probe=3)
                out[f"{key}_kernel_nodes"] = graph.kernel_nodes
                out[f"{key}_us"] = round(time_loop(torch, replay, n, warmup=3) * 1e6 / chains, 2)
                out[f"{key}_submit_us"] = submit_us(replay, chains, n)
    return out


def stage_report(torch, device, ch, model, n=50):
    """Each stage operator alone, `n` calls per graph (graph_time)."""
    out = {}
    for name in ch.stage_args:
        sec = graph_time(torch, device, lambda s: ch.stage(name, s), n=n)
        nbytes, flops = model[name]
        out[name] = {"us": round(sec * 1e6, 2), "bytes": int(nbytes), "flops": flops,
                     "roofline": roofline(name, nbytes, flops, sec)}
    return out


def launch_report(torch, device, ch, model, n=50):
    """Each launch of the fused chain alone (what chain_from_* runs), `n`
    launches per graph (graph_time)."""
    out = {}
    for index, name in enumerate(ch.rr.chain_fused_launch_names(ch.chain_args, ch.cfg.from_tokens)):
        sec = graph_time(torch, device, lambda s: ch.fused_launch(index, s), n=n)
        nbytes, flops = model[name]
        out[name] = {"us": round(sec * 1e6, 2), "bytes": int(nbytes), "flops": flops,
                     "roofline": roofline(name, nbytes, flops, sec)}
    return out


# ------------------------------------------------------------------ workloads

def headline(torch, device, args):
    """The headline chain: `--warmup` untimed chains (then more untimed chains
    up to SETTLE_CHAINS in all: the chain reaches its steady state after about
    20 ms of back-to-back chains), then exactly `--steps` chains in batches of at least
    MIN_BATCH (reference runner: each sample is the event span of a batch
    divided by its size); value = T / p50 of the batch means. The outputs of
    the last timed chain are copied to the host for validation. Then the cold
    chain, the graph report and the per-launch / per-stage breakdown
    (graph_time)."""
    from raggedroute_amd import workloads
    cfg = workloads.HEADLINE
    inputs = workloads.chain_inputs_device(cfg, 0, device)
    ch = Chain(cfg, inputs, device)
    settle = max(0, SETTLE_CHAINS - args.warmup)
    for _ in range(args.warmup + settle):
        ch.chain()
    torch.cuda.synchronize()
    sizes = batch_sizes(args.steps)
    t0 = time.perf_counter()
    means = batch_means(torch, ch.chain, sizes=sizes)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    timed_outputs = {name: getattr(ch, attr).cpu().numpy() for name, attr in (
        ("logits", "logits"), ("ids", "ids"), ("weights", "w"), ("counts", "counts"), ("offsets", "offsets"),
        ("route_pos", "pos"), ("x_permuted", "xp"), ("y", "y"))}
    warm = sample_stats(means)
    warm["batch_sizes"] = sorted(set(sizes))
    warm["clock_settle_chains"] = settle
    mean_s = sum(m * n for m, n in zip(means, sizes)) / args.steps
    cold = sample_stats(cold_spans(torch, ch, device, samples=20))
    active = int((ch.counts.cpu().numpy() > 0).sum())
    for _ in range(SETTLE_CHAINS):  # (the cold samples let the clock drop)
        ch.chain()
    torch.cuda.synchronize()
    launches = launch_report(torch, device, ch,
                             fused_work_model(cfg.tokens, cfg.experts, cfg.hidden, cfg.output, active))
    ch.chain()  # restore y (timing the last launch alone keeps adding into it)
    graph = graph_report(torch, device, ch)
    model = work_model(cfg.tokens, cfg.experts, cfg.hidden, cfg.output, active)
    stages = stage_report(torch, device, ch, model)
    return cfg, ch, inputs, {"p50_s": percentile(means, 0.5), "mean_s": mean_s, "wall_s": wall,
                             "warm": warm, "cold": cold, "graph": graph, "samples": len(sizes),
                             "launches": launches, "stages": stages, "active_experts": active,
                             "timed_outputs": timed_outputs}


def c4(torch, device, hidden=4096, output=14336, reps=5, samples=10, cpu_sample=False):
    """Mixtral-shaped ragged grouped GEMM + permute + unpermute: T=8192, R=16384,
    E=8 with 7 active (Zipf 1.2), expert 7 empty. Permute and unpermute are
    timed warm (back-to-back calls: x, 134 MB, stays in the 256 MB Infinity
    Cache) and cold (each call after a 512 MiB scrub); their roofline is the
    cold one. The grouped GEMM (1.9 TFLOP, 1.9 GB of weights) is timed warm."""
    import raggedroute_amd as rr
    from raggedroute_amd import workloads
    t, e = 8192, 8
    ids_h, w_h = workloads.c4_routing(t, e, 7, 1.2, seed=0)
    stream = torch.cuda.current_stream(device).cuda_stream
    x = torch.empty(t, hidden, device=device)
    we = torch.empty(e, hidden, output, device=device)
    assert rr.fill_normal(x.data_ptr(), x.numel(), 0, workloads.S_X, 0.0, 1.0, stream) == 0
    sd = float(np.float32(1.0 / np.sqrt(hidden)))
    assert rr.fill_normal(we.data_ptr(), we.numel(), 0, workloads.S_EXPERTS, 0.0, sd, stream) == 0
    cfg = workloads.ChainConfig("C4", t, e, hidden, output, from_tokens=False)
    ch = Chain(cfg, {"x": x, "expert_weights": we, "logits": torch.empty(t, e, device=device)}, device)
    ch.ids.copy_(torch.from_numpy(ids_h))
    ch.w.copy_(torch.from_numpy(w_h))
    for name in ("histogram_scan", "token_permute", "grouped_gemm", "unpermute"):
        ch.stage(name)
    torch.cuda.synchronize()
    active = int((ch.counts.cpu().numpy() > 0).sum())
    model = work_model(t, e, hidden, output, active)
    out = {"T": t, "E": e, "K": hidden, "N": output, "active_experts": active}
    for name in ("token_permute", "grouped_gemm", "unpermute"):
        nbytes, flops = model[name]
        if name == "grouped_gemm":
            sec = time_loop(torch, lambda: ch.stage(name), reps, warmup=2)  # (two calls: ~30 ms of load)
            out[name] = {"us": round(sec * 1e6, 1), "roofline": roofline(name, nbytes, flops, sec)}
            continue
        warm = statistics.median(batch_means(torch, lambda: ch.stage(name), samples=samples, repeats=5))
        cold = sample_stats(cold_spans(torch, ch, device, samples, call=lambda: ch.stage(name)))
        cold_s = cold["p50_us"] * 1e-6
        out[name] = {"us": cold["p50_us"], "cold": cold, "warm_us": round(warm * 1e6, 1),
                     "warm_roofline": roofline(name, nbytes, flops, warm),
                     "roofline": roofline(name, nbytes, flops, cold_s)}
    out["permute_gbs_reference_model"] = round(2 * 4 * 2 * t * hidden / (out["token_permute"]["us"] * 1e-6) / 1e9, 1)
    if cpu_sample:
        out["cpu_sample"] = cpu_sample_c4(ch, we, 2 * t)
    del ch, x, we
    torch.cuda.empty_cache()
    return out


def c5(torch, device, steps=20, cpu_sample=False):
    from raggedroute_amd import workloads
    cfg = workloads.C5
    inputs = workloads.chain_inputs_device(cfg, 0, device)
    ch = Chain(cfg, inputs, device)
    settle(torch, ch.chain, probe=3)
    sec = time_loop(torch, ch.chain, steps, warmup=3)
    active = int((ch.counts.cpu().numpy() > 0).sum())
    launches = launch_report(torch, device, ch,
                             fused_work_model(cfg.tokens, cfg.experts, cfg.hidden, cfg.output, active), n=5)
    model = work_model(cfg.tokens, cfg.experts, cfg.hidden, cfg.output, active)
    stages = stage_report(torch, device, ch, model, n=5)
    out = {"tokens_per_s": round(cfg.tokens / sec, 1), "chain_us": round(sec * 1e6, 1),
           "launches": launches, "stages": stages}
    if cpu_sample:
        out["cpu_sample"] = cpu_sample_c5(inputs, cfg)
    del ch, inputs
    torch.cuda.empty_cache()
    return out


def cpu_sample_c4(ch, expert_weights, routes, rows=41):
    """C4 grouped GEMM on the oracle (single thread) over a seeded sample of
    `rows` rows of x_permuted (0.25 % of R: the measurement plan's 1 % would be
    about 50 s of CPU time here, the full 1.9 TFLOP is out of reach on one
    core), extrapolated linearly to all R rows."""
    import oracle
    offsets = ch.offsets.cpu().numpy().astype(np.int64)
    pick = np.sort(np.random.default_rng(0).choice(routes, size=rows, replace=False)).astype(np.int64)
    xs = ch.xp[torch_index(pick, ch.xp.device)].cpu().numpy()
    expert = np.searchsorted(offsets, pick, side="right") - 1
    offs = np.searchsorted(expert, np.arange(len(offsets)), side="left").astype(np.int32)
    w = expert_weights.cpu().numpy()
    t0 = time.perf_counter()
    oracle.grouped_gemm_f32_seq(xs, w, offs)
    sec = time.perf_counter() - t0
    flops = 2.0 * rows * w.shape[1] * w.shape[2]
    return {"kind": "port", "cores": 1,
            "sample": f"{rows} of {routes} x_permuted rows (seeded random sample, seed 0) through the oracle "
                      "grouped GEMM (single thread, -O2 -ffp-contract=off); full time extrapolated linearly",
            "sample_ms": round(sec * 1e3, 3), "gflops": round(flops / sec / 1e9, 3),
            "extrapolated_grouped_gemm_ms": round(sec * routes / rows * 1e3, 1)}


def cpu_sample_c5(inputs, cfg, frac=100):
    """C5 chain_from_tokens on the oracle (single thread) over a seeded 1 %
    sample of the tokens (the full chain is 112 GFLOP scalar), extrapolated
    linearly."""
    import oracle
    n = max(1, cfg.tokens // frac)
    pick = np.sort(np.random.default_rng(0).choice(cfg.tokens, size=n, replace=False))
    x = inputs["x"][torch_index(pick, inputs["x"].device)].cpu().numpy()
    rw = inputs["router_weights"].cpu().numpy()
    we = inputs["expert_weights"].cpu().numpy()
    t0 = time.perf_counter()
    oracle.chain(x, we, router_weights=rw)
    sec = time.perf_counter() - t0
    return {"kind": "port", "cores": 1,
            "sample": f"{n} of {cfg.tokens} tokens (seeded random sample, seed 0) through the oracle "
                      "chain_from_tokens (single thread, -O2 -ffp-contract=off); full time extrapolated linearly",
            "sample_ms": round(sec * 1e3, 3), "tokens_per_s": round(n / sec, 1),
            "extrapolated_chain_ms": round(sec * cfg.tokens / n * 1e3, 1)}


def torch_index(idx, device):
    import torch
    return torch.from_numpy(np.asarray(idx, np.int64)).to(device)


def small_chain(torch, device, cfg, reps=200):
    """C1 / C2 chain on the GPU (parity configs; timed for context)."""
    from raggedroute_amd import workloads
    inputs = workloads.chain_inputs(cfg, 0)
    dev_inputs = {k: torch.from_numpy(v).to(device) for k, v in inputs.items()}
    ch = Chain(cfg, dev_inputs, device)
    settle(torch, ch.chain)
    sec = time_loop(torch, ch.chain, reps, warmup=10)
    stats = sample_stats(batch_means(torch, ch.chain, samples=20, repeats=10))
    del ch, dev_inputs
    return {"T": cfg.tokens, "E": cfg.experts, "K": cfg.hidden, "N": cfg.output,
            "entry": "chain_from_tokens" if cfg.from_tokens else "chain_from_logits",
            "chain_us": round(sec * 1e6, 2), "tokens_per_s": round(cfg.tokens / sec, 1), "warm": stats}


def route_chain(torch, device, reps=200):
    """chain_from_route_ids at the reference's post-route release shapes
    (representative / large for top_k 2, 4, 8 and max_route_pairs), uniform ids."""
    import raggedroute_amd as rr
    from raggedroute_amd import workloads
    stream = torch.cuda.current_stream(device).cuda_stream
    out = {}
    for name, cfg in workloads.route_chain_configs().items():
        if name.startswith("small"):
            continue
        inp = workloads.route_chain_inputs(cfg, 0)
        t, e, k, n, top = cfg.tokens, cfg.experts, cfg.hidden, cfg.output, cfg.top_k
        r = t * top
        d = {key: torch.from_numpy(np.ascontiguousarray(v)).to(device) for key, v in inp.items()}
        i32 = dict(dtype=torch.int32, device=device)
        bufs = {"counts": torch.empty(e, **i32), "offsets": torch.empty(e + 1, **i32),
                "route_pos": torch.empty(r, **i32), "sorted_route": torch.empty(r, **i32),
                "y_permuted": torch.empty(r, n, device=device), "y": torch.empty(t, n, device=device)}
        args = rr.RouteChainArgs(
            x=d["x"].data_ptr(), expert_ids=d["ids"].data_ptr(), route_weights=d["weights"].data_ptr(),
            expert_weights=d["expert_weights"].data_ptr(), counts=bufs["counts"].data_ptr(),
            offsets=bufs["offsets"].data_ptr(), x_permuted=None, route_pos=bufs["route_pos"].data_ptr(),
            sorted_route=bufs["sorted_route"].data_ptr(), y_permuted=bufs["y_permuted"].data_ptr(),
            y=bufs["y"].data_ptr(), tokens=t, experts=e, top_k=top, hidden=k, output=n)
        ws = torch.empty(rr.get_route_chain_workspace_size(args) // 4, **i32)
        ctx = rr.RuntimeContext(stream=stream, workspace=ws.data_ptr(), workspace_bytes=ws.numel() * 4,
                                architecture=int(rr.DeviceArchitecture.kGfx950))

        def call():
            status = rr.chain_from_route_ids(args, ctx)
            assert status.ok(), status.message
        settle(torch, call)
        sec = time_loop(torch, call, reps, warmup=10)
        out[name] = {"T": t, "E": e, "K": k, "N": n, "top_k": top, "us": round(sec * 1e6, 2),
                     "tokens_per_s": round(t / sec, 1),
                     "warm": sample_stats(batch_means(torch, call, samples=20, repeats=10))}
        del d, bufs, ws
    return out


def trace_replay(torch, device, path=None, hidden=256, output=128, reps=100):
    """Route-trace replay: every frame of a `.rrtrace` file (read by the
    library's native reader) through chain_from_logits (top_k = 2: logits that
    select the frame's ids) and chain_from_route_ids. Without a path: a
    generated T4096 / E64 trace with uniform, Zipf(1.4), round-robin and
    single-hot frames (every token on experts 0 and 1)."""
    import tempfile
    import raggedroute_amd as rr
    from raggedroute_amd import route_trace, workloads
    tmp = None
    if path is None:
        tmp = tempfile.TemporaryDirectory()
        frames = {d.replace("zipf", "zipf1.4"): workloads.topk_route_ids(4096, 2, 64, d, seed=i)
                  for i, d in enumerate(("uniform", "zipf", "round_robin", "single_hot"))}
        path = Path(tmp.name) / "generated.rrtrace"
        route_trace.write(path, "generated_t4096_e64", "synthetic_fixture", 64, frames)
    out = {}
    stream = torch.cuda.current_stream(device).cuda_stream
    for tr in route_trace.read_all(path):
        t, e, top = tr.tokens, tr.experts, tr.top_k
        rec = {"T": t, "E": e, "top_k": top, "K": hidden, "N": output,
               "max_expert_routes": int(np.bincount(tr.ids.reshape(-1), minlength=e).max())}
        if top == 2:
            cfg = workloads.ChainConfig(tr.frame_id, t, e, hidden, output, from_tokens=False)
            host = workloads.chain_inputs(cfg, 0)
            host["logits"] = route_trace.logits_for_ids(tr.ids, e)
            ch = Chain(cfg, {k: torch.from_numpy(v).to(device) for k, v in host.items()}, device)
            sec = time_loop(torch, ch.chain, reps, warmup=10)
            rec["chain_from_logits_us"] = round(sec * 1e6, 2)
            del ch
        rcfg = workloads.RouteChainConfig(tr.frame_id, t, e, hidden, output, top)
        inp = workloads.route_chain_inputs(rcfg, 0)
        d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(device) for k, v in inp.items()}
        d["ids"] = torch.from_numpy(tr.ids).to(device)
        i32 = dict(dtype=torch.int32, device=device)
        r = t * top
        bufs = [torch.empty(e, **i32), torch.empty(e + 1, **i32), torch.empty(r, **i32),
                torch.empty(r, output, device=device), torch.empty(t, output, device=device)]
        args = rr.RouteChainArgs(x=d["x"].data_ptr(), expert_ids=d["ids"].data_ptr(),
                                 route_weights=d["weights"].data_ptr(),
                                 expert_weights=d["expert_weights"].data_ptr(), counts=bufs[0].data_ptr(),
                                 offsets=bufs[1].data_ptr(), route_pos=bufs[2].data_ptr(),
                                 y_permuted=bufs[3].data_ptr(), y=bufs[4].data_ptr(), tokens=t, experts=e,
                                 top_k=top, hidden=hidden, output=output)
        ws = torch.empty(rr.get_route_chain_workspace_size(args) // 4, **i32)
        ctx = rr.RuntimeContext(stream=stream, workspace=ws.data_ptr(), workspace_bytes=ws.numel() * 4,
                                architecture=int(rr.DeviceArchitecture.kGfx950))

        def call():
            status = rr.chain_from_route_ids(args, ctx)
            assert status.ok(), status.message
        rec["chain_from_route_ids_us"] = round(time_loop(torch, call, reps, warmup=10) * 1e6, 2)
        out[tr.frame_id] = rec
        del d, bufs, ws
    if tmp is not None:
        tmp.cleanup()
    return {"trace": str(path) if tmp is None else "generated", "frames": out}


def c3(torch, device):
    """Fused histogram + exclusive scan at R = 2^20 (graph_time, warm and
    cold), with its roofline, next to the launch floor: a trivial kernel
    (a 64-byte cache scrub) timed alone and as three dependent launches."""
    import raggedroute_amd as rr
    from raggedroute_amd import workloads
    routes = 1 << 20
    out = {}
    tiny = torch.empty(16, dtype=torch.int32, device=device)

    def trivial(stream, launches):
        for _ in range(launches):
            assert rr.ops.launch_cache_scrub(tiny.data_ptr(), 16, stream) == 0
    one = graph_time(torch, device, lambda s: trivial(s, 1), n=50)
    three = graph_time(torch, device, lambda s: trivial(s, 3), n=50)
    out["launch_floor"] = {"one_trivial_kernel_us": round(one * 1e6, 2),
                           "three_dependent_trivial_kernels_us": round(three * 1e6, 2)}
    scrub = torch.empty(512 << 18, dtype=torch.int32, device=device)
    for experts in (1, 33, 256):
        for dist in ("uniform", "hot50"):
            ids = torch.from_numpy(workloads.route_ids(routes, experts, dist, 0)).to(device)
            counts = torch.empty(experts, dtype=torch.int32, device=device)
            offsets = torch.empty(experts + 1, dtype=torch.int32, device=device)
            args = rr.HistogramExclusiveScanArgs(expert_ids=ids.data_ptr(), counts=counts.data_ptr(),
                                                 offsets=offsets.data_ptr(), route_pairs=routes, experts=experts)

            def call(stream):
                ctx = rr.RuntimeContext(stream=stream, architecture=int(rr.DeviceArchitecture.kGfx950))
                status = rr.histogram_exclusive_scan(args, ctx)
                assert status.ok(), status.message
            sec = graph_time(torch, device, call, n=50)
            cold = []
            cur = torch.cuda.current_stream(device).cuda_stream
            for _ in range(10):
                assert rr.ops.launch_cache_scrub(scrub.data_ptr(), scrub.numel(), cur) == 0
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(); call(cur); b.record()
                b.synchronize()
                cold.append(a.elapsed_time(b) / 1e3)
            nbytes = 4 * routes + 4 * experts + 4 * (experts + 1)
            cold_s = statistics.median(cold)
            out[f"E{experts}_{dist}"] = {"us": round(sec * 1e6, 2), "roofline": roofline("c3", nbytes, 0.0, sec),
                                        "cold_us": round(cold_s * 1e6, 2),
                                        "cold_roofline": roofline("c3", nbytes, 0.0, cold_s)}
    del scrub
    return out


def cpu_chain_seconds(inputs_host, from_tokens, runs=5, keep=None):
    """Reference CPU oracle chain (oracle/, single thread, -O2
    -ffp-contract=off), median of `runs` full runs. `keep` (a dict) receives
    the last run's outputs."""
    import oracle
    out = []
    for _ in range(runs):
        t0 = time.perf_counter()
        if from_tokens:
            res = oracle.chain(inputs_host["x"], inputs_host["expert_weights"],
                               router_weights=inputs_host["router_weights"])
        else:
            res = oracle.chain(inputs_host["x"], inputs_host["expert_weights"], logits=inputs_host["logits"])
        out.append(time.perf_counter() - t0)
    if keep is not None:
        keep.update(res)
    return statistics.median(out)


def validate_chain(cfg, host, dev, ref):
    """The outputs of the last timed chain_from_tokens against the oracle chain
    run on the same inputs (the reference runner validates after measuring,
    benchmarks/core/runner.cpp:372-381, with the chain checks of
    benchmarks/adapters/chain_adapter.cpp:469-495). ids are exact against the
    oracle top-2 of the device logits, the logits within the
    accumulation-aware GEMM bound of the exact product, and ids may differ from
    the CPU-logit oracle only on rows whose CPU rank-1/2 or rank-2/3 margin
    lies within that bound (counted); counts, offsets, the stable route map and
    the copied rows are exact; weights within 1e-6, y within atol 1e-4 +
    rtol 4e-5*K."""
    import oracle
    t, e, k = cfg.tokens, cfg.experts, cfg.hidden
    x, wr, we = host["x"], host["router_weights"], host["expert_weights"]
    x64, wr64 = x.astype(np.float64), wr.astype(np.float64)
    gamma = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    bound = 4 * gamma * (np.abs(x64) @ np.abs(wr64)) + 1e-7
    checks = {"logits_within_gemm_bound": bool((np.abs(dev["logits"] - x64 @ wr64) <= bound).all())}
    ids, w = oracle.top2_f32(dev["logits"])
    checks["ids_exact"] = bool(np.array_equal(dev["ids"], ids))
    checks["weights_within_1e-6"] = oracle.compare_floating(dev["weights"], w, 1e-6, 1e-6)[0] == 0
    counts = oracle.histogram(ids, e)
    offsets = oracle.exclusive_scan(counts)
    pos = oracle.stable_route_pos(ids, offsets)
    checks["counts_exact"] = bool(np.array_equal(dev["counts"], counts))
    checks["offsets_exact"] = bool(np.array_equal(dev["offsets"], offsets))
    checks["route_pos_exact"] = bool(np.array_equal(dev["route_pos"], pos))
    src = np.arange(2 * t) // 2
    checks["x_permuted_exact"] = bool(np.array_equal(dev["x_permuted"][pos].view(np.uint32),
                                                     x[src].view(np.uint32)))
    srt = np.sort(ref["logits"].astype(np.float64), axis=1)[:, ::-1]
    margin = np.minimum(srt[:, 0] - srt[:, 1], srt[:, 1] - srt[:, 2])
    near = margin <= 2 * bound.max(axis=1)
    differ = (ref["ids"] != dev["ids"]).any(axis=1)
    checks["ids_differ_from_cpu_logits_only_on_near_ties"] = bool(near[differ].all())
    y_fails, y_abs, y_rel = oracle.compare_floating(dev["y"], oracle.chain_output_f32(x, we, ids, w),
                                                    1e-4, 4e-5 * k)
    checks["y_within_chain_tolerance"] = y_fails == 0
    return {"ok": bool(all(checks.values())), "what": "outputs of the last timed chain", "checks": checks,
            "near_tie_rows": int(near.sum()), "id_rows_differing_from_cpu_logits": int(differ.sum()),
            "y_failures": y_fails, "y_max_abs": y_abs, "y_max_rel": y_rel,
            "reference": "benchmarks/core/runner.cpp:372-381; benchmarks/adapters/chain_adapter.cpp:469-495"}


def environment(torch, device):
    """Run environment (the reference record's environment / build fields,
    benchmarks/core/runner.cpp:413-543): device, runtimes, and the source
    revision the library was built from (written by the build)."""
    props = torch.cuda.get_device_properties(device)
    env = {"device": props.name, "arch": getattr(props, "gcnArchName", None),
           "compute_units": props.multi_processor_count, "hbm_gib": round(props.total_memory / 2 ** 30, 1),
           "torch": torch.__version__, "torch_hip": getattr(torch.version, "hip", None),
           "python": sys.version.split()[0], "host_cpu": cpu_model(), "host_cpus": os.cpu_count()}
    hip = Marks._hip
    if hip is not None:
        for name in ("hipRuntimeGetVersion", "hipDriverGetVersion"):
            v = ctypes.c_int()
            if getattr(hip, name)(ctypes.byref(v)) == 0:
                env[name[3:].replace("GetVersion", "_version").lower()] = v.value
    info = REPO / "raggedroute_amd" / "build_info.json"
    env["build"] = json.loads(info.read_text()) if info.exists() else None
    return env


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def profile(torch, device, case):
    """Fixed launch sequence for counter runs: first a plain 64 MiB copy (three
    launches, the calibration of FETCH_SIZE / WRITE_SIZE), then the case."""
    from raggedroute_amd import workloads
    src = torch.ones(16 << 20, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    print("profile: copy calibration done (3 x 64 MiB)", flush=True)
    if case == "headline":
        cfg = workloads.HEADLINE
        ch = Chain(cfg, workloads.chain_inputs_device(cfg, 0, device), device)
        # SETTLE_CHAINS untimed chains bring the chain to its steady state;
        # the 50 chains after them are the ones the summary reads
        for _ in range(SETTLE_CHAINS + 50):
            ch.chain()
        torch.cuda.synchronize()
        for index in range(len(ch.rr.chain_fused_launch_names(ch.chain_args, cfg.from_tokens))):
            for _ in range(20):
                ch.fused_launch(index)
        for name in ch.stage_args:
            for _ in range(20):
                ch.stage(name)
        torch.cuda.synchronize()
        print(f"profile: headline done ({SETTLE_CHAINS} + 50 chains, 20 x each fused launch, 20 x each stage)", flush=True)
    elif case == "c4":
        c4(torch, device, reps=2, samples=3)
        print("profile: c4 (K 4096, N 14336) done", flush=True)
        c4(torch, device, hidden=4095, output=14335, reps=2, samples=3)
        print("profile: c4 (K 4095, N 14335) done", flush=True)
    elif case == "c3":
        c3(torch, device)
        print("profile: c3 done", flush=True)
    elif case == "c5":
        cfg = workloads.C5
        ch = Chain(cfg, workloads.chain_inputs_device(cfg, 0, device), device)
        # Back to back with no host wait between calls: the expert GEMM needs
        # about 20 calls before its clock settles, so the last 10 of 30 are
        # the steady state of the timed bench loops.
        for _ in range(30):
            ch.chain()
        for _ in range(30):
            ch.stage("grouped_gemm")
        torch.cuda.synchronize()
        print("profile: c5 done (30 chains, 30 x grouped_gemm)", flush=True)


# ------------------------------------------------------------ phase stamps

STAMP_SLOTS = 48   # per wave, as g_phase_stamps in strip.hip
STAMP_BLOCKS = 1024
STAMP_PHASES = [   # (slot, phase ending at that stamp)
    (1, "route-id loads issued, LDS cleared"), (2, "barrier (ids arrive during it)"),
    (3, "histogram of the ids"), (4, "barrier"), (5, "per-expert sums and scans"),
    (6, "strip assignment"), (7, "strip table, first k chunks of B issued"),
    (8, "stable ranks of the range's routes"), (9, "barrier"),
    (10, "route map, rest of B issued")]


def phase_stamps(torch, device, chains=SETTLE_CHAINS, out=""):
    """Phase times of the headline chain's expert launch (the merged route
    preparation + expert GEMM + combine) from the instrumentation build, whose
    strip kernel writes the shader clock at each phase boundary of every wave
    (slots in raggedroute_amd/csrc/strip.hip). Runs `chains` chains and reads
    the stamps of the last launch; each wave's shader-clock rate comes from the
    100 MHz clock read at its start and end. Prints a markdown summary and one
    JSON line. The stamps and their stores perturb the launch: the chain time
    printed is the instrumented one."""
    import ctypes
    import raggedroute_amd as rr
    from raggedroute_amd import workloads
    try:
        read = rr.lib.rr_debug_phase_stamps
    except AttributeError:
        print("phase stamps: the loaded library has no stamps; run with "
              "RR_LIBRARY=raggedroute_amd/libraggedroute_amd_stamps.so", file=sys.stderr)
        return 2
    read.restype = ctypes.c_int
    read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    cfg = workloads.HEADLINE
    ch = Chain(cfg, workloads.chain_inputs_device(cfg, 0, device), device)
    for _ in range(chains):
        ch.chain()
    torch.cuda.synchronize()
    means = batch_means(torch, ch.chain, samples=10, repeats=10)
    torch.cuda.synchronize()
    buf = np.zeros(STAMP_BLOCKS * 8 * STAMP_SLOTS, np.uint64)
    assert read(buf.ctypes.data, buf.nbytes) == 0, "stamp copy failed"
    st = buf.reshape(STAMP_BLOCKS, 8, STAMP_SLOTS).astype(np.int64)
    st = st[st[:, 0, 39] > 0]  # the launch's workgroups (the array starts zeroed)
    grid = st.shape[0]
    if out:
        np.save(out, st)
    # each wave's shader-clock rate (cycles per us) from its 100 MHz clock reads
    rate = (st[:, :, 37] - st[:, :, 0]) / np.maximum(1, st[:, :, 39] - st[:, :, 38]) * 100.0
    us = (st - st[:, :, :1]) / rate[:, :, None]
    strips = st[:, 0, 40]
    halves = st[:, 0, 41]
    total = us[:, :, 37].max(axis=1)
    busy = total >= np.percentile(total, 90)
    rows = []
    prev = 0
    for slot, name in STAMP_PHASES:
        d = us[:, 0, slot] - us[:, 0, prev]
        rows.append({"phase": name, "wave0_median_us": round(float(np.median(d)), 3),
                     "wave0_busiest_median_us": round(float(np.median(d[busy])), 3)})
        prev = slot
    strip_rows = []
    for k in range(3):
        have = strips > k
        if not have.any():
            continue
        top, past, done = 11 + 4 * k, 13 + 4 * k, 14 + 4 * k
        for w in (0, 7):
            strip_rows.append({"strip": k, "wave": w,
                               "start_us": round(float(np.median(us[have, w, top])), 3),
                               "top_to_barrier_us": round(float(np.median(us[have, w, past] - us[have, w, top])), 3),
                               "mfma_us": round(float(np.median(us[have, w, done] - us[have, w, past])), 3)})
    tail = us[:, 0, 37] - us[:, 0, 36]
    rec = {"what": "phase stamps of the headline expert launch (instrumentation build)",
           "chain_us_instrumented": round(statistics.median(means) * 1e6, 2),
           "grid": grid, "strips_per_workgroup": np.bincount(strips).tolist(),
           "half_strips_per_workgroup": np.bincount(halves).tolist(),
           "shader_clock_ghz_median": round(float(np.median(rate)) / 1000.0, 3),
           "workgroup_span_us": {"median": round(float(np.median(total)), 2), "max": round(float(total.max()), 2)},
           "prologue": rows, "strips": strip_rows,
           "last_epilogue_to_memory_done_us": round(float(np.median(tail)), 3)}
    print("| phase (wave 0) | median us | busiest 10 % median us |")
    print("|---|---|---|")
    for r in rows:
        print(f"| {r['phase']} | {r['wave0_median_us']} | {r['wave0_busiest_median_us']} |")
    print(json.dumps(rec))
    return 0


# ------------------------------------------------------------ runner mode

RUNNER_DEFAULTS = {"T": 4096, "E": 64, "K": 256, "N": 128, "top_k": 2, "distribution": "uniform",
                   "zipf_s": None, "tie_fraction": 0.0, "seed": 0}


def runner_params(pairs):
    """--param key=value pairs over the defaults (the headline shape)."""
    out = dict(RUNNER_DEFAULTS)
    for pair in pairs:
        key, sep, value = pair.partition("=")
        if not sep or key not in out:
            raise SystemExit(f"--param {pair!r}: expected key=value with key in {', '.join(out)}")
        if key == "distribution":
            out[key] = value
        elif key in ("zipf_s", "tie_fraction"):
            out[key] = float(value)
        else:
            out[key] = int(value)
    return out


def run_runner(torch, device, args):
    """One chain entry or operator at any shape, timed like the reference
    runner (benchmarks/core/runner.cpp:336-370): `--warmup` iterations, then
    `--samples` samples; each iteration and sample is `--kernel-repeats`
    back-to-back calls, preceded in cold_scrub mode by a
    `--cache-scrub-bytes` scrub and a synchronisation, and a sample is the
    event span of its calls divided by the repeat count; the reported value
    uses the p50 sample. Defaults are the reference's (types.h:71-76: warmup
    5, samples 10, kernel_repeats 1) except the scrub size, which the
    reference requires on the command line and which defaults to 512 MiB
    here. Warm samples run back to back with timing-only events between them
    (batch_means) instead of a host synchronisation per sample. Prints one
    JSON record shaped like the headline line, with these settings under
    "runner". Outputs are not validated in this mode (the record says so):
    the GPU tests check every entry against the oracle, and the default
    headline run validates its timed chain."""
    import raggedroute_amd as rr
    from raggedroute_amd import workloads
    p = runner_params(args.param)
    t, e, k, n, top = p["T"], p["E"], p["K"], p["N"], p["top_k"]
    family = {"auto": rr.KernelFamily.kAuto, "naive": rr.KernelFamily.kNaive,
              "optimized": rr.KernelFamily.kOptimized}[args.variant]
    kernel = rr.kernel(family, rr.GFX950_NATIVE if family == rr.KernelFamily.kOptimized else 0)
    target = args.suite or args.operator
    if target is None:
        raise SystemExit("runner mode needs --suite or --operator")
    stream = torch.cuda.current_stream(device).cuda_stream
    keep = []  # device buffers the timed call reads or writes

    if args.suite == "chain_from_route_ids":
        cfg = workloads.RouteChainConfig("runner", t, e, k, n, top, p["distribution"],
                                         p["zipf_s"] if p["zipf_s"] is not None else 1.4)
        inp = workloads.route_chain_inputs(cfg, p["seed"])
        d = {key: torch.from_numpy(np.ascontiguousarray(v)).to(device) for key, v in inp.items()}
        r = t * top
        i32 = dict(dtype=torch.int32, device=device)
        bufs = {"counts": torch.empty(e, **i32), "offsets": torch.empty(e + 1, **i32),
                "x_permuted": torch.empty(r, k, device=device), "route_pos": torch.empty(r, **i32),
                "sorted_route": torch.empty(r, **i32), "y_permuted": torch.empty(r, n, device=device),
                "y": torch.empty(t, n, device=device)}
        rargs = rr.RouteChainArgs(
            x=d["x"].data_ptr(), expert_ids=d["ids"].data_ptr(), route_weights=d["weights"].data_ptr(),
            expert_weights=d["expert_weights"].data_ptr(), counts=bufs["counts"].data_ptr(),
            offsets=bufs["offsets"].data_ptr(), x_permuted=bufs["x_permuted"].data_ptr(),
            route_pos=bufs["route_pos"].data_ptr(), sorted_route=bufs["sorted_route"].data_ptr(),
            y_permuted=bufs["y_permuted"].data_ptr(), y=bufs["y"].data_ptr(), tokens=t, experts=e,
            top_k=top, hidden=k, output=n, kernel=kernel)
        ws = torch.empty(max(1, rr.get_route_chain_workspace_size(rargs) // 4), **i32)
        ctx = rr.RuntimeContext(stream=stream, workspace=ws.data_ptr(), workspace_bytes=ws.numel() * 4,
                                architecture=int(rr.DeviceArchitecture.kGfx950))
        keep += [d, bufs, ws]

        def call():
            status = rr.chain_from_route_ids(rargs, ctx)
            if not status.ok():
                raise RuntimeError(status.message)
        unit_count, unit = t, "tokens/s"
        nbytes = flops = None
    else:
        if top != 2:
            raise SystemExit("chain_from_tokens / chain_from_logits and the operators run top_k = 2")
        from_tokens = args.suite != "chain_from_logits" and args.operator != "topk_gate"
        cfg = workloads.ChainConfig("runner", t, e, k, n, from_tokens=from_tokens,
                                    logit_bias_s=p["zipf_s"], tie_fraction=p["tie_fraction"])
        if from_tokens:
            inputs = workloads.chain_inputs_device(cfg, p["seed"], device)
        else:
            inputs = {key: torch.from_numpy(v).to(device)
                      for key, v in workloads.chain_inputs(cfg, p["seed"]).items() if key != "tie_rows"}
        ch = Chain(cfg, inputs, device)
        ch.chain_args.kernel = kernel
        for _, op_args in ch.stage_args.values():
            op_args.kernel = kernel
        keep += [ch, inputs]
        ch.chain()  # every intermediate an operator reads
        if p["distribution"] != "uniform" and args.operator is not None:
            ids = workloads.topk_route_ids(t, 2, e, p["distribution"], p["seed"],
                                           p["zipf_s"] if p["zipf_s"] is not None else 1.4)
            ch.ids.copy_(torch.from_numpy(ids.astype(np.int32)))
            for name in ("histogram_scan", "token_permute", "grouped_gemm", "unpermute"):
                ch.stage(name)
        torch.cuda.synchronize()
        active = int((ch.counts.cpu().numpy() > 0).sum())
        if args.suite is not None:
            call, unit_count, unit = ch.chain, t, "tokens/s"
            nbytes = flops = None
        else:
            stage = {"histogram_exclusive_scan": "histogram_scan"}.get(args.operator, args.operator)
            nbytes, flops = work_model(t, e, k, n, active)[stage]
            call, unit_count, unit = (lambda: ch.stage(stage)), None, None

    repeats = args.kernel_repeats
    if repeats < 1 or args.samples < 1 or args.warmup < 0:
        raise SystemExit("--kernel-repeats and --samples must be >= 1, --warmup >= 0")
    scrub = None
    if args.cache_mode == "cold_scrub":
        if args.cache_scrub_bytes < 4:
            raise SystemExit("cold_scrub needs --cache-scrub-bytes >= 4")
        scrub = torch.empty(args.cache_scrub_bytes // 4, dtype=torch.int32, device=device)

    def scrub_cache():
        if scrub is not None:
            assert rr.ops.launch_cache_scrub(scrub.data_ptr(), scrub.numel(), stream) == 0
            torch.cuda.synchronize()

    # reference benchmarks/core/runner.cpp:336-370: every warmup iteration and
    # every sample is a scrub (cold_scrub) followed by kernel_repeats calls
    for _ in range(args.warmup):
        scrub_cache()
        for _ in range(repeats):
            call()
    torch.cuda.synchronize()
    if args.profile_once:
        call()
        torch.cuda.synchronize()
        return None
    if scrub is None:
        samples = batch_means(torch, call, samples=args.samples, repeats=repeats)
    else:
        samples = []
        for _ in range(args.samples):
            scrub_cache()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(repeats):
                call()
            b.record()
            b.synchronize()
            samples.append(a.elapsed_time(b) / 1e3 / repeats)
        del scrub
    p50 = percentile(samples, 0.5)
    line = {"metric": f"{target} {'tokens/s' if unit else 'roofline rate'} @T{t}/E{e}/K{k}/N{n} FP32",
            "n_gpus": 1, "steps": args.samples * repeats, "warmup": args.warmup,
            "ms_per_step": round(p50 * 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp32", "data": f"synthetic (SplitMix64, seed {p['seed']})",
            "config": {"workload": target, "T": t, "E": e, "K": k, "N": n, "top_k": top,
                       "distribution": p["distribution"], "zipf_s": p["zipf_s"],
                       "tie_fraction": p["tie_fraction"], "variant": args.variant,
                       "cache_mode": args.cache_mode},
            "runner": {"warmup": args.warmup, "samples": args.samples, "kernel_repeats": repeats,
                       "cache_scrub_bytes": args.cache_scrub_bytes if args.cache_mode == "cold_scrub" else 0,
                       "validated": False},
            "samples": sample_stats(samples)}
    if unit is not None:
        line.update(value=round(unit_count / p50, 1), unit=unit)
    else:
        roof = roofline(target, nbytes, flops, p50)
        line.update(value=roof["achieved"], unit=roof["unit"], roofline=roof,
                    bytes=int(nbytes), flops=flops)
    del keep
    return line


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this build measures one MI355X; "
                                   "multi-GPU runs are not part of it (each GPU would run the same "
                                   "chain on its own token shard)"}))
        return 2
    import torch
    import raggedroute_amd  # noqa: F401  (loads the HIP library or fails)

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.suite or args.operator:
        args.warmup = 5 if args.warmup is None else args.warmup
        line = run_runner(torch, device, args)
        if line is not None:
            print(json.dumps(line))
        return 0
    if args.profile:
        profile(torch, device, args.profile)
        return 0
    if args.phase_stamps:
        return phase_stamps(torch, device, out=args.phase_stamps_out)
    args.warmup = 20 if args.warmup is None else args.warmup
    cfg, ch, inputs, head = headline(torch, device, args)
    tokens_per_s = cfg.tokens / head["p50_s"]
    launches = head["launches"]
    dominant = max(launches, key=lambda s: launches[s]["us"])
    roof = dict(launches[dominant]["roofline"])
    roof["kernel"] = dominant
    roof["traffic"] = None
    traffic_file = REPO / "profiles" / f"{dominant}_headline_traffic.json"
    if traffic_file.exists():
        roof["traffic"] = json.loads(traffic_file.read_text()).get("hbm_bytes_per_launch")

    extras = {}
    if not args.quick or args.only:
        only = set(filter(None, args.only.split(","))) or {"c1", "c2", "c3", "c4", "c4u", "c5", "route", "trace"}
        from raggedroute_amd import workloads
        if "c1" in only:
            extras["C1"] = small_chain(torch, device, workloads.C1)
        if "c2" in only:
            extras["C2"] = small_chain(torch, device, workloads.C2)
        if "c1" in only:
            # the only shape with a published reference chain time (not a
            # BASELINE config; other hardware): context, not vs_baseline
            ref = small_chain(torch, device, workloads.ChainConfig("reference_l3", 512, 64, 128, 128))
            ref["reference_published"] = {
                "p50_us": 69.734, "hardware": "RTX 3080 (SM86)",
                "source": "reference docs/reports/l3_three_way_20260805/RaggedRoute_L3_3way_comparison.md:7,51"}
            extras["reference_l3_shape"] = ref
        if "c4" in only:
            extras["C4"] = c4(torch, device, cpu_sample=not args.quick)
        if "c4u" in only:
            extras["C4_nonaligned"] = c4(torch, device, 4095, 14335, reps=3)
        if "c5" in only:
            extras["C5"] = c5(torch, device, cpu_sample=not args.quick)
        if "c3" in only:
            extras["C3"] = c3(torch, device)
        if "route" in only:
            extras["route_chain"] = route_chain(torch, device)
        if "trace" in only:
            extras["route_trace"] = trace_replay(torch, device, args.route_trace or None)
    elif args.route_trace:
        extras["route_trace"] = trace_replay(torch, device, args.route_trace)

    # cpu_baseline leg: the oracle chain on the same headline inputs, timed
    # (not with --quick) and used to validate the timed run (always)
    cpu = None
    host = {k: v.cpu().numpy() for k, v in inputs.items()}
    ref = {}
    sec = cpu_chain_seconds(host, True, runs=1 if args.quick else 5, keep=ref)
    validation = validate_chain(cfg, host, head["timed_outputs"], ref)
    if not args.quick:
        from raggedroute_amd import workloads
        others = {}
        for c in (workloads.C1, workloads.C2):
            sec_c = cpu_chain_seconds(workloads.chain_inputs(c, 0), c.from_tokens)
            others[c.name] = {"tokens_per_s": round(c.tokens / sec_c, 1), "chain_ms": round(sec_c * 1e3, 3),
                              "entry": "chain_from_tokens" if c.from_tokens else "chain_from_logits"}
        for name in ("C4", "C5"):  # row / token samples taken while their inputs were on the device
            if name in extras and "cpu_sample" in extras[name]:
                others[name] = extras[name].pop("cpu_sample")
        cpu = {"value": round(cfg.tokens / sec, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"full headline chain_from_tokens (T={cfg.tokens}, E={cfg.experts}, K={cfg.hidden}, "
                         f"N={cfg.output}) on the oracle/ C restatement of the reference CPU chain "
                         f"(single thread, -O2 -ffp-contract=off), median of 5 runs",
               "chain_ms": round(sec * 1e3, 3), "configs": others, "cpu_model": cpu_model(),
               "host_cpus": os.cpu_count(), "threads_used": 1}

    line = {
        "metric": "chain_from_tokens tokens/s @T4096/E64 FP32; grouped GEMM TFLOP/s; GB/s",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["p50_s"] * 1e3, 5),
        "mean_chain_us": round(head["mean_s"] * 1e6, 2),
        "chain_warm": head["warm"],
        "validation": validation,
        "release_gate": {"ok": args.warmup >= 10 and head["samples"] >= 20 and validation["ok"],
                         "warmup": args.warmup, "samples": head["samples"], "validated": validation["ok"],
                         "requires": "warmup >= 10, samples >= 20, validation after measurement "
                                     "(reference benchmarks/core/runner.cpp:293-312)"},
        "environment": environment(torch, device),
        "chain_cold": head["cold"],
        "chain_graph": head["graph"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (SplitMix64 normal inputs generated in HBM, seed 0)",
        "config": {"workload": "chain_from_tokens", "T": cfg.tokens, "E": cfg.experts, "K": cfg.hidden,
                   "N": cfg.output, "top_k": 2, "active_experts": head["active_experts"]},
        "roofline": roof,
        "cpu_baseline": cpu,
        "launches": launches,
        "stages": head["stages"],
        "extras": extras,
    }
    print(json.dumps(line))
    if not validation["ok"]:
        print("post-benchmark validation failed: " + json.dumps(validation["checks"]), file=sys.stderr)
        return 3
    return 0


if __name__ == "__main__":
    sys.exit(main())
