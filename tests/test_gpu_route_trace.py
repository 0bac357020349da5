"""Route-trace replay on the gfx950 library: frames read by the native reader
drive chain_from_logits (logits built to select the frame's ids, reference
benchmarks/adapters/chain_adapter.cpp:209-230), chain_from_route_ids and the
grouped GEMM (segment sizes from the frame, reference
benchmarks/adapters/grouped_gemm_adapter.cpp:185-197), each against the oracle.
Frames: the reference fixture and a generated T4096 / E64 trace with
uniform, Zipf-skewed and single-hot frames, written as text and read back.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
import raggedroute_amd as rr
from raggedroute_amd import route_trace, workloads
from conftest import to_dev, to_host
from test_gpu_chain import ChainRun, check_chain
from test_gpu_route_chain import RouteChainRun, check_route_chain

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "synthetic_fixture.rrtrace"


def generated_trace(tmp_path, tokens=4096, experts=64, top_k=2):
    frames = {
        "uniform": workloads.topk_route_ids(tokens, top_k, experts, "uniform", seed=1),
        "zipf1.4": workloads.topk_route_ids(tokens, top_k, experts, "zipf", seed=2, s=1.4),
        "round_robin": workloads.topk_route_ids(tokens, top_k, experts, "round_robin", seed=3),
        "single_hot": workloads.topk_route_ids(tokens, top_k, experts, "single_hot", seed=4),
    }
    path = tmp_path / "generated.rrtrace"
    route_trace.write(path, "generated_t4096", "synthetic_fixture", experts, frames)
    return path, frames


def test_fixture_replay_chain_from_logits(ctx, device):
    for tr in route_trace.read_all(FIXTURE):
        cfg = workloads.ChainConfig("trace", tr.tokens, tr.experts, 64, 64, from_tokens=False)
        inp = workloads.chain_inputs(cfg, seed=1)
        inp["logits"] = route_trace.logits_for_ids(tr.ids, tr.experts)
        dev = ChainRun(cfg, inp, device).run(ctx)
        assert np.array_equal(dev["ids"], tr.ids), tr.frame_id
        check_chain(cfg, inp, dev)


@pytest.mark.parametrize("top_k", [2, 4, 8])
def test_generated_trace_replay_route_chain(ctx, device, tmp_path, top_k):
    path, frames = generated_trace(tmp_path, top_k=top_k)
    for index, (name, ids) in enumerate(frames.items()):
        tr = route_trace.read(path, index)
        assert tr.frame_id == name and np.array_equal(tr.ids, ids)
        print(f"replay route chain top_k={top_k} frame={name}", flush=True)
        cfg = workloads.RouteChainConfig(name, tr.tokens, tr.experts, 256, 128, top_k)
        inp = workloads.route_chain_inputs(cfg, seed=index)
        inp["ids"] = tr.ids
        check_route_chain(cfg, inp, RouteChainRun(cfg, inp, device).run(ctx))


def test_generated_trace_replay_chain_from_logits(ctx, device, tmp_path):
    path, _ = generated_trace(tmp_path)
    for tr in route_trace.read_all(path):
        print(f"replay chain_from_logits frame={tr.frame_id}", flush=True)
        cfg = workloads.ChainConfig(tr.frame_id, tr.tokens, tr.experts, 256, 128, from_tokens=False)
        inp = workloads.chain_inputs(cfg, seed=5)
        inp["logits"] = route_trace.logits_for_ids(tr.ids, tr.experts)
        dev = ChainRun(cfg, inp, device).run(ctx)
        assert np.array_equal(dev["ids"], tr.ids), tr.frame_id
        check_chain(cfg, inp, dev)


def test_generated_trace_replay_grouped_gemm(ctx, device, tmp_path):
    """Grouped GEMM segments sized by a frame's counts (rows = routes of each expert)."""
    path, _ = generated_trace(tmp_path, tokens=2048)
    k, n = 192, 96
    for tr in route_trace.read_all(path):
        counts = oracle.histogram(tr.ids, tr.experts)
        offsets = oracle.exclusive_scan(counts)
        r = int(offsets[-1])
        x = workloads.uniform(r * k, 3, workloads.S_X).reshape(r, k)
        w = workloads.uniform(tr.experts * k * n, 3, workloads.S_EXPERTS).reshape(tr.experts, k, n)
        xd, wd, od = to_dev(x, device), to_dev(w, device), to_dev(offsets, device)
        y = torch.empty(r, n, device=device)
        st = rr.grouped_gemm(rr.GroupedGemmArgs(
            x_permuted=rr.cview(xd.data_ptr()), expert_weights=rr.cview(wd.data_ptr()),
            offsets=od.data_ptr(), y_permuted=rr.mview(y.data_ptr()), experts=tr.experts, hidden=k,
            output=n, max_expert_tokens=int(counts.max())), ctx)
        assert st.ok(), st.message
        got = to_host(y).astype(np.float64)
        exact = oracle.grouped_gemm_f64(x, w, offsets)
        # accumulation-aware bound 4*gamma_K*sum|x*w| + 1e-7 per element, per segment
        gamma = k * 2.0**-24 / (1 - k * 2.0**-24)
        for e in range(tr.experts):
            lo, hi = offsets[e], offsets[e + 1]
            bound = 4 * gamma * (np.abs(x[lo:hi].astype(np.float64)) @ np.abs(w[e].astype(np.float64))) + 1e-7
            assert (np.abs(got[lo:hi] - exact[lo:hi]) <= bound).all(), (tr.frame_id, e)
