"""Chain graphs on the gfx950 library (rr_chain_graph_*, rr_chain_graph_cache_*):
the reference's CUDA-graph chain variants (benchmarks/adapters/chain_adapter.cpp:
730-826, :962-1000) and their tests (tests/correctness_tests.cpp:60-128: replay,
logical-case match, cache eviction).

Every replay is checked bit for bit against the eager call on the same inputs;
replays are interleaved with eager chain calls and synchronisations, outputs
are poisoned before each replay, and inputs are rewritten in place between
replays (a graph reads its buffers' current contents).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import raggedroute_amd as rr
from raggedroute_amd import workloads
from conftest import to_dev, to_host
from test_gpu_chain import ChainRun, check_chain
from test_gpu_route_chain import RouteChainRun, check_route_chain

pytestmark = pytest.mark.gpu

CHAIN_OUT = ("logits", "ids", "w", "counts", "offsets", "pos", "inv", "xp", "yp", "y")
ROUTE_OUT = ("counts", "offsets", "pos", "inv", "xp", "yp", "y")


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = to_host(a), to_host(b)
    return np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                          b.view(np.uint32) if b.dtype == np.float32 else b)


def _poison(run, names):
    for n in names:
        t = getattr(run, n)
        if t is not None and t.numel():
            t.fill_(float("nan") if t.dtype == torch.float32 else -7)


def _side_ctx(run, stream):
    return rr.RuntimeContext(stream=stream.cuda_stream, workspace=run.ws.data_ptr(),
                             workspace_bytes=run.ws.numel() * 4,
                             architecture=int(rr.DeviceArchitecture.kGfx950))


CASES = [
    ("tokens", workloads.HEADLINE),
    ("tokens", workloads.C1),
    ("logits", workloads.ChainConfig("C2g", 4096, 64, 256, 128, from_tokens=False)),
    ("tokens", workloads.ChainConfig("k300", 1000, 32, 300, 40)),  # three-launch plan
]


@pytest.mark.parametrize("kind,cfg", CASES, ids=[c[1].name for c in CASES])
def test_graph_replays_equal_eager(device, kind, cfg):
    inp = workloads.chain_inputs(cfg, seed=21)
    eager, graphed = ChainRun(cfg, inp, device), ChainRun(cfg, inp, device)
    stream = torch.cuda.Stream(device)
    ctx = _side_ctx(graphed, stream)
    entry = rr.CHAIN_FROM_TOKENS if cfg.from_tokens else rr.CHAIN_FROM_LOGITS
    ectx = _side_ctx(eager, stream)
    with rr.ChainGraph(entry, graphed.args, ctx) as graph:
        assert graph.kernel_nodes in (2, 3, 4)
        for replay in range(4):
            if replay == 2:  # new inputs in place: the graph reads them at replay time
                new = workloads.chain_inputs(cfg, seed=99)
                inp = dict(inp, x=new["x"], **({} if cfg.from_tokens else {"logits": new["logits"]}))
                for run in (eager, graphed):
                    run.x.copy_(to_dev(inp["x"], device))
                    if not cfg.from_tokens:
                        run.logits.copy_(to_dev(inp["logits"], device))
            eager.run(ectx)  # eager work between replays
            _poison(graphed, CHAIN_OUT if cfg.from_tokens else [n for n in CHAIN_OUT if n != "logits"])
            torch.cuda.synchronize()
            st = graph.launch(stream.cuda_stream)
            assert st.ok(), st.message
            torch.cuda.synchronize()
            for n in CHAIN_OUT:
                assert _same(getattr(graphed, n), getattr(eager, n)), (replay, n)
        dev = {k: to_host(getattr(graphed, a)) for k, a in
               [("logits", "logits"), ("ids", "ids"), ("weights", "w"), ("counts", "counts"),
                ("offsets", "offsets"), ("route_pos", "pos"), ("y", "y"), ("x_permuted", "xp"),
                ("y_permuted", "yp")]}
        check_chain(cfg, inp, dev)


def test_graph_long_replay(device):
    """200 replays; checked at replay 1, 2 and the last (reference replay test)."""
    cfg = workloads.ChainConfig("r", 17, 16, 64, 64, from_tokens=False)
    inp = workloads.chain_inputs(cfg, seed=3)
    eager, graphed = ChainRun(cfg, inp, device), ChainRun(cfg, inp, device)
    stream = torch.cuda.Stream(device)
    eager.run(_side_ctx(eager, stream))
    with rr.ChainGraph(rr.CHAIN_FROM_LOGITS, graphed.args, _side_ctx(graphed, stream)) as graph:
        for replay in range(200):
            st = graph.launch(stream.cuda_stream)
            assert st.ok(), st.message
            if replay < 2 or replay == 199:
                torch.cuda.synchronize()
                for n in [n for n in CHAIN_OUT if n != "logits"]:
                    assert _same(getattr(graphed, n), getattr(eager, n)), (replay, n)
                _poison(graphed, [n for n in CHAIN_OUT if n != "logits"])
                torch.cuda.synchronize()


@pytest.mark.parametrize("top_k", [2, 4, 8])
def test_route_chain_graph_and_update(device, top_k):
    """Post-route chain graph; update() re-points it at a second set of buffers
    (same shape) and then at a different token count."""
    cfg = workloads.RouteChainConfig("g", 512, 64, 128, 128, top_k, "zipf")
    inp = workloads.route_chain_inputs(cfg, seed=4)
    eager, first, second = (RouteChainRun(cfg, inp, device) for _ in range(3))
    stream = torch.cuda.Stream(device)
    eager.run(_side_ctx(eager, stream))
    with rr.ChainGraph(rr.CHAIN_FROM_ROUTE_IDS, first.args, _side_ctx(first, stream)) as graph:
        for replay in range(2):
            _poison(first, ROUTE_OUT)
            torch.cuda.synchronize()
            assert graph.launch(stream.cuda_stream).ok()
            torch.cuda.synchronize()
            for n in ROUTE_OUT:
                assert _same(getattr(first, n), getattr(eager, n)), (replay, n)
        st = graph.update(second.args, _side_ctx(second, stream))
        assert st.ok(), st.message
        _poison(first, ROUTE_OUT)
        _poison(second, ROUTE_OUT)
        torch.cuda.synchronize()
        assert graph.launch(stream.cuda_stream).ok()
        torch.cuda.synchronize()
        for n in ROUTE_OUT:
            assert _same(getattr(second, n), getattr(eager, n)), ("updated", n)
        assert np.isnan(to_host(first.y)).all()  # the old buffers are no longer written
        # a different token count (another launch plan) through update()
        small = workloads.RouteChainConfig("g2", 300, 64, 128, 128, top_k, "uniform")
        sinp = workloads.route_chain_inputs(small, seed=5)
        s_eager, s_graph = RouteChainRun(small, sinp, device), RouteChainRun(small, sinp, device)
        s_eager.run(_side_ctx(s_eager, stream))
        assert graph.update(s_graph.args, _side_ctx(s_graph, stream)).ok()
        torch.cuda.synchronize()
        assert graph.launch(stream.cuda_stream).ok()
        torch.cuda.synchronize()
        for n in ROUTE_OUT:
            assert _same(getattr(s_graph, n), getattr(s_eager, n)), ("resized", n)
        dev = {"counts": to_host(s_graph.counts), "offsets": to_host(s_graph.offsets),
               "route_pos": to_host(s_graph.pos), "sorted_route": to_host(s_graph.inv),
               "x_permuted": to_host(s_graph.xp), "y_permuted": to_host(s_graph.yp), "y": to_host(s_graph.y)}
        check_route_chain(small, sinp, dev)


def test_graph_cache_eviction(device):
    """reference tests/correctness_tests.cpp:93-115: 17 token counts over a
    16-entry cache, 18 launches revisiting the first (evicted) key."""
    stream = torch.cuda.Stream(device)
    runs = {}
    for t in range(64, 81):
        cfg = workloads.ChainConfig(f"c{t}", t, 16, 64, 64, from_tokens=False)
        inp = workloads.chain_inputs(cfg, seed=t)
        runs[t] = (cfg, inp, ChainRun(cfg, inp, device))
    with rr.ChainGraphCache(16) as cache:
        order = list(range(64, 81)) + [64]
        for t in order:
            cfg, inp, run = runs[t]
            st = cache.launch(rr.CHAIN_FROM_LOGITS, run.args, _side_ctx(run, stream))
            assert st.ok(), st.message
        torch.cuda.synchronize()
        s = cache.stats()
        assert (s.capacity, s.entries) == (16, 16)
        assert s.misses == 18 and s.hits == 0
        for t in (64, 80, 79):  # resident keys hit
            cfg, inp, run = runs[t]
            _poison(run, [n for n in CHAIN_OUT if n != "logits"])
            torch.cuda.synchronize()
            assert cache.launch(rr.CHAIN_FROM_LOGITS, run.args, _side_ctx(run, stream)).ok()
            torch.cuda.synchronize()
            dev = {k: to_host(getattr(run, a)) for k, a in
                   [("logits", "logits"), ("ids", "ids"), ("weights", "w"), ("counts", "counts"),
                    ("offsets", "offsets"), ("route_pos", "pos"), ("y", "y"), ("x_permuted", "xp"),
                    ("y_permuted", "yp")]}
            check_chain(cfg, inp, dev)
        s = cache.stats()
        assert s.hits == 3 and s.misses == 18 and s.entries == 16


def test_graph_rejections(device):
    cfg = workloads.ChainConfig("rej", 64, 16, 64, 64, from_tokens=False)
    inp = workloads.chain_inputs(cfg, seed=0)
    run = ChainRun(cfg, inp, device, kernel=rr.kernel(rr.KernelFamily.kNaive))
    stream = torch.cuda.Stream(device)
    with pytest.raises(RuntimeError, match="optimized family"):
        rr.ChainGraph(rr.CHAIN_FROM_LOGITS, run.args, _side_ctx(run, stream))
    run.args.kernel = rr.kernel()
    default_ctx = rr.RuntimeContext(stream=None, workspace=run.ws.data_ptr(),
                                    workspace_bytes=run.ws.numel() * 4)
    with pytest.raises(RuntimeError, match="non-default stream"):
        rr.ChainGraph(rr.CHAIN_FROM_LOGITS, run.args, default_ctx)
    with pytest.raises(RuntimeError, match="unknown chain entry"):
        rr.ChainGraph(7, run.args, _side_ctx(run, stream))
    run.args.top_k = 3  # invalid call: the direct entry's validation, nothing captured
    with pytest.raises(RuntimeError, match="top_k=2"):
        rr.ChainGraph(rr.CHAIN_FROM_LOGITS, run.args, _side_ctx(run, stream))
    with pytest.raises(RuntimeError):
        rr.ChainGraphCache(0)


def test_graph_sequence_of_chains(device):
    """Three chain calls with their own buffers and shapes (three MoE layers
    of a step) recorded into one graph: every replay writes each layer's
    outputs bit-identically to that layer's eager call; an update with the
    layers' args in another order rebinds them; an update with another call
    count is rejected."""
    cfgs = [workloads.HEADLINE, workloads.C1, workloads.ChainConfig("seq3", 700, 16, 300, 40)]
    inps = [workloads.chain_inputs(c, seed=40 + i) for i, c in enumerate(cfgs)]
    eager = [ChainRun(c, x, device) for c, x in zip(cfgs, inps)]
    graphed = [ChainRun(c, x, device) for c, x in zip(cfgs, inps)]
    stream = torch.cuda.Stream(device)
    # one workspace large enough for every layer (calls run in order)
    ws = max(graphed, key=lambda r: r.ws.numel()).ws
    ctx = rr.RuntimeContext(stream=stream.cuda_stream, workspace=ws.data_ptr(), workspace_bytes=ws.numel() * 4,
                            architecture=int(rr.DeviceArchitecture.kGfx950))
    for run in eager:
        run.run(_side_ctx(run, stream))
    with rr.ChainGraph(rr.CHAIN_FROM_TOKENS, [g.args for g in graphed], ctx) as graph:
        assert graph.kernel_nodes >= 6
        for order in ([0, 1, 2], [2, 0, 1]):
            if order != [0, 1, 2]:
                st = graph.update([graphed[i].args for i in order], ctx)
                assert st.ok(), st.message
            for _ in range(3):
                for run in graphed:
                    _poison(run, CHAIN_OUT)
                eager[1].run(_side_ctx(eager[1], stream))  # eager work between replays
                torch.cuda.synchronize()
                st = graph.launch(stream.cuda_stream)
                assert st.ok(), st.message
                torch.cuda.synchronize()
                for e, g in zip(eager, graphed):
                    for name in CHAIN_OUT:
                        assert _same(getattr(g, name), getattr(e, name)), f"{g.cfg.name}: {name} differs"
        st = graph.update([graphed[0].args, graphed[1].args], ctx)
        assert st.code == rr.StatusCode.kInvalidArgument
