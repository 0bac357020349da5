"""Post-route chain parity: chain_from_route_ids on the gfx950 library against
the oracle (reference benchmarks/adapters/postroute_chain_adapter.cpp:655-676
oracle, :357-385 validation).

counts, offsets, the stable route map and sorted_route are bit-exact; the
naive family (atomic placement) must satisfy the reference's bijection check
instead. y_permuted rows lie within the accumulation-aware GEMM bound
4*gamma_K*sum|x*w| + 1e-7 of the float64 product; y within the reference's
atol 1e-4 + rtol 4e-5*K*top_k (:381). Cases: the reference's own
(tests/correctness_tests.cpp:788-823: T5/E4/K7/N5 and T17/E16/K64/N64
duplicate_route for top_k 4, 8) and the post-route release shapes
(configs/project/benchmark/six_ops_v4_postroute_release.json).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import raggedroute_amd as rr
from raggedroute_amd import workloads
from conftest import to_dev, to_host

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


class RouteChainRun:
    def __init__(self, cfg: workloads.RouteChainConfig, inp: dict, device, kernel=None,
                 with_x_permuted=True, with_inverse=True):
        t, e, k, n, top = cfg.tokens, cfg.experts, cfg.hidden, cfg.output, cfg.top_k
        r = t * top
        i32 = dict(dtype=torch.int32, device=device)
        self.cfg = cfg
        self.x = to_dev(inp["x"], device)
        self.we = to_dev(inp["expert_weights"], device)
        self.ids = to_dev(inp["ids"].astype(np.int32), device)
        self.w = to_dev(inp["weights"], device)
        self.counts = torch.full((e,), -1, **i32)
        self.offsets = torch.full((e + 1,), -1, **i32)
        self.xp = torch.full((r, k), float("nan"), device=device) if with_x_permuted else None
        self.pos = torch.full((r,), -1, **i32)
        self.inv = torch.full((r,), -1, **i32) if with_inverse else None
        self.yp = torch.full((r, n), float("nan"), device=device)
        self.y = torch.full((t, n), float("nan"), device=device)
        ptr = lambda a: a.data_ptr() if a is not None else None  # noqa: E731
        self.args = rr.RouteChainArgs(
            x=ptr(self.x), expert_ids=ptr(self.ids), route_weights=ptr(self.w),
            expert_weights=ptr(self.we), counts=ptr(self.counts), offsets=ptr(self.offsets),
            x_permuted=ptr(self.xp), route_pos=ptr(self.pos), sorted_route=ptr(self.inv),
            y_permuted=ptr(self.yp), y=ptr(self.y), tokens=t, experts=e, top_k=top, hidden=k,
            output=n, kernel=kernel or rr.kernel())
        self.ws = torch.empty(max(1, rr.get_route_chain_workspace_size(self.args) // 4), **i32)

    def run(self, ctx):
        c = rr.RuntimeContext(stream=ctx.stream, workspace=self.ws.data_ptr(),
                              workspace_bytes=self.ws.numel() * 4, architecture=ctx.architecture)
        status = rr.chain_from_route_ids(self.args, c)
        assert status.ok(), status.message
        torch.cuda.synchronize()
        out = {"counts": to_host(self.counts), "offsets": to_host(self.offsets),
               "route_pos": to_host(self.pos), "y_permuted": to_host(self.yp), "y": to_host(self.y)}
        if self.xp is not None:
            out["x_permuted"] = to_host(self.xp)
        if self.inv is not None:
            out["sorted_route"] = to_host(self.inv)
        return out


def check_route_chain(cfg, inp, dev, stable=True):
    t, e, k, top = cfg.tokens, cfg.experts, cfg.hidden, cfg.top_k
    ids, w = inp["ids"], inp["weights"]
    exp = oracle.route_chain(inp["x"], inp["expert_weights"], ids, w)
    assert np.array_equal(dev["counts"], exp["counts"]), "counts differ from the oracle"
    assert np.array_equal(dev["offsets"], exp["offsets"]), "offsets differ from the oracle"
    flat = ids.reshape(-1)
    pos = dev["route_pos"]
    if stable:
        assert np.array_equal(pos, exp["route_pos"]), "route_pos differs from the stable oracle"
        if "sorted_route" in dev:
            assert np.array_equal(dev["sorted_route"], exp["sorted_route"])
    else:
        # reference bijection check (postroute_chain_adapter.cpp:363-376)
        off = exp["offsets"]
        assert ((pos >= off[flat]) & (pos < off[flat + 1])).all()
        assert np.array_equal(np.sort(pos), np.arange(flat.size))
        if "sorted_route" in dev:
            assert np.array_equal(dev["sorted_route"][pos], np.arange(flat.size))
    if "x_permuted" in dev:
        token = np.arange(flat.size) // top
        assert np.array_equal(dev["x_permuted"][pos].view(np.uint32), inp["x"][token].view(np.uint32))
    # expert rows: x[t] @ W[e] within the GEMM bound of the float64 product
    # (one product per expert segment)
    x64 = inp["x"].astype(np.float64)
    we64 = inp["expert_weights"].astype(np.float64)
    token = np.arange(flat.size) // top
    gamma = k * U32 / (1 - k * U32)
    yp = dev["y_permuted"]
    for e in np.unique(flat):
        routes = np.nonzero(flat == e)[0]
        xs = x64[token[routes]]
        exact = xs @ we64[e]
        bound = 4 * gamma * (np.abs(xs) @ np.abs(we64[e])) + 1e-7
        err = np.abs(yp[pos[routes]].astype(np.float64) - exact)
        assert (err <= bound).all(), f"y_permuted exceeds the GEMM bound (expert {e}, max ratio {(err / bound).max()})"
    fails, max_abs, _ = oracle.compare_floating(dev["y"], exp["y"], 1e-4, 4e-5 * k * top)
    assert fails == 0, f"route chain output: max |err| {max_abs}"


FAMILIES = [rr.KernelFamily.kAuto, rr.KernelFamily.kNaive]


@pytest.mark.parametrize("family", FAMILIES)
@pytest.mark.parametrize("top_k,distribution", [(2, "uniform"), (4, "duplicate_route"),
                                                (8, "duplicate_route")])
def test_route_chain_reference_cases(ctx, device, family, top_k, distribution):
    """reference tests/correctness_tests.cpp:788-823"""
    shape = (5, 4, 7, 5) if top_k == 2 else (17, 16, 64, 64)
    cfg = workloads.RouteChainConfig("ref", *shape, top_k, distribution)
    inp = workloads.route_chain_inputs(cfg, seed=2)
    run = RouteChainRun(cfg, inp, device, kernel=rr.kernel(family))
    check_route_chain(cfg, inp, run.run(ctx), stable=family != rr.KernelFamily.kNaive)


def _release_cases():
    cases = []
    for name, cfg in workloads.route_chain_configs().items():
        dists = ["uniform", "zipf", "single_hot"] if name.startswith("small") else ["uniform", "zipf"]
        cases += [(name, d) for d in dists]
    return cases


@pytest.mark.parametrize("name,distribution", _release_cases())
def test_route_chain_release_shapes(ctx, device, name, distribution):
    base = workloads.route_chain_configs()[name]
    cfg = workloads.RouteChainConfig(base.name, base.tokens, base.experts, base.hidden, base.output,
                                     base.top_k, distribution)
    print(f"route chain {name} {distribution}", flush=True)
    inp = workloads.route_chain_inputs(cfg, seed=7)
    check_route_chain(cfg, inp, RouteChainRun(cfg, inp, device).run(ctx))


@pytest.mark.parametrize("shape", [(1, 1, 1, 4, 4), (33, 5, 3, 12, 9), (300, 1024, 8, 20, 12),
                                   (2000, 128, 4, 260, 40), (700, 256, 2, 64, 130), (9, 6, 2, 0, 8),
                                   (9, 6, 2, 8, 0), (600, 64, 2, 252, 128), (500, 32, 4, 228, 64)])
def test_route_chain_edge_shapes(ctx, device, shape):
    """E = top_k = 1, odd K / N (no vector path), E = 1024, K above the strip
    limit (route_prep + tiled gathered GEMM), N above it, K = 0 and N = 0,
    and K tails of the strip kernel's register B (252: masked rows in the
    last k chunk; 228: fifteen chunks)."""
    t, e, top, k, n = shape
    cfg = workloads.RouteChainConfig("edge", t, e, k, n, top, "uniform")
    inp = workloads.route_chain_inputs(cfg, seed=13)
    print(f"route chain edge {shape}", flush=True)
    check_route_chain(cfg, inp, RouteChainRun(cfg, inp, device).run(ctx))


def test_route_chain_empty(ctx, device):
    cfg = workloads.RouteChainConfig("empty", 1, 8, 16, 16, 4)
    inp = workloads.route_chain_inputs(cfg, seed=0)
    run = RouteChainRun(cfg, inp, device)
    run.args.tokens = 0
    dev = run.run(ctx)
    assert (dev["counts"] == -1).all() and np.isnan(dev["y"]).all()  # nothing written


def _stages(cfg, inp, device, ctx):
    """The five public operators one by one with the native kernels."""
    t, e, k, n, top = cfg.tokens, cfg.experts, cfg.hidden, cfg.output, cfg.top_k
    r = t * top
    native = rr.kernel(rr.KernelFamily.kOptimized, rr.GFX950_NATIVE)
    i32 = dict(dtype=torch.int32, device=device)
    x, we = to_dev(inp["x"], device), to_dev(inp["expert_weights"], device)
    ids, w = to_dev(inp["ids"], device), to_dev(inp["weights"], device)
    counts, offsets = torch.empty(e, **i32), torch.empty(e + 1, **i32)
    xp, pos, inv = torch.empty(r, k, device=device), torch.empty(r, **i32), torch.empty(r, **i32)
    yp, y, cursors = torch.empty(r, n, device=device), torch.empty(t, n, device=device), torch.empty(e, **i32)

    def ok(status):
        assert status.ok(), status.message
    ok(rr.histogram(rr.HistogramArgs(expert_ids=ids.data_ptr(), counts=counts.data_ptr(), route_pairs=r,
                                     experts=e, kernel=native), ctx))
    ok(rr.exclusive_scan(rr.ExclusiveScanArgs(counts=counts.data_ptr(), offsets=offsets.data_ptr(),
                                              experts=e, kernel=native), ctx))
    pctx = rr.RuntimeContext(stream=ctx.stream, workspace=cursors.data_ptr(), workspace_bytes=4 * e,
                             architecture=ctx.architecture)
    ok(rr.token_permute(rr.TokenPermuteArgs(
        x=rr.cview(x.data_ptr()), expert_ids=ids.data_ptr(), offsets=offsets.data_ptr(),
        x_permuted=rr.mview(xp.data_ptr()), route_pos=pos.data_ptr(), sorted_route=inv.data_ptr(), tokens=t,
        experts=e, top_k=top, hidden=k, kernel=native), pctx))
    ok(rr.grouped_gemm(rr.GroupedGemmArgs(
        x_permuted=rr.cview(xp.data_ptr()), expert_weights=rr.cview(we.data_ptr()), offsets=offsets.data_ptr(),
        y_permuted=rr.mview(yp.data_ptr()), experts=e, hidden=k, output=n, max_expert_tokens=r,
        kernel=native), ctx))
    ok(rr.unpermute(rr.UnpermuteArgs(
        y_permuted=rr.cview(yp.data_ptr()), route_pos=pos.data_ptr(), route_weights=rr.cview(w.data_ptr()),
        y=rr.mview(y.data_ptr()), tokens=t, top_k=top, output=n, kernel=native), ctx))
    torch.cuda.synchronize()
    return {"counts": to_host(counts), "offsets": to_host(offsets), "route_pos": to_host(pos),
            "sorted_route": to_host(inv), "x_permuted": to_host(xp), "y_permuted": to_host(yp),
            "y": to_host(y)}


def _same(a, b):
    return np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                          b.view(np.uint32) if b.dtype == np.float32 else b)


@pytest.mark.parametrize("shape", [(512, 64, 2, 128, 128), (2048, 64, 8, 128, 128), (8192, 64, 8, 64, 64),
                                   (333, 7, 4, 13, 9), (1000, 128, 4, 300, 40),
                                   # 16384 routes: the merged launch's limit, four waves
                                   (4096, 64, 4, 128, 64)])
@pytest.mark.parametrize("with_x_permuted", [True, False])
def test_fused_route_chain_matches_stage_by_stage(ctx, device, shape, with_x_permuted):
    """The fused route chain (one merged launch + unpermute where the strip
    kernel covers the shape, route_prep + gathered GEMM + unpermute otherwise)
    writes the five stages' outputs bit-identically to the operators run one
    by one; without x_permuted every other output is unchanged."""
    t, e, top, k, n = shape
    cfg = workloads.RouteChainConfig("fused", t, e, k, n, top, "zipf")
    inp = workloads.route_chain_inputs(cfg, seed=17)
    print(f"fused route chain {shape} x_permuted={with_x_permuted}", flush=True)
    fused = RouteChainRun(cfg, inp, device, with_x_permuted=with_x_permuted).run(ctx)
    ref = _stages(cfg, inp, device, ctx)
    for key, a in fused.items():
        assert _same(a, ref[key]), f"{key} differs"
    check_route_chain(cfg, inp, fused)


@pytest.mark.parametrize("shape", [(512, 64, 2, 128, 128), (2048, 32, 4, 64, 64), (1000, 7, 3, 40, 24)])
def test_route_chain_repeats_bit_for_bit(ctx, device, shape):
    """Several calls on one set of buffers, every output poisoned before each:
    a slot, row or map entry that a call fails to write shows up as NaN or -7
    instead of passing on the previous call's value."""
    t, e, top, k, n = shape
    cfg = workloads.RouteChainConfig("repeat", t, e, k, n, top, "zipf")
    inp = workloads.route_chain_inputs(cfg, seed=11)
    run = RouteChainRun(cfg, inp, device)
    first = run.run(ctx)
    check_route_chain(cfg, inp, first)
    for _ in range(3):
        for attr in ("counts", "offsets", "xp", "pos", "inv", "yp", "y"):
            getattr(run, attr).fill_(float("nan") if getattr(run, attr).dtype == torch.float32 else -7)
        again = run.run(ctx)
        for key, v in first.items():
            a, b = (again[key].view(np.uint32), v.view(np.uint32)) if v.dtype == np.float32 else (again[key], v)
            assert np.array_equal(a, b), key


@pytest.mark.parametrize("shape", [(512, 64, 2, 128, 128), (2048, 32, 4, 64, 64), (1000, 128, 4, 300, 40)])
def test_route_chain_invalid_ids(ctx, device, shape):
    """Ids outside [0, E) (negative, E, E + 5) are never placed: they leave the
    counts, route_pos says -1 for them even where it held a valid index
    before the call, and y sums the valid routes of a token in rank order.
    Both launch plans (one merged strip launch; route_prep + tiled GEMM)."""
    t, e, top, k, n = shape
    r = t * top
    cfg = workloads.RouteChainConfig("invalid", t, e, k, n, top, "zipf")
    inp = workloads.route_chain_inputs(cfg, seed=23)
    ids = inp["ids"].reshape(-1).copy()
    rng = np.random.default_rng(5)
    bad = rng.choice(r, max(1, r // 20), replace=False)
    ids[bad] = rng.choice(np.array([-1, -9, e, e + 5], np.int32), bad.size)
    inp = dict(inp, ids=ids.reshape(t, top))
    print(f"route chain invalid ids {shape}", flush=True)
    run = RouteChainRun(cfg, inp, device)
    run.pos.fill_(0)  # a valid index: an entry the call leaves alone would stay 0
    dev = run.run(ctx)

    valid = (ids >= 0) & (ids < e)
    counts = np.bincount(ids[valid], minlength=e).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    assert np.array_equal(dev["counts"], counts)
    assert np.array_equal(dev["offsets"], offsets)
    want_pos = np.full(r, -1, np.int32)
    seen = offsets[:-1].copy()
    for route in range(r):  # stable order: route index ascending inside each expert
        if valid[route]:
            want_pos[route] = seen[ids[route]]
            seen[ids[route]] += 1
    assert np.array_equal(dev["route_pos"], want_pos), "route_pos differs (invalid routes must read -1)"
    placed = np.nonzero(valid)[0]
    assert np.array_equal(dev["sorted_route"][want_pos[placed]], placed)
    token = np.arange(r) // top
    assert np.array_equal(dev["x_permuted"][want_pos[placed]].view(np.uint32),
                          inp["x"][token[placed]].view(np.uint32))
    x64, we64 = inp["x"].astype(np.float64), inp["expert_weights"].astype(np.float64)
    gamma = k * U32 / (1 - k * U32)
    for ex in np.unique(ids[valid]):
        routes = np.nonzero(ids == ex)[0]
        xs = x64[token[routes]]
        exact = xs @ we64[ex]
        bound = 4 * gamma * (np.abs(xs) @ np.abs(we64[ex])) + 1e-7
        assert (np.abs(dev["y_permuted"][want_pos[routes]].astype(np.float64) - exact) <= bound).all()
    # y: rank-order FP32 sum from zero over the token's valid routes
    w = inp["weights"].reshape(-1).astype(np.float32)
    want_y = np.zeros((t, n), np.float32)
    for j in range(top):
        routes = np.arange(t) * top + j
        ok_r = valid[routes]
        term = np.zeros((t, n), np.float32)
        term[ok_r] = w[routes[ok_r], None] * dev["y_permuted"][want_pos[routes[ok_r]]]
        want_y = np.where(ok_r[:, None], want_y + term, want_y)
    assert np.array_equal(dev["y"].view(np.uint32), want_y.view(np.uint32)), "y differs"
