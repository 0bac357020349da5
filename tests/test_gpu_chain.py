"""Chain parity: chain_from_tokens / chain_from_logits on the gfx950 library
against the reference chain oracle (reference
benchmarks/adapters/chain_adapter.cpp:188-239, validate :469-495).

Integer outputs are bit-exact: top-2 ids against the oracle top-2 applied to
the device logits (chain_from_tokens: the MFMA router sums in a different
order than the sequential CPU loop, so the logits themselves are checked
against the accumulation-aware GEMM bound and rows whose CPU rank-2/rank-3
margin lies inside that bound are counted as near-ties), counts, offsets and
the stable route map. Weights within 1e-6 (reference chain tolerance), the
final output within atol 1e-4 + rtol 4e-5*K (reference chain_adapter.cpp:492).
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


class ChainRun:
    def __init__(self, cfg: workloads.ChainConfig, inputs: dict, device, kernel=None, with_inverse=True):
        t, e, k, n = cfg.tokens, cfg.experts, cfg.hidden, cfg.output
        self.cfg = cfg
        dev = lambda a: a if isinstance(a, torch.Tensor) else to_dev(a, device)  # noqa: E731
        self.x = dev(inputs["x"])
        self.we = dev(inputs["expert_weights"])
        self.wr = dev(inputs["router_weights"]) if cfg.from_tokens else None
        self.logits = (torch.empty(t, e, device=device) if cfg.from_tokens
                       else to_dev(inputs["logits"], device))
        i32 = dict(dtype=torch.int32, device=device)
        self.ids = torch.full((t, 2), -1, **i32)
        self.w = torch.empty(t, 2, device=device)
        self.counts = torch.full((e,), -1, **i32)
        self.offsets = torch.full((e + 1,), -1, **i32)
        self.xp = torch.empty(2 * t, k, device=device)
        self.pos = torch.full((2 * t,), -1, **i32)
        self.inv = torch.full((2 * t,), -1, **i32) if with_inverse else None
        self.yp = torch.empty(2 * t, n, device=device)
        self.y = torch.empty(t, n, device=device)
        self.args = rr.ChainArgs(
            x=self.x.data_ptr(), router_weights=self.wr.data_ptr() if self.wr is not None else None,
            logits=self.logits.data_ptr(), expert_ids=self.ids.data_ptr(), route_weights=self.w.data_ptr(),
            counts=self.counts.data_ptr(), offsets=self.offsets.data_ptr(), x_permuted=self.xp.data_ptr(),
            route_pos=self.pos.data_ptr(), sorted_route=self.inv.data_ptr() if self.inv is not None else None,
            expert_weights=self.we.data_ptr(), y_permuted=self.yp.data_ptr(), y=self.y.data_ptr(),
            tokens=t, experts=e, hidden=k, output=n, kernel=kernel or rr.kernel())
        self.ws = torch.empty(rr.get_chain_workspace_size(self.args) // 4, **i32)

    def run(self, ctx):
        c = rr.RuntimeContext(stream=ctx.stream, workspace=self.ws.data_ptr(),
                              workspace_bytes=self.ws.numel() * 4, architecture=ctx.architecture)
        fn = rr.chain_from_tokens if self.cfg.from_tokens else rr.chain_from_logits
        status = fn(self.args, c)
        assert status.ok(), status.message
        torch.cuda.synchronize()
        return {name: to_host(getattr(self, attr)) for name, attr in
                [("logits", "logits"), ("ids", "ids"), ("weights", "w"), ("counts", "counts"),
                 ("offsets", "offsets"), ("route_pos", "pos"), ("y", "y"), ("x_permuted", "xp"),
                 ("y_permuted", "yp")]} | ({"sorted_route": to_host(self.inv)} if self.inv is not None else {})


def logits_bound(x, wr):
    """Per-element accumulation-aware bound 4*gamma_K*sum|x*w| + 1e-7."""
    k = x.shape[1]
    gamma = k * U32 / (1 - k * U32)
    return 4 * gamma * (np.abs(x.astype(np.float64)) @ np.abs(wr.astype(np.float64))) + 1e-7


def check_chain(cfg, inp, dev, sample_tokens=None, stable=True):
    t, e, k = cfg.tokens, cfg.experts, cfg.hidden
    report = {}
    if cfg.from_tokens:
        rows = np.arange(t) if sample_tokens is None else sample_tokens
        x_s = inp["x"][rows]
        exact = oracle.dense_gemm_f64(x_s, inp["router_weights"])
        err = np.abs(dev["logits"][rows].astype(np.float64) - exact)
        bound = logits_bound(x_s, inp["router_weights"])
        assert (err <= bound).all(), f"router logits exceed the GEMM bound (max ratio {(err / bound).max()})"
        # near-tie rows: the CPU's 1st/2nd or 2nd/3rd logits closer than twice the bound
        cpu_logits = oracle.dense_gemm_f32_seq(x_s, inp["router_weights"])
        srt = np.sort(cpu_logits.astype(np.float64), axis=1)[:, ::-1]
        margin = np.minimum(srt[:, 0] - srt[:, 1], srt[:, 1] - srt[:, 2])
        near = margin <= 2 * bound.max(axis=1)
        report["near_tie_rows"] = int(near.sum())
        cpu_ids, _ = oracle.top2_f32(cpu_logits)
        differ = (cpu_ids != dev["ids"][rows]).any(axis=1)
        report["id_rows_differing_from_cpu_logits"] = int(differ.sum())
        # ids may differ from the CPU-logit oracle only on near-tie rows
        assert near[differ].all()
        logits = dev["logits"]
    else:
        logits = inp["logits"]
        assert np.array_equal(dev["logits"], logits)
    ids, w = oracle.top2_f32(logits)
    assert np.array_equal(dev["ids"], ids), "chain ids differ from the oracle top-2"
    fails, max_abs, _ = oracle.compare_floating(dev["weights"], w, 1e-6, 1e-6)
    assert fails == 0, f"chain weights: max |err| {max_abs}"
    counts = oracle.histogram(ids, e)
    offsets = oracle.exclusive_scan(counts)
    assert np.array_equal(dev["counts"], counts) and np.array_equal(dev["offsets"], offsets)
    if stable:
        pos = oracle.stable_route_pos(ids, offsets)
        assert np.array_equal(dev["route_pos"], pos)
        if "sorted_route" in dev:
            assert np.array_equal(dev["sorted_route"], oracle.inverse_route(pos))
    else:
        # naive family: atomic placement, order unspecified (reference
        # token_permute_adapter.cpp:436-443); every reference invariant holds
        pos = dev["route_pos"]
        assert oracle.validate_permute(inp["x"], ids, offsets, dev["x_permuted"], pos,
                                       dev.get("sorted_route"), 2) == []
    # final output: reference chain oracle on the device ids/weights
    tok = np.arange(t) if sample_tokens is None else sample_tokens
    y_exp = oracle.chain_output_f32(inp["x"][tok], inp["expert_weights"], ids[tok], w[tok])
    fails, max_abs, max_rel = oracle.compare_floating(dev["y"][tok], y_exp, 1e-4, 4e-5 * k)
    assert fails == 0, f"chain output: max |err| {max_abs}"
    report["y_max_abs"] = max_abs
    # x_permuted rows are bitwise copies (reference permute reference.cpp:65-71)
    src = pos.reshape(t, 2)[tok]
    assert np.array_equal(dev["x_permuted"][src[:, 0]].view(np.uint32), inp["x"][tok].view(np.uint32))
    assert np.array_equal(dev["x_permuted"][src[:, 1]].view(np.uint32), inp["x"][tok].view(np.uint32))
    return report


@pytest.mark.parametrize("kernel_family", [rr.KernelFamily.kAuto, rr.KernelFamily.kNaive])
def test_chain_tiny_shape(ctx, device, kernel_family):
    # reference tests/correctness_tests.cpp:788-802 runs every chain at T5/E4/K7/N5
    for from_tokens in (True, False):
        cfg = workloads.ChainConfig("tiny", 5, 4, 7, 5, from_tokens=from_tokens)
        inp = workloads.chain_inputs(cfg, seed=0)
        dev = ChainRun(cfg, inp, device, rr.kernel(kernel_family)).run(ctx)
        check_chain(cfg, inp, dev, stable=kernel_family != rr.KernelFamily.kNaive)


@pytest.mark.parametrize("name", ["C1", "headline", "C2"])
def test_chain_configs(ctx, device, name):
    cfg = workloads.CHAIN_CONFIGS[name]
    inp = workloads.chain_inputs(cfg, seed=0)
    run = ChainRun(cfg, inp, device)
    report = check_chain(cfg, inp, run.run(ctx))
    print(f"{name}: {report}")
    # repeated invocation on the same buffers is deterministic; every output is
    # poisoned before each repeat, so a row or map entry a run fails to write
    # cannot pass on the previous run's value
    first = run.run(ctx)
    for _ in range(3):
        for attr in ("ids", "w", "counts", "offsets", "pos", "inv", "xp", "yp", "y") + \
                (("logits",) if cfg.from_tokens else ()):
            t = getattr(run, attr)
            if t is not None and t.numel():
                t.fill_(float("nan") if t.dtype == torch.float32 else -7)
        again = run.run(ctx)
        for key in ("ids", "weights", "counts", "offsets", "route_pos", "x_permuted", "y_permuted", "y"):
            assert np.array_equal(again[key].view(np.uint32) if again[key].dtype == np.float32 else again[key],
                                  first[key].view(np.uint32) if first[key].dtype == np.float32 else first[key]), key


def test_chain_c5_every_element(ctx, device):
    """C5 (T=16384, K=2048, E=128, N=768). Against the oracle: integer outputs
    in full, floats on a seeded sample of 192 tokens (the full FP32 CPU chain
    is ~52 GMAC). Every float element on the device, as the reference's chain
    check compares the entire output (reference
    benchmarks/adapters/chain_adapter.cpp:487-494): the naive family's
    chain_from_logits runs on the fused run's device logits, so both take the
    same ids, and its output is pinned to the oracle's loop bit for bit on
    the sampled tokens. Then y on every token within the chain tolerance of
    the naive chain, y_permuted on every route (row by row through each run's
    route map) within 3 * gamma_K * S / (1 - gamma_K) + 1e-7 of the naive
    rows, S = sum_k |a*b| from the naive GEMM on |x| and |W| (so within the
    reference bound 4 * gamma_K * S + 1e-7 of the exact product, since the
    naive sequential sum lies within gamma_K * S of it), and x_permuted on
    every route bitwise."""
    cfg = workloads.C5
    t, e, k, n = cfg.tokens, cfg.experts, cfg.hidden, cfg.output
    r = 2 * t
    inp_dev = workloads.chain_inputs_device(cfg, 0, device)
    fused = ChainRun(cfg, inp_dev, device)
    dev = fused.run(ctx)
    inp = {key: to_host(v) for key, v in inp_dev.items()}
    sample = np.sort(workloads.seeded_permutation(t, 0, 77)[:192])
    report = check_chain(cfg, inp, dev, sample_tokens=sample)

    lcfg = workloads.ChainConfig("C5 naive on device logits", t, e, k, n, from_tokens=False)
    naive = ChainRun(lcfg, {"x": inp_dev["x"], "expert_weights": inp_dev["expert_weights"],
                            "logits": dev["logits"]}, device, rr.kernel(rr.KernelFamily.kNaive))
    nd = naive.run(ctx)
    assert np.array_equal(nd["ids"], dev["ids"]), "naive and fused chains picked different ids"
    assert oracle.compare_floating(nd["weights"], dev["weights"], 1e-6, 1e-6)[0] == 0
    assert np.array_equal(nd["counts"], dev["counts"]) and np.array_equal(nd["offsets"], dev["offsets"])
    assert oracle.validate_permute(inp["x"], nd["ids"], nd["offsets"], nd["x_permuted"], nd["route_pos"],
                                   nd.get("sorted_route"), 2) == []
    # the naive chain is the oracle's loop: bit-exact on the sampled tokens
    # given its own weights
    y_seq = oracle.chain_output_f32(inp["x"][sample], inp["expert_weights"], nd["ids"][sample],
                                    nd["weights"][sample])
    assert np.array_equal(nd["y"][sample].view(np.uint32), y_seq.view(np.uint32)), \
        "naive chain output differs from the oracle loop"

    # y: every token
    fails, max_abs, _ = oracle.compare_floating(dev["y"], nd["y"], 1e-4, 4e-5 * k)
    assert fails == 0, f"chain output: {fails} elements outside the chain tolerance (max |err| {max_abs})"
    report["y_every_token_max_abs_vs_naive"] = max_abs
    del dev, nd

    # y_permuted: every route, through each run's map
    pos_f, pos_n = fused.pos.long(), naive.pos.long()
    sabs = torch.full((r, n), float("nan"), device=device)
    xa, wa = naive.xp.abs(), naive.we.abs()
    assert rr.grouped_gemm(rr.GroupedGemmArgs(
        x_permuted=rr.cview(xa.data_ptr()), expert_weights=rr.cview(wa.data_ptr()),
        offsets=naive.offsets.data_ptr(), y_permuted=rr.mview(sabs.data_ptr()), experts=e, hidden=k,
        output=n, max_expert_tokens=r, kernel=rr.kernel(rr.KernelFamily.kNaive)), ctx).ok()
    torch.cuda.synchronize()
    del xa, wa
    gamma = k * U32 / (1 - k * U32)
    worst = 0.0
    for lo in range(0, r, 8192):
        pf, pn = pos_f[lo:lo + 8192], pos_n[lo:lo + 8192]
        diff = (fused.yp[pf].double() - naive.yp[pn].double()).abs()
        allowed = 3 * gamma * sabs[pn].double() / (1 - gamma) + 1e-7
        bad = int((diff > allowed).sum())
        assert bad == 0, f"y_permuted routes [{lo}, {lo + 8192}): {bad} elements outside the GEMM bound"
        worst = max(worst, (diff / allowed).max().item())
        # x_permuted: every route's row is x[route // 2], bitwise
        src = torch.arange(lo, min(r, lo + 8192), device=device) // 2
        assert torch.equal(fused.xp[pf].view(torch.int32), fused.x[src].view(torch.int32)), \
            f"x_permuted rows of routes [{lo}, {lo + 8192}) differ from x"
    report["y_permuted_worst_fraction_of_bound"] = worst
    print(f"C5: {report}")


def test_chain_from_logits_route_trace(ctx, device, kat):
    """chain_from_logits driven by the reference route-trace fixture: logits
    -8 everywhere, +2 / +1 at the desired ids (reference chain_adapter.cpp:209-230)."""
    raw = kat.raw["route_trace_fixture"]
    t, e = raw["tokens"], raw["experts"]
    for frame, desired in raw["frames"].items():
        desired = np.array(desired, np.int32).reshape(t, 2)
        logits = np.full((t, e), -8.0, np.float32)
        logits[np.arange(t), desired[:, 0]] = 2.0
        logits[np.arange(t), desired[:, 1]] = 1.0
        cfg = workloads.ChainConfig("trace", t, e, 16, 8, from_tokens=False)
        inp = workloads.chain_inputs(cfg, seed=1)
        inp["logits"] = logits
        dev = ChainRun(cfg, inp, device).run(ctx)
        assert np.array_equal(dev["ids"], desired), frame
        check_chain(cfg, inp, dev)


def run_stages(cfg, inp, device, ctx):
    """The seven public operators one by one (native kernels), as the
    reference chain_adapter enqueues them."""
    t, e, k, n = cfg.tokens, cfg.experts, cfg.hidden, cfg.output
    native = rr.kernel(rr.KernelFamily.kOptimized, rr.GFX950_NATIVE)
    dev = lambda a: a if isinstance(a, torch.Tensor) else to_dev(a, device)  # noqa: E731
    x, we = dev(inp["x"]), dev(inp["expert_weights"])
    i32 = dict(dtype=torch.int32, device=device)
    logits = torch.empty(t, e, device=device) if cfg.from_tokens else dev(inp["logits"])
    ids, w = torch.empty(t, 2, **i32), torch.empty(t, 2, device=device)
    counts, offsets = torch.empty(e, **i32), torch.empty(e + 1, **i32)
    xp, pos, inv = torch.empty(2 * t, k, device=device), torch.empty(2 * t, **i32), torch.empty(2 * t, **i32)
    yp, y, cursors = torch.empty(2 * t, n, device=device), torch.empty(t, n, device=device), torch.empty(e, **i32)

    def ok(status):
        assert status.ok(), status.message
    if cfg.from_tokens:
        wr = dev(inp["router_weights"])
        ok(rr.dense_gemm(rr.DenseGemmArgs(a=rr.cview(x.data_ptr()), b=rr.cview(wr.data_ptr()),
                                          c=rr.mview(logits.data_ptr()), m=t, n=e, k=k, kernel=native), ctx))
    ok(rr.topk_gate(rr.TopKGateArgs(logits=rr.cview(logits.data_ptr()), expert_ids=ids.data_ptr(),
                                    weights=rr.mview(w.data_ptr()), tokens=t, experts=e, kernel=native), ctx))
    ok(rr.histogram_exclusive_scan(rr.HistogramExclusiveScanArgs(
        expert_ids=ids.data_ptr(), counts=counts.data_ptr(), offsets=offsets.data_ptr(), route_pairs=2 * t,
        experts=e, kernel=native), ctx))
    pctx = rr.RuntimeContext(stream=ctx.stream, workspace=cursors.data_ptr(), workspace_bytes=4 * e,
                             architecture=ctx.architecture)
    ok(rr.token_permute(rr.TokenPermuteArgs(
        x=rr.cview(x.data_ptr()), expert_ids=ids.data_ptr(), offsets=offsets.data_ptr(),
        x_permuted=rr.mview(xp.data_ptr()), route_pos=pos.data_ptr(), sorted_route=inv.data_ptr(), tokens=t,
        experts=e, top_k=2, hidden=k, kernel=native), pctx))
    ok(rr.grouped_gemm(rr.GroupedGemmArgs(
        x_permuted=rr.cview(xp.data_ptr()), expert_weights=rr.cview(we.data_ptr()), offsets=offsets.data_ptr(),
        y_permuted=rr.mview(yp.data_ptr()), experts=e, hidden=k, output=n, max_expert_tokens=2 * t,
        kernel=native), ctx))
    ok(rr.unpermute(rr.UnpermuteArgs(
        y_permuted=rr.cview(yp.data_ptr()), route_pos=pos.data_ptr(), route_weights=rr.cview(w.data_ptr()),
        y=rr.mview(y.data_ptr()), tokens=t, top_k=2, output=n, kernel=native), ctx))
    torch.cuda.synchronize()
    return {"logits": to_host(logits), "ids": to_host(ids), "weights": to_host(w), "counts": to_host(counts),
            "offsets": to_host(offsets), "route_pos": to_host(pos), "sorted_route": to_host(inv),
            "x_permuted": to_host(xp), "y_permuted": to_host(yp), "y": to_host(y), "cursors": to_host(cursors)}


@pytest.mark.parametrize("shape", [
    ("tokens", 5, 4, 7, 5), ("tokens", 512, 32, 256, 64), ("tokens", 4096, 64, 256, 128),
    ("tokens", 1000, 128, 96, 40), ("tokens", 777, 256, 64, 33), ("tokens", 300, 1024, 20, 12),
    ("logits", 4096, 64, 256, 128), ("logits", 333, 7, 13, 9), ("tokens", 50, 8, 16, 0),
    # K tails of the strip kernel's register B: 16 chunks with masked rows
    # (B issued after the route map), 14 chunks (before it)
    ("tokens", 700, 64, 252, 128), ("logits", 900, 32, 224, 96),
    # K = 256 with two-strip segments: workgroup ranges span up to three
    # segments (a later segment's B loaded ahead, the middle one on the switch)
    ("tokens", 4096, 256, 256, 128), ("tokens", 2048, 256, 256, 64),
    # the merged launch's route limit (16384 routes held in registers): 16
    # id chunks per wave with four waves (N <= 64), 8 with eight
    ("tokens", 8192, 64, 256, 64), ("logits", 8192, 64, 128, 128),
])
@pytest.mark.parametrize("with_inverse", [True, False])
def test_fused_chain_matches_stage_by_stage(ctx, device, shape, with_inverse):
    """The fused chain (three launches) writes every output of the seven stages
    bit-identically to the operators run one by one."""
    kind, t, e, k, n = shape
    cfg = workloads.ChainConfig("fused", t, e, k, n, from_tokens=kind == "tokens")
    inp = workloads.chain_inputs(cfg, seed=3)
    run = ChainRun(cfg, inp, device, with_inverse=with_inverse)
    fused = run.run(ctx)
    fused["cursors"] = to_host(run.ws[:e])
    ref = run_stages(cfg, inp, device, ctx)
    for key in ("logits", "ids", "weights", "counts", "offsets", "route_pos", "x_permuted", "y_permuted",
                "y", "cursors") + (("sorted_route",) if with_inverse else ()):
        a, b = fused[key], ref[key]
        assert a.shape == b.shape, key
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b), f"{key} differs"
    check_chain(cfg, inp, fused)


@pytest.mark.parametrize("distribution,tokens,experts,hidden,output", [
    ("single_hot", 4096, 64, 256, 128), ("single_hot", 4096, 64, 256, 64), ("single_hot", 777, 16, 128, 96),
    ("zipf", 4096, 64, 256, 128), ("round_robin", 4096, 64, 256, 128), ("duplicate_free_hot", 8192, 64, 256, 64),
])
def test_fused_chain_skewed_routing_matches_stage_by_stage(ctx, device, distribution, tokens, experts, hidden,
                                                           output):
    """chain_from_logits with logits that select skewed routings (every token
    on experts 0 and 1; Zipf; round robin; one expert in every token): the
    merged launch's dominant-expert counting gives the same counts, offsets,
    route map and outputs, bit for bit, as the operators run one by one."""
    t, e = tokens, experts
    if distribution == "duplicate_free_hot":
        rng = np.random.default_rng(5)
        ids = np.stack([np.full(t, 3), (3 + 1 + rng.integers(0, e - 1, t)) % e], axis=1).astype(np.int32)
    else:
        ids = workloads.topk_route_ids(t, 2, e, distribution, seed=2)
    logits = np.full((t, e), -8.0, np.float32)
    logits[np.arange(t), ids[:, 0]] = 2.0
    logits[np.arange(t), ids[:, 1]] = 1.0
    cfg = workloads.ChainConfig("skew", t, e, hidden, output, from_tokens=False)
    inp = workloads.chain_inputs(cfg, seed=4)
    inp["logits"] = logits
    run = ChainRun(cfg, inp, device)
    fused = run.run(ctx)
    fused["cursors"] = to_host(run.ws[:e])
    assert np.array_equal(fused["ids"], ids)
    ref = run_stages(cfg, inp, device, ctx)
    for key in ("ids", "weights", "counts", "offsets", "route_pos", "sorted_route", "x_permuted", "y_permuted",
                "y", "cursors"):
        a, b = fused[key], ref[key]
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b), f"{key} differs"
    check_chain(cfg, inp, fused)


@pytest.mark.parametrize("kind,hidden", [("tokens", 48), ("logits", 48), ("tokens", 260), ("logits", 260)])
def test_fused_launches_one_by_one_equal_chain(ctx, device, kind, hidden):
    """rr_chain_fused_launch over every launch in order writes what one chain
    call writes (merged route prep for K <= 256, separate above); an index past
    the last launch is rejected."""
    cfg = workloads.ChainConfig("hook", 300, 16, hidden, 40, from_tokens=kind == "tokens")
    inp = workloads.chain_inputs(cfg, seed=11)
    whole = ChainRun(cfg, inp, device).run(ctx)
    run = ChainRun(cfg, inp, device)
    c = rr.RuntimeContext(stream=ctx.stream, workspace=run.ws.data_ptr(),
                          workspace_bytes=run.ws.numel() * 4, architecture=ctx.architecture)
    names = rr.chain_fused_launch_names(run.args, cfg.from_tokens)
    assert names[0] == ("router_gate" if kind == "tokens" else "gate") and len(names) in (2, 3)
    for index in range(len(names)):
        status = rr.chain_fused_launch(run.args, c, cfg.from_tokens, index)
        assert status.ok(), status.message
    torch.cuda.synchronize()
    status = rr.chain_fused_launch(run.args, c, cfg.from_tokens, len(names))
    assert status.code == rr.StatusCode.kInvalidArgument
    parts = {name: to_host(getattr(run, attr)) for name, attr in
             [("logits", "logits"), ("ids", "ids"), ("weights", "w"), ("counts", "counts"),
              ("offsets", "offsets"), ("route_pos", "pos"), ("y", "y"), ("x_permuted", "xp"),
              ("y_permuted", "yp"), ("sorted_route", "inv")]}
    for key, a in parts.items():
        b = whole[key]
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b), f"{key} differs"


@pytest.mark.parametrize("experts", [64, 128])
def test_fused_router_gate_special_values(ctx, device, experts):
    """Token rows that make NaN, +-Inf and all-equal logits go through the
    router's fused gate epilogue (16 or 32 lanes per row): ids and weights
    match the dense GEMM + top-2 gate operators bit for bit and the oracle
    top-2 of the device logits (NaN ranks as -Inf; equal values -> {0.5, 0.5};
    +Inf first -> {1, 0})."""
    cfg = workloads.ChainConfig("special", 96, experts, 64, 32, from_tokens=True)
    inp = workloads.chain_inputs(cfg, seed=5)
    x = inp["x"].copy()
    x[0, :] = np.nan               # every logit NaN -> ids {0, 1}, weights {0.5, 0.5}
    x[1, :] = 0.0                  # every logit 0 -> ids {0, 1}, weights {0.5, 0.5}
    x[2, :] = 0.0
    x[2, 5] = np.inf               # +-Inf or NaN logits, by the sign of router row 5
    x[3, 7] = -np.inf
    x[4, :] = 1e30                 # logits overflow to +-Inf
    inp["x"] = x
    run = ChainRun(cfg, inp, device)
    fused = run.run(ctx)
    ref = run_stages(cfg, inp, device, ctx)
    for key in ("logits", "ids", "weights"):
        a, b = fused[key], ref[key]
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b), key
    ids, w = oracle.top2_f32(fused["logits"])
    assert np.array_equal(fused["ids"], ids)
    fails, max_abs, _ = oracle.compare_floating(fused["weights"], w, 1e-6, 1e-6)  # device vs host expf
    assert fails == 0, max_abs
    assert fused["ids"][0].tolist() == [0, 1] and fused["weights"][0].tolist() == [0.5, 0.5]
    assert fused["ids"][1].tolist() == [0, 1] and fused["weights"][1].tolist() == [0.5, 0.5]


@pytest.mark.parametrize("experts", list(range(4, 129, 4)))
def test_router_gate_sweep(ctx, device, experts):
    """The chain's router launch (GEMM + fused top-2) for every E the strip
    router takes (E % 4 == 0, E <= 128; 16 lanes per row up to E = 64, 32
    above) at T = 65 (a ragged last strip) with exact ties in the router
    weights: ids are the oracle top-2 of the device logits, weights within the
    reference's 1e-6."""
    cfg = workloads.ChainConfig("router", 65, experts, 32, 8, from_tokens=True)
    inp = workloads.chain_inputs(cfg, seed=experts)
    wr = inp["router_weights"].copy()
    wr[:, experts // 2] = wr[:, 0]  # identical columns -> exactly tied logits
    inp["router_weights"] = wr
    run = ChainRun(cfg, inp, device)
    c = rr.RuntimeContext(stream=ctx.stream, workspace=run.ws.data_ptr(),
                          workspace_bytes=run.ws.numel() * 4, architecture=ctx.architecture)
    assert rr.chain_fused_launch_names(run.args, True)[0] == "router_gate"
    status = rr.chain_fused_launch(run.args, c, True, 0)
    assert status.ok(), status.message
    logits, ids, w = to_host(run.logits), to_host(run.ids), to_host(run.w)
    e_ids, e_w = oracle.top2_f32(logits)
    assert np.array_equal(ids, e_ids)
    fails, max_abs, _ = oracle.compare_floating(w, e_w, 1e-6, 1e-6)
    assert fails == 0, max_abs


@pytest.mark.parametrize("shape", [(512, 16, 64, 64), (700, 32, 300, 40)])
def test_fused_combine_subnormal_products(ctx, device, shape):
    """The fused combine adds w * y_permuted into y with hardware FP32 atomics;
    the stage-by-stage unpermute sums with plain FP32 operations. With
    y_permuted entries just above the smallest normal (2^-126 (1 + u)) and
    weights below one, most products w * y_permuted are subnormal: the fused
    y must still equal the staged y and the host's IEEE FP32 rank-order sum
    bit for bit (subnormals kept, not flushed). Merged strip launch (K <= 256)
    and the tiled GEMM's combine (K > 256)."""
    t, e, k, n = shape
    cfg = workloads.ChainConfig("subnormal", t, e, k, n, from_tokens=False)
    inp = workloads.chain_inputs(cfg, seed=29)
    x = np.zeros((t, k), np.float32)
    x[np.arange(t), np.arange(t) % k] = np.float32(2.0 ** -63)  # one non-zero per row
    u = workloads.unit_doubles(e * k * n, 29, workloads.S_EXPERTS).reshape(e, k, n)
    we = (np.float32(2.0 ** -63) * (1.0 + u)).astype(np.float32)  # products x * W are normal
    inp = dict(inp, x=x, expert_weights=we)
    print(f"fused combine subnormal products {shape}", flush=True)
    fused = ChainRun(cfg, inp, device).run(ctx)
    ref = run_stages(cfg, inp, device, ctx)
    yp, w, pos = fused["y_permuted"], fused["weights"], fused["route_pos"].reshape(t, 2)
    prods = w[:, :, None] * yp[pos]
    tiny = np.finfo(np.float32).tiny
    assert ((prods != 0) & (np.abs(prods) < tiny)).mean() > 0.5, "products are not mostly subnormal"
    want = (np.float32(0) + prods[:, 0]) + prods[:, 1]
    assert np.array_equal(ref["y"].view(np.uint32), want.view(np.uint32)), "staged unpermute flushed subnormals"
    assert np.array_equal(fused["y"].view(np.uint32), ref["y"].view(np.uint32)), \
        "fused combine differs from the staged unpermute on subnormal products"


@pytest.mark.parametrize("experts,output", [(64, 128), (128, 96)])
def test_chain_router_four_strips_per_workgroup(ctx, device, experts, output):
    """T=16384 with K=256: the router launch gives every workgroup four 16-token
    strips, so both A buffers and the logit tile are reused (strip s takes
    the buffer of strip s - 2); ids, weights and the route map in full, the
    output on a seeded sample of 256 tokens."""
    cfg = workloads.ChainConfig("router4", 16384, experts, 256, output, from_tokens=True)
    inp_dev = workloads.chain_inputs_device(cfg, 0, device)
    dev = ChainRun(cfg, inp_dev, device).run(ctx)
    inp = {key: to_host(v) for key, v in inp_dev.items()}
    sample = np.sort(workloads.seeded_permutation(cfg.tokens, 0, 78)[:256])
    report = check_chain(cfg, inp, dev, sample_tokens=sample)
    print(f"router four strips: {report}")
