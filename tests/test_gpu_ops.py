"""Per-operator parity of the gfx950 library against the CPU oracle, through
the C ABI. Structure follows the reference's operator tests
(reference tests/operator_api_tests.cpp, tests/correctness_tests.cpp):
known-answer vectors, redzone-guarded buffers, edge shapes, then seeded random
cases checked bit-exactly (ids, counts, offsets, route maps, copied rows) or
within the accumulation-aware GEMM bound / stated tolerance (floats).
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

F = rr.KernelFamily
NATIVE = rr.kernel(F.kOptimized, rr.GFX950_NATIVE)
NAIVE = rr.kernel(F.kNaive, 0)
AUTO = rr.kernel()
# Weight tolerance of the reference chain and top-k adapters
# (reference benchmarks/adapters/chain_adapter.cpp:483-486, topk_gate_adapter.cpp:157).
W_ATOL = W_RTOL = 1e-6


def ok(status):
    assert status.ok(), f"{rr.StatusCode(status.code).name}: {status.message}"


def p(t):
    return t.data_ptr()


def gemm_ok(actual, a, b):
    """Accumulation-aware bound of reference src/correctness/reference_validation.cpp:78-100."""
    expect = oracle.dense_gemm_f64(a, b)
    fails, max_abs, ratio = oracle.compare_gemm(actual.astype(np.float64), expect, a, b)
    assert fails == 0, f"{fails} elements exceed the GEMM bound (max |err| {max_abs}, ratio {ratio})"
    return ratio


# ------------------------------------------------------------------ dense GEMM

@pytest.mark.parametrize("kernel", [AUTO, NAIVE, NATIVE] + [rr.kernel(F.kOptimized, i) for i in range(1, 8)])
def test_dense_gemm_kat(ctx, guarded, kat, kernel):
    a = guarded(4, np.float32, kat("dense_gemm_2x2", "a"))
    b = guarded(4, np.float32, kat("dense_gemm_2x2", "b"))
    c = guarded(4, np.float32)
    args = rr.DenseGemmArgs(a=rr.cview(a.ptr), b=rr.cview(b.ptr), c=rr.mview(c.ptr), m=2, n=2, k=2,
                            kernel=kernel)
    ok(rr.dense_gemm(args, ctx))
    assert c.read().tolist() == [19.0, 22.0, 43.0, 50.0]
    # K = 0 writes mathematical zeros without reading A or B
    args.a = rr.cview(None); args.b = rr.cview(None); args.k = 0
    ok(rr.dense_gemm(args, ctx))
    assert c.read().tolist() == [0.0] * 4
    assert a.canaries_intact() and b.canaries_intact() and c.canaries_intact()


@pytest.mark.parametrize("m,n,k,offset", [
    (17, 19, 13, 1),       # reference tests/operator_api_tests.cpp:575-624 (unaligned fallback)
    (512, 32, 256, 0),     # C1 router
    (4096, 64, 256, 0),    # headline router
    (300, 64, 255, 0),     # K tail
    (1000, 128, 2048, 0),  # C5-shaped slice
    (129, 72, 96, 1),
    (16384, 64, 256, 0),   # strip kernel: four 16-row strips per workgroup (A stage reused)
    (16500, 128, 192, 0),  # ... and a ragged last strip
])
@pytest.mark.parametrize("kernel", [NATIVE, NAIVE])
def test_dense_gemm_random(ctx, guarded, m, n, k, offset, kernel):
    rng = np.random.default_rng(m * 7 + n)
    a_h = rng.standard_normal((m, k)).astype(np.float32)
    b_h = (rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    a = guarded(m * k, np.float32, a_h, offset_elems=offset)
    b = guarded(k * n, np.float32, b_h, offset_elems=offset)
    c = guarded(m * n, np.float32, offset_elems=offset)
    ok(rr.dense_gemm(rr.DenseGemmArgs(a=rr.cview(a.ptr), b=rr.cview(b.ptr), c=rr.mview(c.ptr),
                                      m=m, n=n, k=k, kernel=kernel), ctx))
    out = c.read().reshape(m, n)
    gemm_ok(out, a_h, b_h)
    if kernel.family == F.kNaive:
        # naive = sequential k with separately rounded mul/add: bit-exact vs the FP32 oracle
        assert np.array_equal(out, oracle.dense_gemm_f32_seq(a_h, b_h))
    assert a.canaries_intact() and b.canaries_intact() and c.canaries_intact()


# ------------------------------------------------------------------ top-2 gate

def run_gate(ctx, logits_h, kernel, device, offset=0):
    t, e = logits_h.shape
    buf = torch.empty(t * e + offset, dtype=torch.float32, device=device)
    buf[offset:] = torch.from_numpy(logits_h.reshape(-1)).to(device)
    ids = torch.full((t, 2), -7, dtype=torch.int32, device=device)
    w = torch.full((t, 2), -7.0, dtype=torch.float32, device=device)
    args = rr.TopKGateArgs(logits=rr.cview(p(buf) + 4 * offset), expert_ids=p(ids), weights=rr.mview(p(w)),
                           tokens=t, experts=e, kernel=kernel)
    ok(rr.topk_gate(args, ctx))
    return to_host(ids), to_host(w)


@pytest.mark.parametrize("kernel", [AUTO, NAIVE, NATIVE] + [rr.kernel(F.kOptimized, i) for i in range(1, 5)])
def test_topk_gate_kat(ctx, device, kat, kernel):
    logits = np.array(kat("topk_gate_3x4", "logits"), np.float32)
    ids, w = run_gate(ctx, logits, kernel, device)
    assert ids.tolist() == kat("topk_gate_3x4", "ids")
    assert w.tolist() == kat("topk_gate_3x4", "weights")


def check_gate(ids, w, logits):
    e_ids, e_w = oracle.top2_f32(logits)
    assert np.array_equal(ids, e_ids), "top-2 ids differ from the oracle"
    fails, max_abs, _ = oracle.compare_floating(w, e_w, W_ATOL, W_RTOL)
    assert fails == 0, f"weights: max |err| {max_abs}"


def _gate_sweep_case(ctx, device, experts, tokens):
    rng = np.random.default_rng(experts * 1000 + tokens)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    logits[rng.random((tokens, experts)) < 0.1] = 0.5  # exact ties
    for kernel in (NATIVE, NAIVE):
        for offset in (0, 1):
            ids, w = run_gate(ctx, logits, kernel, device, offset)
            check_gate(ids, w, logits)


@pytest.mark.parametrize("experts", list(range(2, 65)) + [65, 128, 256, 257, 1024])
def test_topk_gate_sweep(ctx, device, experts):
    # exhaustive E = 2..64 x T in {1, 7, 65}, like reference tests/correctness_tests.cpp:609-628
    for tokens in (1, 7, 65):
        _gate_sweep_case(ctx, device, experts, tokens)


@pytest.mark.parametrize("experts", [2, 3, 5, 16, 33, 64, 128, 1024])
def test_topk_gate_sweep_many_rows(ctx, device, experts):
    _gate_sweep_case(ctx, device, experts, 4096)


@pytest.mark.parametrize("mode", ["ties", "all_nan", "duplicate_max", "signed_zero", "mixed_nan_neg_inf",
                                  "single_infinity", "multiple_infinity", "extreme"])
@pytest.mark.parametrize("experts", [2, 4, 8, 33, 64, 128, 1024])
def test_topk_gate_special_inputs(ctx, device, mode, experts):
    from test_oracle import special_rows
    rng = np.random.default_rng(3)
    logits = np.stack([special_rows(mode, experts, rng) for _ in range(70)])
    for kernel in (NATIVE, NAIVE):
        ids, w = run_gate(ctx, logits, kernel, device)
        check_gate(ids, w, logits)


def test_topk_gate_c2_ties(ctx, device):
    inp = workloads.chain_inputs(workloads.C2, seed=0)
    ids, w = run_gate(ctx, inp["logits"], NATIVE, device)
    check_gate(ids, w, inp["logits"])
    rows = inp["tie_rows"]
    assert rows.size > 0
    # at tie rows the lower of the two tied experts is second
    lg = inp["logits"][rows]
    order = np.argsort(-lg, axis=1, kind="stable")
    assert np.array_equal(ids[rows, 1], np.minimum(order[:, 1], order[:, 2]))


# ------------------------------------------------------- histogram and scans

@pytest.mark.parametrize("kernel", [AUTO, NAIVE, NATIVE, rr.kernel(F.kOptimized, 101)])
def test_histogram_reset(ctx, guarded, kat, kernel):
    # reference tests/operator_api_tests.cpp:662-731
    ids = guarded(4, np.int32, [0, 1, 1, 1])
    counts = guarded(2, np.int32, [99, 99])
    args = rr.HistogramArgs(expert_ids=ids.ptr, counts=counts.ptr, route_pairs=4, experts=2, kernel=kernel)
    ok(rr.histogram(args, ctx))
    assert counts.read().tolist() == [1, 3]
    counts.write([77, 88])
    args.expert_ids = None; args.route_pairs = 0
    ok(rr.histogram(args, ctx))
    assert counts.read().tolist() == [0, 0]
    assert ids.read().tolist() == [0, 1, 1, 1]
    assert ids.canaries_intact() and counts.canaries_intact()
    for routes in (8192, 32768):
        h = (np.arange(routes) & 1).astype(np.int32)
        big = guarded(routes, np.int32, h)
        c2 = guarded(2, np.int32, [9, 9])
        ok(rr.histogram(rr.HistogramArgs(expert_ids=big.ptr, counts=c2.ptr, route_pairs=routes,
                                         experts=2, kernel=kernel), ctx))
        assert c2.read().tolist() == [routes // 2, routes // 2]
        assert big.canaries_intact() and c2.canaries_intact()


@pytest.mark.parametrize("experts", [1, 31, 32, 33, 63, 64, 256, 1024])
@pytest.mark.parametrize("kernel", [AUTO, NAIVE, NATIVE])
def test_exclusive_scan(ctx, guarded, experts, kernel):
    # reference tests/operator_api_tests.cpp:317-412
    counts_h = (np.arange(experts) % 5).astype(np.int32)
    expect = np.concatenate([[0], np.cumsum(counts_h)]).astype(np.int32)
    counts = guarded(experts, np.int32, counts_h)
    offsets = guarded(experts + 1, np.int32)
    ok(rr.exclusive_scan(rr.ExclusiveScanArgs(counts=counts.ptr, offsets=offsets.ptr, experts=experts,
                                              kernel=kernel), ctx))
    assert np.array_equal(offsets.read(), expect)
    # in place: counts and offsets share storage
    inplace = guarded(experts + 1, np.int32, np.concatenate([counts_h, [-1]]))
    ok(rr.exclusive_scan(rr.ExclusiveScanArgs(counts=inplace.ptr, offsets=inplace.ptr, experts=experts,
                                              kernel=kernel), ctx))
    assert np.array_equal(inplace.read(), expect)
    assert counts.canaries_intact() and offsets.canaries_intact() and inplace.canaries_intact()


@pytest.mark.parametrize("kernel", [NAIVE, NATIVE])
def test_exclusive_scan_edges(ctx, guarded, kernel):
    # 4-byte (not 8-byte) aligned pointers, reference tests/operator_api_tests.cpp:364-393
    e = 33
    counts_h = (np.arange(e) % 7).astype(np.int32)
    counts = guarded(e, np.int32, counts_h, offset_elems=1)
    offsets = guarded(e + 1, np.int32, offset_elems=1)
    assert counts.ptr % 8 == 4 and offsets.ptr % 8 == 4
    ok(rr.exclusive_scan(rr.ExclusiveScanArgs(counts=counts.ptr, offsets=offsets.ptr, experts=e, kernel=kernel), ctx))
    assert np.array_equal(offsets.read(), np.concatenate([[0], np.cumsum(counts_h)]))
    assert counts.canaries_intact() and offsets.canaries_intact()
    # INT32_MAX in place, reference tests/operator_api_tests.cpp:395-412
    h = np.zeros(65, np.int32); h[0] = 2**31 - 1; h[64] = -1
    buf = guarded(65, np.int32, h)
    ok(rr.exclusive_scan(rr.ExclusiveScanArgs(counts=buf.ptr, offsets=buf.ptr, experts=64, kernel=kernel), ctx))
    assert buf.read().tolist() == [0] + [2**31 - 1] * 64


def run_fused(ctx, guarded, ids_h, experts, kernel):
    r = ids_h.size
    ids = guarded(max(r, 1), np.int32, ids_h if r else [0])
    counts = guarded(experts, np.int32, np.full(experts, 123, np.int32))
    offsets = guarded(experts + 1, np.int32, np.full(experts + 1, 456, np.int32))
    args = rr.HistogramExclusiveScanArgs(expert_ids=ids.ptr if r else None, counts=counts.ptr,
                                         offsets=offsets.ptr, route_pairs=r, experts=experts, kernel=kernel)
    assert rr.get_histogram_exclusive_scan_workspace_size(args) == 0
    ok(rr.histogram_exclusive_scan(args, ctx))
    c, o = counts.read(), offsets.read()
    assert counts.canaries_intact() and offsets.canaries_intact() and ids.canaries_intact()
    return c, o


@pytest.mark.parametrize("routes,experts", [(0, 1), (1, 8), (257, 33), (4096, 64), (4097, 64),
                                            (65536, 1024), (65537, 7)])
@pytest.mark.parametrize("kernel", [AUTO, NAIVE, NATIVE, rr.kernel(F.kOptimized, 2)])
def test_histogram_exclusive_scan_round_robin(ctx, guarded, routes, experts, kernel):
    ids = (np.arange(routes) % experts).astype(np.int32)
    c, o = run_fused(ctx, guarded, ids, experts, kernel)
    e_c = oracle.histogram(ids, experts)
    assert np.array_equal(c, e_c) and np.array_equal(o, oracle.exclusive_scan(e_c))


@pytest.mark.parametrize("experts", [1, 33, 256])
@pytest.mark.parametrize("dist", ["uniform", "hot50"])
@pytest.mark.parametrize("routes", [8192, 32768, 1 << 20])
def test_histogram_scan_c3(ctx, guarded, experts, dist, routes):
    # C3 stress: R up to 1,048,576 at E in {1, 33, 256}
    ids = workloads.route_ids(routes, experts, dist, seed=0)
    e_c = oracle.histogram(ids, experts)
    e_o = oracle.exclusive_scan(e_c)
    for kernel in (NATIVE, NAIVE):
        c, o = run_fused(ctx, guarded, ids, experts, kernel)
        assert np.array_equal(c, e_c) and np.array_equal(o, e_o)
        cnt = guarded(experts, np.int32, np.full(experts, 5, np.int32))
        idb = guarded(routes, np.int32, ids)
        ok(rr.histogram(rr.HistogramArgs(expert_ids=idb.ptr, counts=cnt.ptr, route_pairs=routes,
                                         experts=experts, kernel=kernel), ctx))
        assert np.array_equal(cnt.read(), e_c)


@pytest.mark.parametrize("routes,experts,offset", [(65537, 7, 0), (200003, 1024, 0), (150001, 33, 1),
                                                   (1 << 20, 2, 0), (70000, 256, 3)])
def test_histogram_large_paths(ctx, guarded, routes, experts, offset):
    """Multi-block path (R > 65536): ragged end, unaligned ids (scalar loads),
    E = 1024 (several passes per block), out-of-range ids skipped, and two calls
    in a row on the same buffers (the last-block ticket starts from zero each
    call). Counts sit `offset` elements past an aligned base too."""
    rng = np.random.default_rng(routes + experts)
    ids_h = rng.integers(0, experts, routes).astype(np.int32)
    ids_h[rng.integers(0, routes, 50)] = -3
    ids_h[rng.integers(0, routes, 50)] = experts + 5
    valid = ids_h[(ids_h >= 0) & (ids_h < experts)]
    e_c = np.bincount(valid, minlength=experts).astype(np.int32)
    e_o = np.concatenate([[0], np.cumsum(e_c)]).astype(np.int32)
    ids = guarded(routes, np.int32, ids_h, offset_elems=offset)
    for _ in range(2):
        counts = guarded(experts, np.int32, np.full(experts, 123, np.int32), offset_elems=offset)
        offsets = guarded(experts + 1, np.int32, np.full(experts + 1, 456, np.int32))
        ok(rr.histogram_exclusive_scan(rr.HistogramExclusiveScanArgs(
            expert_ids=ids.ptr, counts=counts.ptr, offsets=offsets.ptr, route_pairs=routes,
            experts=experts, kernel=NATIVE), ctx))
        assert np.array_equal(counts.read(), e_c) and np.array_equal(offsets.read(), e_o)
        ok(rr.histogram(rr.HistogramArgs(expert_ids=ids.ptr, counts=counts.ptr, route_pairs=routes,
                                         experts=experts, kernel=NATIVE), ctx))
        assert np.array_equal(counts.read(), e_c)
        assert counts.canaries_intact() and offsets.canaries_intact() and ids.canaries_intact()


@pytest.mark.parametrize("experts,share,offset", [(33, 0.15, 0), (33, 0.5, 1), (1024, 0.95, 0), (256, 0.3, 2),
                                                  (3, 0.2, 0)])
def test_histogram_large_hot_expert(ctx, guarded, experts, share, offset):
    """Multi-block path with a dominant expert at several shares (waves that
    see it among their first ids count it with ballots instead of LDS
    atomics; the rest count it by atomics), out-of-range ids in the mix, and
    two calls in a row; counts and offsets exact, canaries intact."""
    routes = 300007
    rng = np.random.default_rng(experts + int(share * 100))
    ids_h = rng.integers(0, experts, routes).astype(np.int32)
    hot = int(rng.integers(0, experts))
    ids_h[rng.random(routes) < share] = hot
    ids_h[rng.integers(0, routes, 40)] = -1
    ids_h[rng.integers(0, routes, 40)] = experts
    valid = ids_h[(ids_h >= 0) & (ids_h < experts)]
    e_c = np.bincount(valid, minlength=experts).astype(np.int32)
    e_o = np.concatenate([[0], np.cumsum(e_c)]).astype(np.int32)
    ids = guarded(routes, np.int32, ids_h, offset_elems=offset)
    for _ in range(2):
        counts = guarded(experts, np.int32, np.full(experts, 77, np.int32), offset_elems=offset)
        offsets = guarded(experts + 1, np.int32, np.full(experts + 1, -9, np.int32))
        ok(rr.histogram_exclusive_scan(rr.HistogramExclusiveScanArgs(
            expert_ids=ids.ptr, counts=counts.ptr, offsets=offsets.ptr, route_pairs=routes,
            experts=experts, kernel=NATIVE), ctx))
        assert np.array_equal(counts.read(), e_c) and np.array_equal(offsets.read(), e_o)
        ok(rr.histogram(rr.HistogramArgs(expert_ids=ids.ptr, counts=counts.ptr, route_pairs=routes,
                                         experts=experts, kernel=NATIVE), ctx))
        assert np.array_equal(counts.read(), e_c)
        assert counts.canaries_intact() and offsets.canaries_intact() and ids.canaries_intact()


def _hist_case(routes, experts, seed, device):
    rng = np.random.default_rng(seed)
    ids_h = rng.integers(0, experts, routes).astype(np.int32)
    ids_h[rng.random(routes) < 0.3] = int(rng.integers(0, experts))
    e_c = np.bincount(ids_h, minlength=experts).astype(np.int32)
    e_o = np.concatenate([[0], np.cumsum(e_c)]).astype(np.int32)
    ids = to_dev(ids_h, device)
    counts = torch.full((experts,), 77, dtype=torch.int32, device=device)
    offsets = torch.full((experts + 1,), -9, dtype=torch.int32, device=device)
    return ids, counts, offsets, e_c, e_o


def _hist_call(ids, counts, offsets, routes, experts, stream, fused=True):
    cx = rr.RuntimeContext(stream=stream, architecture=int(rr.DeviceArchitecture.kGfx950))
    if fused:
        ok(rr.histogram_exclusive_scan(rr.HistogramExclusiveScanArgs(
            expert_ids=p(ids), counts=p(counts), offsets=p(offsets), route_pairs=routes,
            experts=experts, kernel=NATIVE), cx))
    else:
        ok(rr.histogram(rr.HistogramArgs(expert_ids=p(ids), counts=p(counts), route_pairs=routes,
                                         experts=experts, kernel=NATIVE), cx))


def test_histogram_large_streams(device):
    """Large R on twenty streams, each with its own ids, enqueued without waits
    between them so the calls overlap; twice; both the fused and the
    counts-only operator (each call's counts and ticket live in its own
    buffers, so concurrent calls never share state)."""
    routes, experts = 200003, 33
    streams = [torch.cuda.Stream(device) for _ in range(20)]
    cases = [_hist_case(routes, experts, 100 + i, device) for i in range(len(streams))]
    torch.cuda.synchronize()
    for rnd in range(2):
        for (ids, counts, offsets, _, _), s in zip(cases, streams):
            counts.fill_(77)
            offsets.fill_(-9)
        torch.cuda.synchronize()
        for i, ((ids, counts, offsets, _, _), s) in enumerate(zip(cases, streams)):
            _hist_call(ids, counts, offsets, routes, experts, s.cuda_stream, fused=(i + rnd) % 3 != 0)
        torch.cuda.synchronize()
        for i, (ids, counts, offsets, e_c, e_o) in enumerate(cases):
            assert np.array_equal(to_host(counts), e_c), (rnd, i)
            if (i + rnd) % 3 != 0:
                assert np.array_equal(to_host(offsets), e_o), (rnd, i)


def test_histogram_large_graph_replays(device):
    """Large R captured in a graph (zeroing kernel and counting kernel, no
    memset node), replayed three times with eager calls of other ids on the
    same stream between the replays; every replay and every eager call exact."""
    routes, experts = 300007, 256
    ids, counts, offsets, e_c, e_o = _hist_case(routes, experts, 7, device)
    ids2, counts2, offsets2, e_c2, e_o2 = _hist_case(routes, experts, 8, device)
    stream = torch.cuda.Stream(device)
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        _hist_call(ids, counts, offsets, routes, experts, stream.cuda_stream)
    for _ in range(3):
        counts.fill_(77)
        offsets.fill_(-9)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_host(counts), e_c) and np.array_equal(to_host(offsets), e_o)
        _hist_call(ids2, counts2, offsets2, routes, experts, stream.cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(to_host(counts2), e_c2) and np.array_equal(to_host(offsets2), e_o2)
    del graph


# -------------------------------------------------------------------- permute

def run_permute(ctx, device, x_h, ids_h, experts, kernel, with_inverse=True, offset=0):
    tokens, hidden = x_h.shape
    top_k = ids_h.shape[1]
    routes = tokens * top_k
    offsets_h = oracle.exclusive_scan(oracle.histogram(ids_h, experts))
    xb = torch.empty(tokens * hidden + offset, dtype=torch.float32, device=device)
    xb[offset:] = to_dev(x_h.reshape(-1), device)
    xp = torch.full((routes * hidden + offset,), float("nan"), dtype=torch.float32, device=device)
    ids = to_dev(ids_h.reshape(-1).astype(np.int32), device)
    offs = to_dev(offsets_h, device)
    pos = torch.full((routes,), -5, dtype=torch.int32, device=device)
    inv = torch.full((routes,), -5, dtype=torch.int32, device=device) if with_inverse else None
    cursors = torch.full((experts,), 99, dtype=torch.int32, device=device)
    args = rr.TokenPermuteArgs(x=rr.cview(p(xb) + 4 * offset), expert_ids=p(ids), offsets=p(offs),
                               x_permuted=rr.mview(p(xp) + 4 * offset), route_pos=p(pos),
                               sorted_route=p(inv) if with_inverse else None, tokens=tokens,
                               experts=experts, top_k=top_k, hidden=hidden, kernel=kernel)
    assert rr.get_token_permute_workspace_size(args) == experts * 4
    pctx = rr.RuntimeContext(stream=ctx.stream, workspace=p(cursors), workspace_bytes=experts * 4,
                             architecture=ctx.architecture)
    ok(rr.token_permute(args, pctx))
    return (offsets_h, to_host(xp)[offset:].reshape(routes, hidden), to_host(pos),
            to_host(inv) if with_inverse else None, to_host(cursors))


@pytest.mark.parametrize("kernel", [AUTO, NAIVE, NATIVE] + [rr.kernel(F.kOptimized, i) for i in range(1, 11)])
def test_permute_workspace_reset(ctx, device, kat, kernel):
    g = lambda f: kat("permute_workspace_reset", f)  # noqa: E731
    x = np.array(g("x"), np.float32)
    ids = np.array(g("ids"), np.int32).reshape(2, 2)
    offsets, xp, pos, inv, cursors = run_permute(ctx, device, x, ids, 2, kernel)
    assert cursors.tolist() == g("final_cursors")
    assert oracle.validate_permute(x, ids, offsets, xp, pos, inv, 2) == []
    if kernel.family != F.kNaive:
        assert pos.tolist() == [0, 2, 1, 3]  # stable order


@pytest.mark.parametrize("kernel", [NAIVE, NATIVE])
def test_permute_unaligned_duplicate_ids(ctx, device, kat, kernel):
    g = lambda f: kat("permute_duplicate_ids_unaligned", f)  # noqa: E731
    x = np.array(g("x"), np.float32)
    ids = np.array(g("ids"), np.int32).reshape(2, 2)
    offsets, xp, pos, inv, _ = run_permute(ctx, device, x, ids, 2, kernel, offset=1)
    assert oracle.validate_permute(x, ids, offsets, xp, pos, inv, 2) == []


@pytest.mark.parametrize("tokens,experts,top_k,hidden", [
    (5, 4, 2, 7), (512, 32, 2, 256), (4096, 64, 2, 256), (1000, 8, 1, 33), (777, 16, 4, 64),
    (3000, 1024, 2, 12), (20000, 128, 2, 4), (300, 600, 8, 20), (64, 4, 2, 0),
    # token-owned row kernel (rows of 1024 floats or more): rows wider than one
    # pass of a wave (2048 floats) with a 3-float tail, more than 64 routes per
    # token (position lanes read in chunks of 64); item kernel with many routes
    (50, 8, 2, 2051), (20, 200, 100, 1500), (9, 16, 3, 1024), (40, 200, 130, 9), (17, 1024, 1024, 5),
    # wide rows, rank + copy in one launch: several tokens per block and wave,
    # top_k 4 with a 7-float tail; beyond 32768 routes the two-launch path
    (2500, 64, 2, 1100), (1500, 300, 4, 1031), (17000, 8, 2, 1024),
    # ... few experts (ballot recount) with block prefixes that end mid-quad
    (3001, 16, 3, 1030), (4100, 5, 1, 1024),
    # ... destination rows at every 16-byte phase across chunk boundaries
    # (a chunk is 2048 floats: the realigned quads take the next chunk's first)
    (700, 16, 2, 2049), (300, 8, 2, 4097), (257, 8, 2, 6143),
    # ... top-2 rows on 128-byte lines (the pipelined copy): a row shorter than
    # one chunk, a second chunk of 8 quads, several rows per wave
    (3000, 16, 2, 1024), (900, 8, 2, 2080), (5000, 64, 2, 1536),
    # ... realigned rows whose source fits one chunk while a destination's
    # phase needs a second (the chunk prefetched before the ranks is then not
    # the one the copy wants next)
    (300, 16, 2, 2041), (257, 8, 2, 2030),
])
def test_permute_stable_bit_exact(ctx, device, tokens, experts, top_k, hidden):
    rng = np.random.default_rng(tokens + experts)
    ids = np.stack([rng.permutation(experts)[:top_k] for _ in range(tokens)]).astype(np.int32)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    offsets, xp, pos, inv, cursors = run_permute(ctx, device, x, ids, experts, NATIVE)
    e_pos = oracle.stable_route_pos(ids, offsets)
    assert np.array_equal(pos, e_pos)
    assert np.array_equal(inv, oracle.inverse_route(e_pos))
    assert np.array_equal(xp.view(np.uint32), oracle.permute_rows(x, e_pos, top_k).view(np.uint32))
    assert np.array_equal(cursors, np.diff(offsets))
    # the naive (atomic) placement satisfies every reference invariant
    offsets, xp, pos, inv, cursors = run_permute(ctx, device, x, ids, experts, NAIVE)
    assert oracle.validate_permute(x, ids, offsets, xp, pos, inv, top_k) == []
    assert np.array_equal(cursors, np.diff(offsets))


@pytest.mark.parametrize("tokens,experts,top_k,hidden,offset", [
    # rows whose width is a multiple of 32 floats but whose base pointers sit
    # 4, 28 or 124 bytes past a 128-byte line: every row is copied through the
    # line-realigned path; with a tail, a 2-chunk row and top_k past 64
    (300, 16, 2, 1024, 1), (129, 8, 3, 2048, 7), (64, 4, 2, 1056, 31), (33, 100, 70, 1024, 5),
    (40, 8, 2, 4093, 3),
    # widths at the chunk-count boundaries of the realigned copy: 2049 floats
    # is the widest one-chunk row (its last quads written by the tail lanes),
    # 2050 takes two chunks, 4095 and 4097 two (the tail lanes again), 4098 three
    (50, 8, 2, 2049, 0), (50, 8, 2, 2050, 1), (37, 8, 2, 4095, 0), (30, 8, 2, 4097, 3),
    (20, 4, 3, 4098, 0),
])
def test_permute_stable_offset_rows(ctx, device, tokens, experts, top_k, hidden, offset):
    rng = np.random.default_rng(tokens + hidden + offset)
    ids = np.stack([rng.permutation(experts)[:top_k] for _ in range(tokens)]).astype(np.int32)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    offsets, xp, pos, inv, cursors = run_permute(ctx, device, x, ids, experts, NATIVE, offset=offset)
    e_pos = oracle.stable_route_pos(ids, offsets)
    assert np.array_equal(pos, e_pos)
    assert np.array_equal(inv, oracle.inverse_route(e_pos))
    assert np.array_equal(xp.view(np.uint32), oracle.permute_rows(x, e_pos, top_k).view(np.uint32))
    assert np.array_equal(cursors, np.diff(offsets))


@pytest.mark.parametrize("tokens,experts,hidden", [(600, 8, 1024), (600, 8, 1100), (90, 4, 4096)])
def test_permute_wide_rows_invalid_ids(ctx, device, tokens, experts, hidden):
    """Wide top-2 rows with a few route ids outside [0, E): those routes map to
    -1 and their rows are not copied (the wave holding such a route takes the
    general copy loop); every other route keeps its stable position. Offsets
    count the valid ids only. The expected map is computed here in numpy: the
    oracle rejects invalid ids, as the reference's does."""
    rng = np.random.default_rng(tokens + hidden)
    ids = np.stack([rng.permutation(experts)[:2] for _ in range(tokens)]).astype(np.int32).reshape(-1)
    bad = rng.choice(ids.size, 7, replace=False)
    ids[bad[:4]] = -1
    ids[bad[4:]] = experts
    valid = (ids >= 0) & (ids < experts)
    counts = np.bincount(ids[valid], minlength=experts).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    e_pos = np.full(ids.size, -1, np.int32)
    cursor = offsets[:-1].copy()
    for r in range(ids.size):
        if valid[r]:
            e_pos[r] = cursor[ids[r]]
            cursor[ids[r]] += 1
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    routes = 2 * tokens
    xd = to_dev(x, device)
    xp = torch.full((routes, hidden), float("nan"), dtype=torch.float32, device=device)
    ids_d = to_dev(ids, device)
    offs_d = to_dev(offsets, device)
    pos = torch.full((routes,), -5, dtype=torch.int32, device=device)
    cursors = torch.full((experts,), 99, dtype=torch.int32, device=device)
    args = rr.TokenPermuteArgs(x=rr.cview(p(xd)), expert_ids=p(ids_d), offsets=p(offs_d),
                               x_permuted=rr.mview(p(xp)), route_pos=p(pos), tokens=tokens,
                               experts=experts, top_k=2, hidden=hidden, kernel=NATIVE)
    pctx = rr.RuntimeContext(stream=ctx.stream, workspace=p(cursors), workspace_bytes=experts * 4,
                             architecture=ctx.architecture)
    ok(rr.token_permute(args, pctx))
    assert np.array_equal(to_host(pos), e_pos)
    got = to_host(xp)
    filled = np.zeros(routes, bool)
    filled[e_pos[valid]] = True
    expect = x[np.nonzero(valid)[0][np.argsort(e_pos[valid])] // 2]
    assert np.array_equal(got[filled].view(np.uint32), expect.view(np.uint32))
    assert np.isnan(got[~filled]).all()
    assert np.array_equal(to_host(cursors), counts)


def test_permute_c4_skew_full_size(ctx, device):
    """C4 routing (Zipf 1.2 over 7 of 8 experts) at T=8192, K=4096: the map is
    bit-exact against the oracle and the copied rows are checked on the device
    (x_permuted[route_pos[r]] == x[r // 2] for every route)."""
    tokens, hidden, experts = 8192, 4096, 8
    ids, _ = workloads.c4_routing(tokens, experts, 7, 1.2, seed=0)
    x = torch.empty(tokens, hidden, device=device)
    assert rr.fill_normal(p(x), x.numel(), 0, workloads.S_X, 0.0, 1.0, ctx.stream) == 0
    x_h = np.zeros((tokens, 0), np.float32)  # map only on the host
    offsets = oracle.exclusive_scan(oracle.histogram(ids, experts))
    xp = torch.empty(2 * tokens, hidden, device=device)
    pos = torch.empty(2 * tokens, dtype=torch.int32, device=device)
    cursors = torch.empty(experts, dtype=torch.int32, device=device)
    ids_d = to_dev(ids.reshape(-1), device)  # kept alive for the call
    offsets_d = to_dev(offsets, device)
    args = rr.TokenPermuteArgs(x=rr.cview(p(x)), expert_ids=p(ids_d),
                               offsets=p(offsets_d), x_permuted=rr.mview(p(xp)),
                               route_pos=p(pos), tokens=tokens, experts=experts, top_k=2, hidden=hidden)
    del x_h
    pctx = rr.RuntimeContext(stream=ctx.stream, workspace=p(cursors), workspace_bytes=experts * 4,
                             architecture=ctx.architecture)
    ok(rr.token_permute(args, pctx))
    e_pos = oracle.stable_route_pos(ids, offsets)
    assert np.array_equal(to_host(pos), e_pos)
    src = torch.arange(2 * tokens, device=device) // 2
    assert torch.equal(xp[pos.long()], x[src])
    assert to_host(cursors)[7] == 0


# -------------------------------------------------------------- grouped GEMM

def run_grouped(ctx, device, x_h, w_h, offsets_h, kernel, max_tokens=None, offset=0, rows_total=None):
    experts, hidden, output = w_h.shape
    rows = rows_total if rows_total is not None else x_h.shape[0]
    xb = torch.empty(rows * hidden + offset, dtype=torch.float32, device=device)
    xb[offset:] = to_dev(x_h.reshape(-1), device)
    wb = torch.empty(w_h.size + offset, dtype=torch.float32, device=device)
    wb[offset:] = to_dev(w_h.reshape(-1), device)
    yb = torch.full((rows * output + offset,), 12345.0, dtype=torch.float32, device=device)
    offs = to_dev(offsets_h.astype(np.int32), device)
    args = rr.GroupedGemmArgs(x_permuted=rr.cview(p(xb) + 4 * offset), expert_weights=rr.cview(p(wb) + 4 * offset),
                              offsets=p(offs), y_permuted=rr.mview(p(yb) + 4 * offset), experts=experts,
                              hidden=hidden, output=output,
                              max_expert_tokens=max_tokens if max_tokens is not None else rows,
                              kernel=kernel)
    ok(rr.grouped_gemm(args, ctx))
    return to_host(yb)[offset:].reshape(rows, output)


def check_grouped(y, x_h, w_h, offsets_h):
    for e in range(w_h.shape[0]):
        s, t = int(offsets_h[e]), int(offsets_h[e + 1])
        if t > s:
            gemm_ok(y[s:t], x_h[s:t], w_h[e])


def test_grouped_gemm_kat(ctx, device, kat):
    g = lambda f: np.array(kat("grouped_unpermute_framework", f))  # noqa: E731
    for kernel in (AUTO, NAIVE, NATIVE):
        y = run_grouped(ctx, device, g("x_permuted").astype(np.float32), g("weights").astype(np.float32),
                        g("offsets"), kernel)
        assert np.array_equal(y, g("y_permuted"))


@pytest.mark.parametrize("counts,hidden,output,offset", [
    ([7, 0, 12, 1, 0], 33, 17, 0),
    ([128] * 64, 256, 128, 0),               # headline-like
    ([0, 300, 5, 1000, 0, 0, 77, 1], 255, 127, 0),  # non-aligned K/N (C4 variant shape, small)
    ([0, 300, 5, 1000, 0, 0, 77, 1], 256, 128, 1),  # unaligned pointers
    ([2000, 100, 0, 3000, 33, 0, 1, 0], 512, 512, 0),
    ([3] * 1024, 16, 16, 0),                  # E = 1024
])
def test_grouped_gemm_random(ctx, device, counts, hidden, output, offset):
    rng = np.random.default_rng(sum(counts) + hidden)
    offsets = oracle.exclusive_scan(np.array(counts, np.int32))
    rows = int(offsets[-1])
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    w = (rng.standard_normal((len(counts), hidden, output)) / np.sqrt(hidden)).astype(np.float32)
    for kernel in (NATIVE, NAIVE):
        y = run_grouped(ctx, device, x, w, offsets, kernel, offset=offset)
        check_grouped(y, x, w, offsets)
        if kernel.family == F.kNaive:
            assert np.array_equal(y, oracle.grouped_gemm_f32_seq(x, w, offsets))


def test_grouped_gemm_rows_outside_segments_untouched(ctx, device):
    rng = np.random.default_rng(4)
    offsets = np.array([0, 10, 10, 30], np.int32)  # rows 30..39 belong to no segment
    x = rng.standard_normal((40, 64)).astype(np.float32)
    w = rng.standard_normal((3, 64, 48)).astype(np.float32)
    for kernel in (NATIVE, NAIVE):
        y = run_grouped(ctx, device, x, w, offsets, kernel, max_tokens=20)
        assert (y[30:] == 12345.0).all()
        check_grouped(y, x, w, offsets)
        # max_expert_tokens = 0 is a no-op (reference src/grouped_gemm/operator.cpp:31)
        y0 = run_grouped(ctx, device, x, w, offsets, kernel, max_tokens=0)
        assert (y0 == 12345.0).all()


def test_grouped_gemm_k0_zeros(ctx, device):
    offsets = np.array([0, 2], np.int32)
    for kernel in (NATIVE, NAIVE):
        y = run_grouped(ctx, device, np.zeros((2, 0), np.float32), np.zeros((1, 0, 2), np.float32), offsets, kernel)
        assert y.reshape(-1).tolist() == [0.0] * 4


# ----------------------------------------------------------------- unpermute

@pytest.mark.parametrize("kernel", [AUTO, NAIVE, NATIVE])
@pytest.mark.parametrize("offset", [0, 1])
def test_unpermute_kat(ctx, device, kat, kernel, offset):
    g = lambda f: kat("unpermute_weighted", f)  # noqa: E731
    width = g("width")
    yp_h = np.repeat(np.arange(1, 5, dtype=np.float32)[:, None], width, axis=1)
    y = run_unpermute(ctx, device, yp_h, np.array(g("route_pos"), np.int32),
                      np.array(g("route_weights"), np.float32), 2, kernel, offset)
    assert np.abs(y[0] - 1.5).max() <= 1e-6 and np.abs(y[1] - 2.8).max() <= 1e-6


def run_unpermute(ctx, device, yp_h, pos_h, w_h, top_k, kernel, offset=0):
    routes, output = yp_h.shape
    tokens = routes // top_k
    ypb = torch.empty(yp_h.size + offset, dtype=torch.float32, device=device)
    ypb[offset:] = to_dev(yp_h.reshape(-1), device)
    yb = torch.full((tokens * output + offset,), -1.0, dtype=torch.float32, device=device)
    pos_d = to_dev(pos_h, device)  # kept alive for the call
    w_d = to_dev(w_h, device)
    args = rr.UnpermuteArgs(y_permuted=rr.cview(p(ypb) + 4 * offset), route_pos=p(pos_d),
                            route_weights=rr.cview(p(w_d)), y=rr.mview(p(yb) + 4 * offset),
                            tokens=tokens, top_k=top_k, output=output, kernel=kernel)
    ok(rr.unpermute(args, ctx))
    return to_host(yb)[offset:].reshape(tokens, output)


@pytest.mark.parametrize("tokens,top_k,output", [(5, 2, 5), (4096, 2, 128), (1000, 1, 33), (333, 8, 64),
                                                 (8192, 2, 1433), (2048, 4, 4), (64, 64, 1030),
                                                 (3, 63, 4097), (7, 3, 1024), (6, 2, 1023)])
def test_unpermute_bit_exact(ctx, device, tokens, top_k, output):
    rng = np.random.default_rng(tokens + output)
    yp = rng.standard_normal((tokens * top_k, output)).astype(np.float32)
    pos = rng.permutation(tokens * top_k).astype(np.int32)
    w = rng.uniform(0.05, 1, tokens * top_k).astype(np.float32)
    expect = oracle.unpermute_f32(yp, pos, w, top_k)
    for kernel in (NATIVE, NAIVE):
        y = run_unpermute(ctx, device, yp, pos, w, top_k, kernel)
        # same rank order, separately rounded multiply and add: bit-exact
        assert np.array_equal(y.view(np.uint32), expect.view(np.uint32))


# ------------------------------------------------------------- input streams

def test_device_fill_matches_host_generator(ctx, device):
    n = 1 << 16
    for seed, sid in ((0, workloads.S_X), (7, workloads.S_EXPERTS)):
        buf = torch.empty(n, device=device)
        assert rr.fill_uniform(p(buf), n, seed, sid, -1.0, 1.0, ctx.stream) == 0
        assert np.array_equal(to_host(buf), workloads.uniform(n, seed, sid))
        assert rr.fill_normal(p(buf), n, seed, sid, 0.0, 0.0625, ctx.stream) == 0
        np.testing.assert_allclose(to_host(buf), workloads.normal(n, seed, sid, 0.0, 0.0625),
                                   rtol=1e-6, atol=1e-7)
