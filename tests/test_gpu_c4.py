"""C4 at full size: Mixtral-shaped ragged grouped GEMM (T=8192, R=16384, E=8
with 7 active experts under Zipf(1.2), K=4096, N=14336) and its non-aligned
variant (K=4095, N=14335), through histogram_exclusive_scan -> token_permute
-> grouped_gemm -> unpermute on the device, every stage checked:

* counts / offsets: bit-exact against the oracle (expert 7 empty);
* route_pos: bit-exact against the oracle's stable map; permute cursors end
  equal to the counts (reference tests/operator_api_tests.cpp:777-778);
* x_permuted: every routed row checked on the device, x_permuted[route_pos[r]]
  == x[r // 2] bitwise (the row copy is exact, reference
  src/permute/cpu_reference/reference.cpp:67-71), so the GEMM checks below
  start from rows known to be right;
* grouped GEMM: the full FP64 CPU product (1.9 TFLOP) is out of reach, so it
  is pinned by (1) a size-independent checksum per expert: sum_r y[r, :]
  equals (sum_r x[r, :]) @ W[e] within the summed accumulation-aware bound,
  which fails if any tile, row or column of an expert is skipped, duplicated
  or misplaced, and (2) sampled rows x sampled columns against the oracle's
  FP64 GEMM under the per-element bound of reference
  src/correctness/reference_validation.cpp:78-100;
* unpermute: bit-exact over every element on the device against
  fl(fl(0 + fl(w0 * yp[p0])) + fl(w1 * yp[p1])), each operation a separately
  rounded FP32 torch op (reference src/unpermute/cpu_reference/reference.cpp:10-36
  sums in rank order from zero), plus a seeded sample of 64 tokens against
  oracle.unpermute_f32 on the host.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import raggedroute_amd as rr
from raggedroute_amd import workloads
from conftest import to_host

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


def ok(status):
    assert status.ok(), status.message


@pytest.mark.parametrize("hidden,output", [(4096, 14336), (4095, 14335)])
def test_c4_pipeline_full_size(ctx, device, hidden, output):
    t, e = 8192, 8
    r = 2 * t
    print(f"C4 pipeline K={hidden} N={output}", flush=True)
    ids_h, w_h = workloads.c4_routing(t, e, 7, 1.2, seed=0)
    x = torch.empty(t, hidden, device=device)
    we = torch.empty(e, hidden, output, device=device)
    ok_fill = rr.fill_normal(x.data_ptr(), x.numel(), 0, workloads.S_X, 0.0, 1.0, ctx.stream)
    sd = float(np.float32(1.0 / np.sqrt(hidden)))
    ok_fill |= rr.fill_normal(we.data_ptr(), we.numel(), 0, workloads.S_EXPERTS, 0.0, sd, ctx.stream)
    assert ok_fill == 0
    ids = torch.from_numpy(ids_h.reshape(-1)).to(device)
    w_d = torch.from_numpy(w_h.reshape(-1)).to(device)
    i32 = dict(dtype=torch.int32, device=device)
    counts, offsets = torch.empty(e, **i32), torch.empty(e + 1, **i32)
    ok(rr.histogram_exclusive_scan(rr.HistogramExclusiveScanArgs(
        expert_ids=ids.data_ptr(), counts=counts.data_ptr(), offsets=offsets.data_ptr(),
        route_pairs=r, experts=e), ctx))
    # poisoned outputs: a row or entry the device never writes cannot pass
    xp = torch.full((r, hidden), float("nan"), device=device)
    pos = torch.full((r,), -7, **i32)
    cursors = torch.full((e,), -7, **i32)
    pctx = rr.RuntimeContext(stream=ctx.stream, workspace=cursors.data_ptr(), workspace_bytes=4 * e,
                             architecture=ctx.architecture)
    ok(rr.token_permute(rr.TokenPermuteArgs(
        x=rr.cview(x.data_ptr()), expert_ids=ids.data_ptr(), offsets=offsets.data_ptr(),
        x_permuted=rr.mview(xp.data_ptr()), route_pos=pos.data_ptr(), tokens=t, experts=e, top_k=2,
        hidden=hidden), pctx))
    yp = torch.full((r, output), float("nan"), device=device)
    ok(rr.grouped_gemm(rr.GroupedGemmArgs(
        x_permuted=rr.cview(xp.data_ptr()), expert_weights=rr.cview(we.data_ptr()),
        offsets=offsets.data_ptr(), y_permuted=rr.mview(yp.data_ptr()), experts=e, hidden=hidden,
        output=output, max_expert_tokens=r), ctx))
    y = torch.full((t, output), float("nan"), device=device)
    ok(rr.unpermute(rr.UnpermuteArgs(
        y_permuted=rr.cview(yp.data_ptr()), route_pos=pos.data_ptr(),
        route_weights=rr.cview(w_d.data_ptr()), y=rr.mview(y.data_ptr()), tokens=t, top_k=2,
        output=output), ctx))
    torch.cuda.synchronize()

    # ---- metadata and the row map: bit-exact ----
    ref_counts = oracle.histogram(ids_h, e)
    ref_off = oracle.exclusive_scan(ref_counts)
    off = to_host(offsets)
    assert np.array_equal(to_host(counts), ref_counts)
    assert np.array_equal(off, ref_off)
    assert off[-1] == r and off[-2] == r  # expert 7 is empty
    pos_h = to_host(pos)
    assert np.array_equal(pos_h, oracle.stable_route_pos(ids_h, ref_off)), "route_pos differs"
    assert np.array_equal(to_host(cursors), ref_counts), "cursors do not end equal to the counts"

    # ---- the copied rows: every routed row, bitwise, on the device ----
    pos_l = pos.long()
    src = torch.arange(r, device=device) // 2
    for lo in range(0, r, 4096):  # (row blocks keep the temporaries small)
        rows = xp[pos_l[lo:lo + 4096]]
        assert torch.equal(rows.view(torch.int32), x[src[lo:lo + 4096]].view(torch.int32)), \
            f"x_permuted rows of routes [{lo}, {lo + 4096}) differ from x"
    del rows

    # ---- grouped GEMM: checksums per expert + sampled elements ----
    assert not torch.isnan(yp).any(), "rows of the routed range were not written"
    gamma = hidden * U32 / (1 - hidden * U32)
    for ex in range(e):
        s, f = int(off[ex]), int(off[ex + 1])
        if f == s:
            continue
        xs, ys, w64 = xp[s:f].double(), yp[s:f].double(), we[ex].double()
        got = ys.sum(0)
        want = xs.sum(0) @ w64
        bound = 4 * gamma * (xs.abs().sum(0) @ w64.abs()) + (f - s) * 1e-7 + 1e-9 * want.abs()
        excess = ((got - want).abs() - bound).max().item()
        assert excess <= 0, f"expert {ex}: row-sum checksum exceeds its bound by {excess}"
        del xs, ys, w64
    rng = np.random.default_rng(hidden)
    cols = np.sort(rng.choice(output, 1024, replace=False))
    cols_t = torch.from_numpy(cols).to(device)
    for ex in range(7):
        s, f = int(off[ex]), int(off[ex + 1])
        rows = np.unique(np.concatenate([[s, f - 1], rng.integers(s, f, 4)]))
        a = to_host(xp[torch.from_numpy(rows).to(device)])
        b = to_host(we[ex][:, cols_t])
        got = to_host(yp[torch.from_numpy(rows).to(device)][:, cols_t])
        expect = oracle.dense_gemm_f64(a, b)
        fails, max_abs, ratio = oracle.compare_gemm(got.astype(np.float64), expect, a, b)
        assert fails == 0, f"expert {ex}: {fails} sampled elements exceed the bound (ratio {ratio})"

    # ---- unpermute: every element bit-exact on the device ----
    w2 = w_d.view(t, 2)
    p2 = pos_l.view(t, 2)
    for lo in range(0, t, 2048):
        hi = lo + 2048
        a0 = w2[lo:hi, 0:1] * yp[p2[lo:hi, 0]]  # fl(w0 * v0)
        a1 = w2[lo:hi, 1:2] * yp[p2[lo:hi, 1]]  # fl(w1 * v1)
        want = (torch.zeros_like(a0) + a0) + a1  # rank order from zero
        assert torch.equal(y[lo:hi].view(torch.int32), want.view(torch.int32)), \
            f"unpermute rows [{lo}, {hi}) differ from the rank-order sum"
    del a0, a1, want
    # and a seeded token sample against the oracle on the host
    toks = np.sort(np.random.default_rng(7).choice(t, 64, replace=False))
    routes = np.stack([2 * toks, 2 * toks + 1], axis=1).reshape(-1)
    sub_pos = np.arange(routes.size, dtype=np.int32)  # rows gathered in route order
    yp_rows = to_host(yp[torch.from_numpy(pos_h[routes].astype(np.int64)).to(device)])
    expect = oracle.unpermute_f32(yp_rows, sub_pos, w_h.reshape(-1)[routes], 2)
    got = to_host(y[torch.from_numpy(toks).to(device)])
    assert np.array_equal(got.view(np.int32), expect.view(np.int32)), "sampled tokens differ from the oracle"
