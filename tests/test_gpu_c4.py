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
* grouped GEMM, every element: the naive family's grouped GEMM (the
  reference cuda_naive loop: one thread per output, sequential FP32 k, each
  product and sum separately rounded; pinned bit-exact to the oracle's
  sequential loop by tests/test_gpu_ops.py::test_grouped_gemm_random and
  here on sampled rows) is run on the same x_permuted and offsets, and
  again on |x_permuted| and |W| for S = sum_k |a*b|. The sequential sum
  lies within gamma_K * S of the exact product, so asserting
  |y - y_naive| <= 3 * gamma_K * S / (1 - gamma_K) + 1e-7 for every element
  puts every element within the reference's bound 4 * gamma_K * S + 1e-7
  of the exact product (reference
  src/correctness/reference_validation.cpp:78-100; the reference compares
  the entire grouped output, benchmarks/adapters/grouped_gemm_adapter.cpp:
  346-347). Sampled rows x columns are also checked against the oracle's
  FP64 GEMM directly;
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

    # ---- grouped GEMM: every element against the naive device GEMM ----
    assert not torch.isnan(yp).any(), "rows of the routed range were not written"
    naive = rr.kernel(rr.KernelFamily.kNaive)

    def naive_gemm(a, b):
        out = torch.full((r, output), float("nan"), device=device)
        ok(rr.grouped_gemm(rr.GroupedGemmArgs(
            x_permuted=rr.cview(a.data_ptr()), expert_weights=rr.cview(b.data_ptr()),
            offsets=offsets.data_ptr(), y_permuted=rr.mview(out.data_ptr()), experts=e, hidden=hidden,
            output=output, max_expert_tokens=r, kernel=naive), ctx))
        return out
    yn = naive_gemm(xp, we)
    sabs = naive_gemm(xp.abs(), we.abs())
    torch.cuda.synchronize()
    gamma = hidden * U32 / (1 - hidden * U32)
    worst = 0.0
    for lo in range(0, r, 1024):
        hi = min(r, lo + 1024)
        diff = (yp[lo:hi].double() - yn[lo:hi].double()).abs()
        allowed = 3 * gamma * sabs[lo:hi].double() / (1 - gamma) + 1e-7
        bad = int((diff > allowed).sum())
        assert bad == 0, f"grouped GEMM rows [{lo}, {hi}): {bad} elements outside the bound of the naive GEMM"
        worst = max(worst, (diff / allowed).max().item())
    print(f"C4 grouped GEMM: every element within {worst:.3g} of its bound", flush=True)
    del diff, allowed
    # the naive GEMM itself: bit-exact against the oracle's sequential FP32
    # loop on each active expert's first and last rows (64-bit offsets at the
    # far end of x_permuted and y_permuted)
    for ex in range(7):
        s, f = int(off[ex]), int(off[ex + 1])
        rows_t = torch.tensor([s, f - 1], device=device)
        expect = oracle.dense_gemm_f32_seq(to_host(xp[rows_t]), to_host(we[ex]))
        assert np.array_equal(to_host(yn[rows_t]).view(np.int32), expect.view(np.int32)), \
            f"naive grouped GEMM differs from the oracle on expert {ex}"
    del yn, sabs
    # and sampled rows x columns of the native output against the FP64 oracle
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
