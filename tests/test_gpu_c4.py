"""C4 at full size: Mixtral-shaped ragged grouped GEMM (T=8192, R=16384, E=8
with 7 active experts under Zipf(1.2), K=4096, N=14336) and its non-aligned
variant (K=4095, N=14335), through histogram_exclusive_scan -> token_permute
-> grouped_gemm -> unpermute on the device.

The full FP64 CPU product (1.9 TFLOP) is out of reach, so parity is pinned by
(1) a size-independent checksum per expert: sum_r y[r, :] equals
(sum_r x[r, :]) @ W[e] within the summed accumulation-aware bound, which fails
if any tile, row or column of an expert is skipped, duplicated or misplaced,
and (2) sampled rows x sampled columns against the oracle's FP64 GEMM under
the per-element bound of reference src/correctness/reference_validation.cpp:78-100.
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
def test_c4_grouped_gemm_full_size(ctx, device, hidden, output):
    t, e = 8192, 8
    r = 2 * t
    ids_h, w_h = workloads.c4_routing(t, e, 7, 1.2, seed=0)
    x = torch.empty(t, hidden, device=device)
    we = torch.empty(e, hidden, output, device=device)
    ok_fill = rr.fill_normal(x.data_ptr(), x.numel(), 0, workloads.S_X, 0.0, 1.0, ctx.stream)
    sd = float(np.float32(1.0 / np.sqrt(hidden)))
    ok_fill |= rr.fill_normal(we.data_ptr(), we.numel(), 0, workloads.S_EXPERTS, 0.0, sd, ctx.stream)
    assert ok_fill == 0
    ids = torch.from_numpy(ids_h.reshape(-1)).to(device)
    i32 = dict(dtype=torch.int32, device=device)
    counts, offsets = torch.empty(e, **i32), torch.empty(e + 1, **i32)
    ok(rr.histogram_exclusive_scan(rr.HistogramExclusiveScanArgs(
        expert_ids=ids.data_ptr(), counts=counts.data_ptr(), offsets=offsets.data_ptr(),
        route_pairs=r, experts=e), ctx))
    xp = torch.empty(r, hidden, device=device)
    pos = torch.empty(r, **i32)
    cursors = torch.empty(e, **i32)
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
    torch.cuda.synchronize()

    off = to_host(offsets)
    assert np.array_equal(off, oracle.exclusive_scan(oracle.histogram(ids_h, e)))
    assert off[-1] == r and off[-2] == r  # expert 7 is empty
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

    # sampled rows x sampled columns against the FP64 oracle and the per-element bound
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
