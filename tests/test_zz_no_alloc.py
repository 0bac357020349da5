"""rr_chain_from_tokens_noalloc: chain_from_tokens with the chain workspace in
the library's static device scratch instead of the caller's context.

GPU: two calls in a row through the C ABI, the second with a smaller input,
each checked bit for bit against rr_chain_from_tokens with a caller
workspace (every output poisoned before each call), on the merged two-launch
plan (K <= 256) and on the three-launch plan (K > 256, whose route
preparation keeps sorted_route in the scratch when the caller passes none).
GPU, in a fresh process: the very first call on the device (which resolves
the scratch address) made inside a thread-local stream capture, the graph
replayed several times with the outputs poisoned between replays, every
replay bit for bit equal to the eager rr_chain_from_tokens.
CPU: shapes beyond the scratch are rejected before any device call.
"""
from __future__ import annotations

import subprocess
import sys
import textwrap
from ctypes import byref
from pathlib import Path

import pytest
import torch

import raggedroute_amd as rr
from raggedroute_amd import workloads


def _outputs(t, e, k, n, device):
    i32 = dict(dtype=torch.int32, device=device)
    return {
        "logits": torch.full((t, e), float("nan"), device=device),
        "ids": torch.full((t, 2), -7, **i32),
        "w": torch.full((t, 2), float("nan"), device=device),
        "counts": torch.full((e,), -7, **i32),
        "offsets": torch.full((e + 1,), -7, **i32),
        "xp": torch.full((2 * t, k), float("nan"), device=device),
        "pos": torch.full((2 * t,), -7, **i32),
        "yp": torch.full((2 * t, n), float("nan"), device=device),
        "y": torch.full((t, n), float("nan"), device=device),
    }


def _args(inp, out, t, e, k, n):
    return rr.ChainArgs(
        x=inp["x"].data_ptr(), router_weights=inp["router_weights"].data_ptr(),
        logits=out["logits"].data_ptr(), expert_ids=out["ids"].data_ptr(),
        route_weights=out["w"].data_ptr(), counts=out["counts"].data_ptr(),
        offsets=out["offsets"].data_ptr(), x_permuted=out["xp"].data_ptr(),
        route_pos=out["pos"].data_ptr(), sorted_route=None,
        expert_weights=inp["expert_weights"].data_ptr(), y_permuted=out["yp"].data_ptr(),
        y=out["y"].data_ptr(), tokens=t, experts=e, hidden=k, output=n)


def _same(a, b):
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("shapes", [
    [(4096, 64, 256, 128), (512, 32, 256, 64)],  # merged launch plan
    [(1000, 16, 300, 40), (300, 16, 300, 40)],   # route_prep + tiled GEMM plan
])
def test_noalloc_chain_matches_workspace_chain(device, shapes):
    stream = torch.cuda.current_stream(device).cuda_stream
    for t, e, k, n in shapes:  # the second call is the smaller one
        print(f"noalloc chain T={t} E={e} K={k} N={n}", flush=True)
        cfg = workloads.ChainConfig("noalloc", t, e, k, n, from_tokens=True)
        inp = workloads.chain_inputs_device(cfg, 0, device)
        ref = _outputs(t, e, k, n, device)
        ref_args = _args(inp, ref, t, e, k, n)
        ws = torch.empty(rr.get_chain_workspace_size(ref_args) // 4, dtype=torch.int32, device=device)
        ctx = rr.RuntimeContext(stream=stream, workspace=ws.data_ptr(), workspace_bytes=ws.numel() * 4,
                                architecture=int(rr.DeviceArchitecture.kGfx950))
        status = rr.chain_from_tokens(ref_args, ctx)
        assert status.ok(), status.message
        got = _outputs(t, e, k, n, device)
        # the caller's workspace fields are ignored: none is passed
        bare = rr.RuntimeContext(stream=stream, architecture=int(rr.DeviceArchitecture.kGfx950))
        status = rr.lib.rr_chain_from_tokens_noalloc(byref(_args(inp, got, t, e, k, n)), byref(bare))
        assert status.ok(), status.message
        torch.cuda.synchronize()
        for key in ref:
            assert _same(got[key], ref[key]), f"{key} differs (T={t})"
        assert not torch.isnan(got["y"]).any()


CAPTURE_CHILD = textwrap.dedent("""
    import sys
    from ctypes import byref
    sys.path.insert(0, REPO)
    import torch
    import raggedroute_amd as rr
    from raggedroute_amd import workloads
    sys.path.insert(0, REPO + "/tests")
    from test_zz_no_alloc import _outputs, _args, _same
    device = torch.device("cuda:0")
    t, e, k, n = 4096, 64, 256, 128
    cfg = workloads.ChainConfig("noalloc", t, e, k, n, from_tokens=True)
    inp = workloads.chain_inputs_device(cfg, 0, device)
    got = _outputs(t, e, k, n, device)
    side = torch.cuda.Stream(device)
    bare = rr.RuntimeContext(stream=side.cuda_stream, architecture=int(rr.DeviceArchitecture.kGfx950))
    args = _args(inp, got, t, e, k, n)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side, capture_error_mode="thread_local"):
        status = rr.lib.rr_chain_from_tokens_noalloc(byref(args), byref(bare))
    assert status.ok(), status.message
    ref = _outputs(t, e, k, n, device)
    ref_args = _args(inp, ref, t, e, k, n)
    ws = torch.empty(rr.get_chain_workspace_size(ref_args) // 4, dtype=torch.int32, device=device)
    ctx = rr.RuntimeContext(stream=torch.cuda.current_stream(device).cuda_stream, workspace=ws.data_ptr(),
                            workspace_bytes=ws.numel() * 4, architecture=int(rr.DeviceArchitecture.kGfx950))
    assert rr.chain_from_tokens(ref_args, ctx).ok()
    torch.cuda.synchronize()
    for replay in range(3):
        for v in got.values():
            v.fill_(float("nan") if v.dtype == torch.float32 else -7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for key in ref:
            assert _same(got[key], ref[key]), f"replay {replay}: {key} differs"
    print("captured first call: 3 replays equal to the eager chain")
""")


@pytest.mark.gpu
def test_noalloc_first_call_inside_a_graph_capture():
    repo = str(Path(__file__).resolve().parent.parent)
    proc = subprocess.run([sys.executable, "-c", f"REPO = {repo!r}\n" + CAPTURE_CHILD],
                          capture_output=True, text=True, timeout=240)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-2000:]


def test_noalloc_rejects_shapes_beyond_the_scratch():
    """experts + 2 * tokens > 262144 int32 words: rejected before any device
    call (so this runs without a GPU); the bound itself is accepted by the
    size check."""
    too_big = rr.ChainArgs(tokens=131000, experts=1024, hidden=16, output=16)
    status = rr.lib.rr_chain_from_tokens_noalloc(byref(too_big), byref(rr.RuntimeContext()))
    assert status.code == rr.StatusCode.kInvalidArgument
    assert "static scratch" in status.message
    fits = rr.ChainArgs(tokens=(262144 - 1024) // 2, experts=1024)
    assert rr.get_chain_workspace_size(fits) <= 1 << 20
    status = rr.lib.rr_chain_from_tokens_noalloc(None, byref(rr.RuntimeContext()))
    assert status.code == rr.StatusCode.kInvalidArgument
