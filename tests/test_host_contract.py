"""Host-side contract of the C ABI, on the CPU (no device call is made).

Mirrors the pure-dispatch and argument/workspace tests of reference
tests/operator_api_tests.cpp:63-315 with the architecture fixed to gfx950 in
the RuntimeContext (so no device query happens) and each call failing, or
returning early, before any launch. Also checks that the library exports every
entry point the C header declares and that an out-of-tree C++ consumer of
include/raggedroute/*.h compiles, links and runs (reference
tests/packaging/consumer.cpp).
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

import raggedroute_amd as rr
from conftest import REPO

S = rr.StatusCode
F = rr.KernelFamily
K = rr.OperatorKind
GFX950 = int(rr.DeviceArchitecture.kGfx950)


def host_ctx(**kw):
    return rr.RuntimeContext(architecture=GFX950, **kw)


def test_library_exports_every_declared_entry():
    header = (REPO / "include" / "raggedroute_capi.h").read_text()
    body = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    declared = set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(rr_\w+)\s*\(", body, flags=re.M))
    assert len(declared) >= 36
    missing = [name for name in sorted(declared) if not hasattr(rr.lib, name)]
    assert not missing, f"not exported: {missing}"
    # and the Python prototypes cover exactly the declared set
    assert {name for name, _, _ in rr.PROTOTYPES} == declared
    assert rr.lib.rr_capi_version() == 2 and rr.lib.rr_build_target() == b"gfx950"


def test_enum_ordinals_match_reference():
    # reference include/raggedroute/types.h:8-95, status.h:7-16
    assert [int(k) for k in K] == list(range(8))
    assert (S.kSuccess, S.kInvalidArgument, S.kUnsupportedArchitecture, S.kUnsupportedDataType,
            S.kUnsupportedLayout, S.kUnsupportedKernelVariant, S.kInsufficientWorkspace,
            S.kDeviceError) == tuple(range(8))
    assert (int(F.kAuto), int(F.kNaive), int(F.kOptimized)) == (0, 1, 2)
    assert [int(a) for a in rr.DeviceArchitecture] == [0, 1, 2, 3, 4]
    assert int(rr.ScalarType.kFp4E2M1) == 7 and int(rr.TensorLayout.kStrided) == 2


def test_struct_layouts():
    # C struct sizes on LP64 (checked against the header's field lists)
    assert ctypes.sizeof(rr.TensorSpec) == 32
    assert ctypes.sizeof(rr.ConstTensorView) == 40
    assert ctypes.sizeof(rr.RuntimeContext) == 32
    assert ctypes.sizeof(rr.Status) == 16
    assert ctypes.sizeof(rr.KernelSelection) == 8


def fp32_signature(kind: K) -> rr.OperatorSignature:
    s = rr.OperatorSignature()
    roles = {
        K.kDenseGemm: "iwao", K.kGroupedGemm: "iwao", K.kUnpermute: "iwao", K.kTopKGate: "iao",
        K.kTokenPermute: "io",
    }.get(kind, "")
    s.has_input, s.has_weight = int("i" in roles), int("w" in roles)
    s.has_accumulator, s.has_output = int("a" in roles), int("o" in roles)
    return s


def select(kind, arch=GFX950, kernel=None, signature=None):
    req = rr.DispatchRequest(operator_kind=int(kind), architecture=arch,
                             requested_kernel=kernel or rr.kernel(),
                             signature=signature if signature is not None else fp32_signature(kind))
    dec = rr.DispatchDecision()
    return rr.select_kernel(req, dec), dec


def test_classification():
    assert rr.classify_compute_capability(8, 6) == rr.DeviceArchitecture.kSm86
    assert rr.classify_compute_capability(8, 0) == rr.DeviceArchitecture.kOther
    assert rr.classify_compute_capability(9, 0) == rr.DeviceArchitecture.kSm90
    assert rr.classify_gcn_arch_name("gfx950:sramecc+:xnack-") == rr.DeviceArchitecture.kGfx950
    assert rr.classify_gcn_arch_name("gfx950") == rr.DeviceArchitecture.kGfx950
    assert rr.classify_gcn_arch_name("gfx942:sramecc+:xnack-") == rr.DeviceArchitecture.kOther
    assert rr.classify_gcn_arch_name("gfx9500") == rr.DeviceArchitecture.kOther
    status, arch = rr.resolve_device_architecture(rr.DeviceArchitecture.kGfx950)
    assert status.ok() and arch == rr.DeviceArchitecture.kGfx950


@pytest.mark.parametrize("kind", list(K))
def test_auto_dispatch_selects_native(kind):
    status, dec = select(kind)
    assert status.ok(), status.message
    assert dec.kernel.family == F.kOptimized and dec.kernel.implementation_id == rr.GFX950_NATIVE
    assert dec.architecture == GFX950 and dec.operator_kind == int(kind)
    status, dec = select(kind, kernel=rr.kernel(F.kNaive, 0))
    assert status.ok() and dec.kernel.family == F.kNaive and dec.kernel.implementation_id == 0
    status, dec = select(kind, kernel=rr.kernel(F.kOptimized, rr.GFX950_NATIVE))
    assert status.ok() and dec.kernel.implementation_id == rr.GFX950_NATIVE


def test_dispatch_rejections():
    kind = K.kDenseGemm
    for arch in (rr.DeviceArchitecture.kOther, rr.DeviceArchitecture.kSm86, rr.DeviceArchitecture.kSm90):
        assert select(kind, arch=int(arch))[0].code == S.kUnsupportedArchitecture
    assert select(kind, arch=0)[0].code == S.kInvalidArgument  # unresolved kAuto
    for dtype in (rr.ScalarType.kFp16, rr.ScalarType.kBf16):
        sig = fp32_signature(kind)
        sig.input.dtype = sig.weight.dtype = sig.output.dtype = int(dtype)
        assert select(kind, signature=sig)[0].code == S.kUnsupportedDataType
    sig = fp32_signature(kind); sig.input.layout = int(rr.TensorLayout.kStrided)
    assert select(kind, signature=sig)[0].code == S.kUnsupportedLayout
    sig = fp32_signature(kind); sig.input.strides[0] = 1
    assert select(kind, signature=sig)[0].code == S.kUnsupportedLayout
    sig = fp32_signature(kind); sig.has_weight = 0
    assert select(kind, signature=sig)[0].code == S.kInvalidArgument
    # layout is checked before the architecture, dtype before the architecture
    sig = fp32_signature(kind); sig.output.layout = int(rr.TensorLayout.kColumnMajorContiguous)
    assert select(kind, arch=int(rr.DeviceArchitecture.kSm86), signature=sig)[0].code == S.kUnsupportedLayout
    assert select(kind, kernel=rr.kernel(F.kOptimized, 0))[0].code == S.kUnsupportedKernelVariant
    assert select(kind, kernel=rr.kernel(F.kNaive, 1))[0].code == S.kUnsupportedKernelVariant
    assert select(kind, kernel=rr.kernel(F.kAuto, 1))[0].code == S.kUnsupportedKernelVariant
    assert select(kind, kernel=rr.KernelSelection(7, 0))[0].code == S.kUnsupportedKernelVariant
    req = rr.DispatchRequest(operator_kind=int(kind), architecture=GFX950, signature=fp32_signature(kind))
    assert rr.select_kernel(req, None).code == S.kInvalidArgument
    req.operator_kind = 99
    assert rr.select_kernel(req, rr.DispatchDecision()).code == S.kInvalidArgument


@pytest.mark.parametrize("kind,accepted,rejected", [
    (K.kDenseGemm, range(1, 8), [8, 101]),
    (K.kTopKGate, range(1, 5), [5]),
    (K.kHistogram, [101], [1, 102]),
    (K.kHistogramExclusiveScan, [2], [1, 99]),
    (K.kTokenPermute, range(1, 11), [11]),
    (K.kExclusiveScan, [], [1]),
    (K.kGroupedGemm, [], range(1, 7)),
    (K.kUnpermute, [], [1, 2]),
])
def test_reference_optimized_ids(kind, accepted, rejected):
    # reference tests/operator_api_tests.cpp:118-266: explicit ids keep their value
    for i in accepted:
        status, dec = select(kind, kernel=rr.kernel(F.kOptimized, i))
        assert status.ok() and dec.kernel.implementation_id == i
    for i in rejected:
        assert select(kind, kernel=rr.kernel(F.kOptimized, i))[0].code == S.kUnsupportedKernelVariant


def test_argument_contracts():
    ctx = host_ctx()
    d = rr.DenseGemmArgs(m=-1)
    assert rr.dense_gemm(d, ctx).code == S.kInvalidArgument
    d = rr.DenseGemmArgs()
    d.a.spec.dtype = d.b.spec.dtype = d.c.spec.dtype = int(rr.ScalarType.kFp16)
    assert rr.dense_gemm(d, ctx).code == S.kUnsupportedDataType
    d = rr.DenseGemmArgs(); d.a.spec.strides[0] = 1
    assert rr.dense_gemm(d, ctx).code == S.kUnsupportedLayout
    buf = ctypes.create_string_buffer(16)
    d = rr.DenseGemmArgs(m=1, n=1, c=rr.mview(ctypes.addressof(buf) + 1))
    assert rr.dense_gemm(d, ctx).code == S.kInvalidArgument  # misaligned
    d = rr.DenseGemmArgs(m=1, n=1, k=1)
    d.alpha = 2.0
    assert rr.dense_gemm(d, ctx).code == S.kInvalidArgument
    assert rr.dense_gemm(rr.DenseGemmArgs(m=0, n=4, k=4), ctx).ok()  # empty: no launch

    g = rr.TopKGateArgs(tokens=1, experts=1)
    assert rr.topk_gate(g, ctx).code == S.kInvalidArgument
    g = rr.TopKGateArgs(tokens=1, experts=rr.MAX_EXPERTS + 1)
    assert rr.topk_gate(g, ctx).code == S.kInvalidArgument
    g = rr.TopKGateArgs(tokens=1, experts=8, top_k=3)
    assert rr.topk_gate(g, ctx).code == S.kInvalidArgument
    g = rr.TopKGateArgs(tokens=1, experts=8); g.tie_break = 1
    assert rr.topk_gate(g, ctx).code == S.kInvalidArgument
    assert rr.topk_gate(rr.TopKGateArgs(tokens=0, experts=1024), ctx).ok()

    assert rr.histogram(rr.HistogramArgs(route_pairs=1, experts=0), ctx).code == S.kInvalidArgument
    assert rr.histogram(rr.HistogramArgs(route_pairs=1, experts=4), ctx).code == S.kInvalidArgument  # null

    scan = rr.ExclusiveScanArgs(experts=1)
    assert rr.exclusive_scan(scan, ctx).code == S.kInvalidArgument  # null pointers
    store = (ctypes.c_int32 * 8)()
    scan = rr.ExclusiveScanArgs(counts=ctypes.addressof(store), offsets=ctypes.addressof(store), experts=1025)
    assert rr.exclusive_scan(scan, ctx).code == S.kInvalidArgument
    scan.experts = 0
    assert rr.exclusive_scan(scan, ctx).code == S.kInvalidArgument
    scan.experts = 1; scan.kernel = rr.kernel(F.kOptimized, 1)
    assert rr.exclusive_scan(scan, ctx).code == S.kUnsupportedKernelVariant
    scan.kernel = rr.kernel(); scan.counts = ctypes.addressof(buf) + 1; scan.offsets = ctypes.addressof(buf) + 1
    assert rr.exclusive_scan(scan, ctx).code == S.kInvalidArgument

    base = ctypes.addressof(store)
    fused = rr.HistogramExclusiveScanArgs(expert_ids=base, counts=base, offsets=base, route_pairs=1, experts=1)
    assert rr.histogram_exclusive_scan(fused, ctx).code == S.kInvalidArgument  # overlap
    fused.counts = None
    assert rr.histogram_exclusive_scan(fused, ctx).code == S.kInvalidArgument
    fused.counts, fused.offsets = base + 8, base + 16
    fused.kernel = rr.kernel(F.kOptimized, 99)
    assert rr.histogram_exclusive_scan(fused, ctx).code == S.kUnsupportedKernelVariant
    fused.route_pairs = -1
    assert rr.histogram_exclusive_scan(fused, ctx).code == S.kInvalidArgument


def test_workspace_contracts():
    ctx = host_ctx()
    placeholder = ctypes.c_int32(0)
    addr = ctypes.addressof(placeholder)
    p = rr.TokenPermuteArgs(tokens=1, experts=2, top_k=1, hidden=0, expert_ids=addr, offsets=addr,
                            route_pos=addr)
    assert rr.get_token_permute_workspace_size(p) == 8
    assert rr.token_permute(p, ctx).code == S.kInsufficientWorkspace
    assert rr.token_permute(p, host_ctx(workspace=addr, workspace_bytes=4)).code == S.kInsufficientWorkspace
    mismatched = rr.TokenPermuteArgs(experts=2, top_k=1)
    mismatched.x.spec.dtype = int(rr.ScalarType.kFp16)
    mismatched.x_permuted.spec.dtype = int(rr.ScalarType.kBf16)
    assert rr.token_permute(mismatched, ctx).code == S.kUnsupportedDataType
    assert rr.token_permute(rr.TokenPermuteArgs(tokens=1, experts=2, top_k=3), ctx).code == S.kInvalidArgument
    assert rr.token_permute(rr.TokenPermuteArgs(tokens=2**30, experts=8, top_k=2), ctx).code == S.kInvalidArgument
    assert rr.token_permute(rr.TokenPermuteArgs(tokens=0, experts=8, top_k=2), ctx).ok()
    for fn, args in ((rr.get_dense_gemm_workspace_size, rr.DenseGemmArgs()),
                     (rr.get_topk_gate_workspace_size, rr.TopKGateArgs()),
                     (rr.get_histogram_workspace_size, rr.HistogramArgs()),
                     (rr.get_exclusive_scan_workspace_size, rr.ExclusiveScanArgs()),
                     (rr.get_histogram_exclusive_scan_workspace_size, rr.HistogramExclusiveScanArgs()),
                     (rr.get_grouped_gemm_workspace_size, rr.GroupedGemmArgs()),
                     (rr.get_unpermute_workspace_size, rr.UnpermuteArgs())):
        assert fn(args) == 0

    gg = rr.GroupedGemmArgs(experts=0)
    assert rr.grouped_gemm(gg, ctx).code == S.kInvalidArgument
    gg = rr.GroupedGemmArgs(experts=8, hidden=4, output=4, max_expert_tokens=0)
    assert rr.grouped_gemm(gg, ctx).ok()  # launch bound 0: no-op
    gg.max_expert_tokens = 4
    assert rr.grouped_gemm(gg, ctx).code == S.kInvalidArgument  # null pointers

    up = rr.UnpermuteArgs(tokens=1, top_k=65, output=1)
    assert rr.unpermute(up, ctx).code == S.kInvalidArgument
    up = rr.UnpermuteArgs(tokens=2**20, top_k=2, output=2**12)
    assert rr.unpermute(up, ctx).code == S.kInvalidArgument  # T*N exceeds int32
    assert rr.unpermute(rr.UnpermuteArgs(tokens=0, top_k=2, output=8), ctx).ok()

    chain = rr.ChainArgs(tokens=4, experts=8, top_k=3)
    assert rr.chain_from_tokens(chain, ctx).code == S.kInvalidArgument
    chain = rr.ChainArgs(tokens=4, experts=8, hidden=4, output=4, logits=addr, expert_ids=addr,
                         route_weights=addr, counts=addr, offsets=addr, route_pos=addr, y_permuted=addr,
                         y=addr, x=addr, x_permuted=addr, expert_weights=addr, router_weights=addr)
    assert rr.get_chain_workspace_size(chain) == (8 + 2 * 4) * 4
    assert rr.chain_from_logits(chain, ctx).code == S.kInsufficientWorkspace
    assert rr.chain_from_tokens(rr.ChainArgs(tokens=0, experts=8), ctx).ok()
    # N = 0: y, y_permuted and the expert weights have no elements (null is
    # accepted); the call reaches the workspace check
    chain = rr.ChainArgs(tokens=4, experts=8, hidden=4, output=0, logits=addr, expert_ids=addr,
                         route_weights=addr, counts=addr, offsets=addr, route_pos=addr, x=addr,
                         x_permuted=addr, router_weights=addr)
    assert rr.chain_from_tokens(chain, ctx).code == S.kInsufficientWorkspace

    # post-route chain: stage limits 1 <= top_k <= E <= 1024, top_k <= 64
    for bad in (dict(top_k=0), dict(top_k=9, experts=8), dict(experts=0), dict(experts=1025),
                dict(top_k=65, experts=128), dict(hidden=-1), dict(output=-1), dict(tokens=-1),
                dict(tokens=2**28, top_k=8)):
        route = rr.RouteChainArgs(**({"tokens": 4, "experts": 8, "top_k": 2, "hidden": 4, "output": 4} | bad))
        assert rr.chain_from_route_ids(route, ctx).code == S.kInvalidArgument, bad
    route = rr.RouteChainArgs(tokens=4, experts=8, top_k=8, hidden=4, output=4)
    assert rr.chain_from_route_ids(route, ctx).code == S.kInvalidArgument  # null pointers
    route = rr.RouteChainArgs(tokens=4, experts=8, top_k=8, hidden=4, output=4, x=addr, expert_ids=addr,
                              route_weights=addr, expert_weights=addr, counts=addr, offsets=addr,
                              route_pos=addr, y_permuted=addr, y=addr)
    assert rr.get_route_chain_workspace_size(route) == (8 + 4 * 8) * 4
    assert rr.chain_from_route_ids(route, ctx).code == S.kInsufficientWorkspace
    assert rr.chain_from_route_ids(rr.RouteChainArgs(tokens=0, experts=8, top_k=4), ctx).ok()
    route = rr.RouteChainArgs(tokens=4, experts=8, top_k=2, hidden=4, output=0, x=addr, expert_ids=addr,
                              counts=addr, offsets=addr, route_pos=addr)
    assert rr.chain_from_route_ids(route, ctx).code == S.kInsufficientWorkspace
    route.hidden = 0
    route.x = None
    assert rr.chain_from_route_ids(route, ctx).code == S.kInsufficientWorkspace
    assert rr.get_route_chain_workspace_size(rr.RouteChainArgs(experts=8, top_k=0)) == 0


def test_naive_launchers_zero_size_contract():
    # reference tests/correctness_framework_tests.cpp:236-250
    ops = rr.ops
    assert ops.launch_dense_gemm_naive(None, None, None, 0, 5, 3) == 0
    assert ops.launch_topk_gate_naive(None, None, None, 0, 8) == 0
    assert ops.launch_token_permute_naive(None, None, None, None, None, None, None, 0, 2, 7) == 0
    assert ops.launch_grouped_gemm_naive(None, None, None, None, 4, 7, 5, 0) == 0
    assert ops.launch_unpermute_naive(None, None, None, None, 0, 2, 7) == 0
    assert ops.launch_histogram_naive(None, None, 0, 4) == 0
    assert ops.launch_topk_gate_naive(None, None, None, 1, 1) != 0  # E = 1 rejected
    assert ops.launch_exclusive_scan_naive(None, None, 0) != 0


def test_cpp_consumer_compiles_links_and_runs(tmp_path):
    exe = tmp_path / "consumer"
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    lib_dir = rr.LIB_PATH.parent
    cmd = ["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{REPO / 'include'}", f"-I{rocm}/include", str(REPO / "tests" / "cpp" / "consumer.cpp"),
           f"-L{lib_dir}", "-lraggedroute_amd", f"-Wl,-rpath,{lib_dir}", f"-L{rocm}/lib", "-lamdhip64",
           f"-Wl,-rpath,{rocm}/lib", "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0 and "consumer OK" in run.stdout, run.stdout + run.stderr


def test_chain_graph_argument_checks_before_capture():
    """Graph entries reject bad calls before any device work: a null handle
    slot, no args, a call count outside [1, 4096], an unknown entry, the
    default stream and the naive family (memset resets stay out of graphs)."""
    import ctypes
    handle = ctypes.c_void_p()
    ctx = rr.RuntimeContext(stream=0x1234, architecture=GFX950)
    args = rr.ChainArgs(tokens=4, experts=4, hidden=8, output=8)
    one = (ctypes.c_void_p * 1)(ctypes.addressof(args))
    bad = [
        rr.lib.rr_chain_graph_create_sequence(rr.CHAIN_FROM_TOKENS, one, 0, ctypes.byref(ctx), ctypes.byref(handle)),
        rr.lib.rr_chain_graph_create_sequence(rr.CHAIN_FROM_TOKENS, None, 1, ctypes.byref(ctx), ctypes.byref(handle)),
        rr.lib.rr_chain_graph_create_sequence(rr.CHAIN_FROM_TOKENS, one, 4097, ctypes.byref(ctx), ctypes.byref(handle)),
        rr.lib.rr_chain_graph_create_sequence(7, one, 1, ctypes.byref(ctx), ctypes.byref(handle)),
        rr.lib.rr_chain_graph_create_sequence(rr.CHAIN_FROM_TOKENS, one, 1,
                                              ctypes.byref(rr.RuntimeContext(architecture=GFX950)),
                                              ctypes.byref(handle)),
        rr.lib.rr_chain_graph_create_sequence(rr.CHAIN_FROM_TOKENS, one, 1, ctypes.byref(ctx), None),
    ]
    naive = rr.ChainArgs(tokens=4, experts=4, hidden=8, output=8, kernel=rr.kernel(rr.KernelFamily.kNaive))
    bad.append(rr.lib.rr_chain_graph_create_sequence(
        rr.CHAIN_FROM_TOKENS, (ctypes.c_void_p * 1)(ctypes.addressof(naive)), 1, ctypes.byref(ctx),
        ctypes.byref(handle)))
    for st in bad:
        assert st.code == rr.StatusCode.kInvalidArgument, st
    assert not handle.value
    st = rr.lib.rr_chain_graph_update_sequence(None, one, 1, ctypes.byref(ctx))
    assert st.code == rr.StatusCode.kInvalidArgument
