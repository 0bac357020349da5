"""RaggedRoute routing pipeline for AMD MI355X (gfx950).

Python mirror of the C++ v0.2 operator API (reference
include/raggedroute/operators.h:114-135, dispatch.h:32-46, baseline_ops.h:14-42)
over the C ABI of libraggedroute_amd.so. All compute runs in the HIP library;
this module only marshals arguments. Importing it loads the library and fails
loudly when it is missing or incomplete: there is no fallback path.

Device memory comes from the caller (for example torch tensors on a ROCm
device); pass raw device pointers (``tensor.data_ptr()``) and the HIP stream
handle (``torch.cuda.current_stream().cuda_stream``).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import byref

# One HIP runtime serves a process: the library binds whichever
# libamdhip64.so.7 is loaded first. PyTorch-ROCm wheels bundle their own, and a
# torch built for another ROCm release stops seeing the GPU when the system
# runtime was loaded before it (the library works on either), so torch, when
# installed, is loaded before the library.
try:
    import torch  # noqa: F401
except ImportError:  # the library does not need it
    pass
from pathlib import Path

from ._capi import (  # noqa: F401  (re-exported vocabulary)
    GFX950_NATIVE,
    MAX_EXPERTS,
    PROTOTYPES,
    CHAIN_FROM_LOGITS,
    CHAIN_FROM_ROUTE_IDS,
    CHAIN_FROM_TOKENS,
    ChainArgs,
    ChainGraphCacheStats,
    ConstTensorView,
    DenseGemmArgs,
    DeviceArchitecture,
    DispatchDecision,
    DispatchRequest,
    ExclusiveScanArgs,
    GroupedGemmArgs,
    HistogramArgs,
    HistogramExclusiveScanArgs,
    KernelFamily,
    KernelSelection,
    MutableTensorView,
    OperatorKind,
    OperatorSignature,
    RouteChainArgs,
    RouteTraceInfo,
    RuntimeContext,
    ScalarType,
    Status,
    StatusCode,
    TensorLayout,
    TensorSpec,
    TokenPermuteArgs,
    TopKGateArgs,
    UnpermuteArgs,
    bind,
)

# RR_LIBRARY names another build of the same library to load instead (the
# host-sanitizer run of tests/sanitize.sh loads its instrumented build).
LIB_PATH = Path(os.environ.get("RR_LIBRARY") or Path(__file__).resolve().parent / "libraggedroute_amd.so")


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python raggedroute_amd/build.py` "
            "(there is no non-HIP fallback)"
        )
    return bind(ctypes.CDLL(str(LIB_PATH)))


lib = _load()


def _ctx(context: RuntimeContext | None) -> RuntimeContext:
    return context if context is not None else RuntimeContext()


# ---- operator wrappers (reference include/raggedroute/operators.h:127-135) ----

def dense_gemm(args: DenseGemmArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_dense_gemm(byref(args), byref(_ctx(context)))


def topk_gate(args: TopKGateArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_topk_gate(byref(args), byref(_ctx(context)))


def histogram(args: HistogramArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_histogram(byref(args), byref(_ctx(context)))


def exclusive_scan(args: ExclusiveScanArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_exclusive_scan(byref(args), byref(_ctx(context)))


def histogram_exclusive_scan(args: HistogramExclusiveScanArgs,
                             context: RuntimeContext | None = None) -> Status:
    return lib.rr_histogram_exclusive_scan(byref(args), byref(_ctx(context)))


def token_permute(args: TokenPermuteArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_token_permute(byref(args), byref(_ctx(context)))


def grouped_gemm(args: GroupedGemmArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_grouped_gemm(byref(args), byref(_ctx(context)))


def unpermute(args: UnpermuteArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_unpermute(byref(args), byref(_ctx(context)))


def chain_from_tokens(args: ChainArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_chain_from_tokens(byref(args), byref(_ctx(context)))


def chain_from_tokens_noalloc(args: ChainArgs, context: RuntimeContext | None = None) -> Status:
    """chain_from_tokens with the workspace in the library's static device
    scratch (context.workspace is ignored)."""
    return lib.rr_chain_from_tokens_noalloc(byref(args), byref(_ctx(context)))


def chain_from_logits(args: ChainArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_chain_from_logits(byref(args), byref(_ctx(context)))


def chain_from_route_ids(args: RouteChainArgs, context: RuntimeContext | None = None) -> Status:
    return lib.rr_chain_from_route_ids(byref(args), byref(_ctx(context)))


def get_route_chain_workspace_size(args: RouteChainArgs) -> int:
    return lib.rr_route_chain_workspace_size(byref(args))


def chain_fused_launch(args: ChainArgs, context: RuntimeContext | None, from_tokens: bool,
                       launch: int) -> Status:
    """One launch of the fused chain alone (numbered in execution order), for
    per-launch timing."""
    return lib.rr_chain_fused_launch(byref(args), byref(_ctx(context)), int(bool(from_tokens)), launch)


def chain_fused_launch_names(args: ChainArgs, from_tokens: bool) -> list[str]:
    """Names of the fused chain's launches for this shape, in execution order."""
    names = []
    while True:
        name = lib.rr_chain_fused_launch_name(byref(args), int(bool(from_tokens)), len(names))
        if name is None:
            return names
        names.append(name.decode())


# ---- chain graphs (rr_chain_graph_*, rr_chain_graph_cache_*) ----

def _arg_pointers(args):
    return (ctypes.c_void_p * len(args))(*[ctypes.addressof(a) for a in args])


class ChainGraph:
    """Chain calls captured into one executable HIP graph. `entry` is
    CHAIN_FROM_TOKENS / CHAIN_FROM_LOGITS (ChainArgs) or CHAIN_FROM_ROUTE_IDS
    (RouteChainArgs); `args` is one args struct or a list of them (recorded
    in order, replayed by one launch). Raises RuntimeError with the library's
    message when the calls cannot be captured."""

    def __init__(self, entry: int, args, context: RuntimeContext):
        self._handle = ctypes.c_void_p()
        self.entry = entry
        if isinstance(args, (list, tuple)):
            ptrs = _arg_pointers(args)
            st = lib.rr_chain_graph_create_sequence(entry, ptrs, len(args), byref(context), byref(self._handle))
        else:
            st = lib.rr_chain_graph_create(entry, ctypes.addressof(args), byref(context), byref(self._handle))
        if not st.ok():
            raise RuntimeError(st.message)

    def launch(self, stream) -> Status:
        return lib.rr_chain_graph_launch(self._handle, stream)

    def update(self, args, context: RuntimeContext) -> Status:
        if isinstance(args, (list, tuple)):
            return lib.rr_chain_graph_update_sequence(self._handle, _arg_pointers(args), len(args), byref(context))
        return lib.rr_chain_graph_update(self._handle, ctypes.addressof(args), byref(context))

    @property
    def kernel_nodes(self) -> int:
        return lib.rr_chain_graph_kernel_nodes(self._handle)

    def close(self) -> None:
        if self._handle:
            lib.rr_chain_graph_destroy(self._handle)
            self._handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()


class ChainGraphCache:
    """LRU cache of chain graphs keyed by the whole call (capacity 16 like the
    reference's graph cache)."""

    def __init__(self, capacity: int = 16):
        self._handle = ctypes.c_void_p()
        st = lib.rr_chain_graph_cache_create(capacity, byref(self._handle))
        if not st.ok():
            raise RuntimeError(st.message)

    def launch(self, entry: int, args, context: RuntimeContext) -> Status:
        return lib.rr_chain_graph_cache_launch(self._handle, entry, ctypes.addressof(args), byref(context))

    def stats(self) -> ChainGraphCacheStats:
        out = ChainGraphCacheStats()
        lib.rr_chain_graph_cache_get_stats(self._handle, byref(out))
        return out

    def close(self) -> None:
        if self._handle:
            lib.rr_chain_graph_cache_destroy(self._handle)
            self._handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()


# ---- workspace queries (reference operators.h:114-122) ----

def get_dense_gemm_workspace_size(args: DenseGemmArgs) -> int:
    return lib.rr_dense_gemm_workspace_size(byref(args))


def get_topk_gate_workspace_size(args: TopKGateArgs) -> int:
    return lib.rr_topk_gate_workspace_size(byref(args))


def get_histogram_workspace_size(args: HistogramArgs) -> int:
    return lib.rr_histogram_workspace_size(byref(args))


def get_exclusive_scan_workspace_size(args: ExclusiveScanArgs) -> int:
    return lib.rr_exclusive_scan_workspace_size(byref(args))


def get_histogram_exclusive_scan_workspace_size(args: HistogramExclusiveScanArgs) -> int:
    return lib.rr_histogram_exclusive_scan_workspace_size(byref(args))


def get_token_permute_workspace_size(args: TokenPermuteArgs) -> int:
    return lib.rr_token_permute_workspace_size(byref(args))


def get_grouped_gemm_workspace_size(args: GroupedGemmArgs) -> int:
    return lib.rr_grouped_gemm_workspace_size(byref(args))


def get_unpermute_workspace_size(args: UnpermuteArgs) -> int:
    return lib.rr_unpermute_workspace_size(byref(args))


def get_chain_workspace_size(args: ChainArgs) -> int:
    return lib.rr_chain_workspace_size(byref(args))


# ---- dispatch (reference include/raggedroute/dispatch.h:32-46) ----

def classify_compute_capability(major: int, minor: int) -> DeviceArchitecture:
    return DeviceArchitecture(lib.rr_classify_compute_capability(major, minor))


def classify_gcn_arch_name(name: str) -> DeviceArchitecture:
    return DeviceArchitecture(lib.rr_classify_gcn_arch_name(name.encode()))


def query_current_device_architecture() -> tuple[Status, DeviceArchitecture]:
    out = ctypes.c_int32(0)
    status = lib.rr_query_current_device_architecture(byref(out))
    return status, DeviceArchitecture(out.value) if status.ok() else DeviceArchitecture.kOther


def resolve_device_architecture(requested: DeviceArchitecture) -> tuple[Status, DeviceArchitecture]:
    out = ctypes.c_int32(0)
    status = lib.rr_resolve_device_architecture(int(requested), byref(out))
    return status, DeviceArchitecture(out.value) if status.ok() else DeviceArchitecture.kOther


def select_kernel(request: DispatchRequest, decision: DispatchDecision | None) -> Status:
    return lib.rr_select_kernel(byref(request), byref(decision) if decision is not None else None)


# ---- low-level launchers (reference include/raggedroute/baseline_ops.h:14-42) ----

class ops:  # noqa: N801  (mirrors the reference namespace raggedroute::ops)
    """Naive HIP baselines: reference semantics, no resets, hipError_t results."""

    @staticmethod
    def launch_dense_gemm_naive(a, b, c, m, n, k, stream=None) -> int:
        return lib.rr_launch_dense_gemm_naive(a, b, c, m, n, k, stream)

    @staticmethod
    def launch_topk_gate_naive(logits, expert_ids, weights, tokens, experts, stream=None) -> int:
        return lib.rr_launch_topk_gate_naive(logits, expert_ids, weights, tokens, experts, stream)

    @staticmethod
    def launch_histogram_naive(expert_ids, counts, route_pairs, experts, stream=None) -> int:
        return lib.rr_launch_histogram_naive(expert_ids, counts, route_pairs, experts, stream)

    @staticmethod
    def launch_exclusive_scan_naive(counts, offsets, experts, stream=None) -> int:
        return lib.rr_launch_exclusive_scan_naive(counts, offsets, experts, stream)

    @staticmethod
    def launch_token_permute_naive(x, expert_ids, offsets, cursors, x_permuted, route_pos,
                                   sorted_route, tokens, top_k, hidden, stream=None) -> int:
        return lib.rr_launch_token_permute_naive(x, expert_ids, offsets, cursors, x_permuted,
                                                 route_pos, sorted_route, tokens, top_k, hidden,
                                                 stream)

    @staticmethod
    def launch_grouped_gemm_naive(x_permuted, expert_weights, offsets, y_permuted, experts,
                                  hidden, output, max_expert_tokens, stream=None) -> int:
        return lib.rr_launch_grouped_gemm_naive(x_permuted, expert_weights, offsets, y_permuted,
                                                experts, hidden, output, max_expert_tokens, stream)

    @staticmethod
    def launch_unpermute_naive(y_permuted, route_pos, route_weights, y, tokens, top_k, output,
                               stream=None) -> int:
        return lib.rr_launch_unpermute_naive(y_permuted, route_pos, route_weights, y, tokens,
                                             top_k, output, stream)

    @staticmethod
    def launch_cache_scrub(buffer, elements, stream=None) -> int:
        return lib.rr_launch_cache_scrub(buffer, elements, stream)


def fill_uniform(ptr, count, seed, stream_id, low, high, stream=None) -> int:
    return lib.rr_fill_uniform(ptr, count, seed, stream_id, low, high, stream)


def fill_normal(ptr, count, seed, stream_id, mean, stddev, stream=None) -> int:
    return lib.rr_fill_normal(ptr, count, seed, stream_id, mean, stddev, stream)


def kernel(family: KernelFamily = KernelFamily.kAuto, implementation_id: int = 0) -> KernelSelection:
    return KernelSelection(int(family), implementation_id)


def cview(ptr) -> ConstTensorView:
    """FP32 row-major view of a device pointer (int or None)."""
    return ConstTensorView(ptr, TensorSpec())


def mview(ptr) -> MutableTensorView:
    return MutableTensorView(ptr, TensorSpec())
