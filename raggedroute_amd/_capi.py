"""ctypes mirror of include/raggedroute_capi.h.

Struct layouts, enum ordinals and function prototypes follow the C header one
to one. The names mirror the reference C++ v0.2 API (reference
include/raggedroute/{types,status,runtime,operators,dispatch}.h) so that tests
written against this module read like the reference's own operator tests.
"""
from __future__ import annotations

import ctypes
import enum
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

i32p = POINTER(c_int32)


class OperatorKind(enum.IntEnum):
    kDenseGemm = 0
    kTopKGate = 1
    kHistogram = 2
    kExclusiveScan = 3
    kTokenPermute = 4
    kGroupedGemm = 5
    kUnpermute = 6
    kHistogramExclusiveScan = 7


class DeviceArchitecture(enum.IntEnum):
    kAuto = 0
    kSm86 = 1
    kSm90 = 2
    kOther = 3
    kGfx950 = 4


class KernelFamily(enum.IntEnum):
    kAuto = 0
    kNaive = 1
    kOptimized = 2


class ScalarType(enum.IntEnum):
    kFp32 = 0
    kFp16 = 1
    kBf16 = 2
    kFp8E4M3 = 3
    kFp8E5M2 = 4
    kFp6E2M3 = 5
    kFp6E3M2 = 6
    kFp4E2M1 = 7


class TensorLayout(enum.IntEnum):
    kRowMajorContiguous = 0
    kColumnMajorContiguous = 1
    kStrided = 2


class StatusCode(enum.IntEnum):
    kSuccess = 0
    kInvalidArgument = 1
    kUnsupportedArchitecture = 2
    kUnsupportedDataType = 3
    kUnsupportedLayout = 4
    kUnsupportedKernelVariant = 5
    kInsufficientWorkspace = 6
    kDeviceError = 7


GFX950_NATIVE = 950
MAX_EXPERTS = 1024


class TensorSpec(ctypes.Structure):
    _fields_ = [("dtype", c_int32), ("layout", c_int32), ("strides", c_int64 * 3)]


class ConstTensorView(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("spec", TensorSpec)]


class MutableTensorView(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("spec", TensorSpec)]


class KernelSelection(ctypes.Structure):
    _fields_ = [("family", c_int32), ("implementation_id", c_uint32)]


class RuntimeContext(ctypes.Structure):
    _fields_ = [
        ("stream", c_void_p),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("architecture", c_int32),
    ]


class Status(ctypes.Structure):
    _fields_ = [("code", c_int32), ("hip_error", c_int32), ("message_", c_char_p)]

    @property
    def message(self) -> str:
        return self.message_.decode() if self.message_ else ""

    def ok(self) -> bool:
        return self.code == StatusCode.kSuccess

    def __repr__(self) -> str:  # pragma: no cover - debugging aid
        return f"Status({StatusCode(self.code).name}, hip_error={self.hip_error}, {self.message!r})"


class DenseGemmArgs(ctypes.Structure):
    _fields_ = [
        ("a", ConstTensorView),
        ("b", ConstTensorView),
        ("c", MutableTensorView),
        ("m", c_int32),
        ("n", c_int32),
        ("k", c_int32),
        ("alpha", c_float),
        ("beta", c_float),
        ("accumulator_dtype", c_int32),
        ("kernel", KernelSelection),
    ]

    def __init__(self, **kw):
        super().__init__(alpha=1.0, beta=0.0, **kw)


class TopKGateArgs(ctypes.Structure):
    _fields_ = [
        ("logits", ConstTensorView),
        ("expert_ids", c_void_p),
        ("weights", MutableTensorView),
        ("tokens", c_int32),
        ("experts", c_int32),
        ("top_k", c_int32),
        ("accumulator_dtype", c_int32),
        ("normalization", c_int32),
        ("tie_break", c_int32),
        ("nan_policy", c_int32),
        ("kernel", KernelSelection),
    ]

    def __init__(self, **kw):
        kw.setdefault("top_k", 2)
        super().__init__(**kw)


class HistogramArgs(ctypes.Structure):
    _fields_ = [
        ("expert_ids", c_void_p),
        ("counts", c_void_p),
        ("route_pairs", c_int32),
        ("experts", c_int32),
        ("kernel", KernelSelection),
    ]


class ExclusiveScanArgs(ctypes.Structure):
    _fields_ = [
        ("counts", c_void_p),
        ("offsets", c_void_p),
        ("experts", c_int32),
        ("kernel", KernelSelection),
    ]


class HistogramExclusiveScanArgs(ctypes.Structure):
    _fields_ = [
        ("expert_ids", c_void_p),
        ("counts", c_void_p),
        ("offsets", c_void_p),
        ("route_pairs", c_int32),
        ("experts", c_int32),
        ("kernel", KernelSelection),
    ]


class TokenPermuteArgs(ctypes.Structure):
    _fields_ = [
        ("x", ConstTensorView),
        ("expert_ids", c_void_p),
        ("offsets", c_void_p),
        ("x_permuted", MutableTensorView),
        ("route_pos", c_void_p),
        ("sorted_route", c_void_p),
        ("tokens", c_int32),
        ("experts", c_int32),
        ("top_k", c_int32),
        ("hidden", c_int32),
        ("kernel", KernelSelection),
    ]


class GroupedGemmArgs(ctypes.Structure):
    _fields_ = [
        ("x_permuted", ConstTensorView),
        ("expert_weights", ConstTensorView),
        ("offsets", c_void_p),
        ("y_permuted", MutableTensorView),
        ("experts", c_int32),
        ("hidden", c_int32),
        ("output", c_int32),
        ("max_expert_tokens", c_int32),
        ("accumulator_dtype", c_int32),
        ("kernel", KernelSelection),
    ]


class UnpermuteArgs(ctypes.Structure):
    _fields_ = [
        ("y_permuted", ConstTensorView),
        ("route_pos", c_void_p),
        ("route_weights", ConstTensorView),
        ("y", MutableTensorView),
        ("tokens", c_int32),
        ("top_k", c_int32),
        ("output", c_int32),
        ("accumulator_dtype", c_int32),
        ("kernel", KernelSelection),
    ]


class RouteTraceInfo(ctypes.Structure):
    _fields_ = [
        ("tokens", c_int32),
        ("experts", c_int32),
        ("top_k", c_int32),
        ("frame_count", c_int32),
        ("trace_id", ctypes.c_char * 128),
        ("source_kind", ctypes.c_char * 32),
        ("frame_id", ctypes.c_char * 128),
    ]


class ChainGraphCacheStats(ctypes.Structure):
    _fields_ = [("capacity", c_int32), ("entries", c_int32), ("hits", c_int64), ("misses", c_int64)]


CHAIN_FROM_TOKENS, CHAIN_FROM_LOGITS, CHAIN_FROM_ROUTE_IDS = 0, 1, 2


class RouteChainArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p),
        ("expert_ids", c_void_p),
        ("route_weights", c_void_p),
        ("expert_weights", c_void_p),
        ("counts", c_void_p),
        ("offsets", c_void_p),
        ("x_permuted", c_void_p),
        ("route_pos", c_void_p),
        ("sorted_route", c_void_p),
        ("y_permuted", c_void_p),
        ("y", c_void_p),
        ("tokens", c_int32),
        ("experts", c_int32),
        ("top_k", c_int32),
        ("hidden", c_int32),
        ("output", c_int32),
        ("kernel", KernelSelection),
    ]

    def __init__(self, **kw):
        kw.setdefault("top_k", 2)
        super().__init__(**kw)


class ChainArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p),
        ("router_weights", c_void_p),
        ("logits", c_void_p),
        ("expert_ids", c_void_p),
        ("route_weights", c_void_p),
        ("counts", c_void_p),
        ("offsets", c_void_p),
        ("x_permuted", c_void_p),
        ("route_pos", c_void_p),
        ("sorted_route", c_void_p),
        ("expert_weights", c_void_p),
        ("y_permuted", c_void_p),
        ("y", c_void_p),
        ("tokens", c_int32),
        ("experts", c_int32),
        ("top_k", c_int32),
        ("hidden", c_int32),
        ("output", c_int32),
        ("kernel", KernelSelection),
    ]

    def __init__(self, **kw):
        kw.setdefault("top_k", 2)
        super().__init__(**kw)


class OperatorSignature(ctypes.Structure):
    _fields_ = [
        ("has_input", c_int32),
        ("input", TensorSpec),
        ("has_weight", c_int32),
        ("weight", TensorSpec),
        ("has_accumulator", c_int32),
        ("accumulator", c_int32),
        ("has_output", c_int32),
        ("output", TensorSpec),
    ]


class DispatchRequest(ctypes.Structure):
    _fields_ = [
        ("operator_kind", c_int32),
        ("architecture", c_int32),
        ("requested_kernel", KernelSelection),
        ("signature", OperatorSignature),
    ]


class DispatchDecision(ctypes.Structure):
    _fields_ = [
        ("operator_kind", c_int32),
        ("architecture", c_int32),
        ("kernel", KernelSelection),
    ]


# (name, restype, argtypes) of every symbol declared in include/raggedroute_capi.h.
_OP_ENTRIES = [
    ("dense_gemm", DenseGemmArgs),
    ("topk_gate", TopKGateArgs),
    ("histogram", HistogramArgs),
    ("exclusive_scan", ExclusiveScanArgs),
    ("histogram_exclusive_scan", HistogramExclusiveScanArgs),
    ("token_permute", TokenPermuteArgs),
    ("grouped_gemm", GroupedGemmArgs),
    ("unpermute", UnpermuteArgs),
]

PROTOTYPES: list[tuple[str, object, list]] = []
for _name, _args in _OP_ENTRIES:
    PROTOTYPES.append((f"rr_{_name}_workspace_size", c_size_t, [POINTER(_args)]))
    PROTOTYPES.append((f"rr_{_name}", Status, [POINTER(_args), POINTER(RuntimeContext)]))
PROTOTYPES += [
    ("rr_chain_workspace_size", c_size_t, [POINTER(ChainArgs)]),
    ("rr_chain_from_tokens", Status, [POINTER(ChainArgs), POINTER(RuntimeContext)]),
    ("rr_chain_from_tokens_noalloc", Status, [POINTER(ChainArgs), POINTER(RuntimeContext)]),
    ("rr_chain_from_logits", Status, [POINTER(ChainArgs), POINTER(RuntimeContext)]),
    ("rr_chain_fused_launch", Status, [POINTER(ChainArgs), POINTER(RuntimeContext), c_int32, c_int32]),
    ("rr_chain_from_route_ids", Status, [POINTER(RouteChainArgs), POINTER(RuntimeContext)]),
    ("rr_chain_graph_create", Status, [c_int32, c_void_p, POINTER(RuntimeContext), POINTER(c_void_p)]),
    ("rr_chain_graph_launch", Status, [c_void_p, c_void_p]),
    ("rr_chain_graph_update", Status, [c_void_p, c_void_p, POINTER(RuntimeContext)]),
    ("rr_chain_graph_create_sequence", Status,
     [c_int32, POINTER(c_void_p), c_int32, POINTER(RuntimeContext), POINTER(c_void_p)]),
    ("rr_chain_graph_update_sequence", Status, [c_void_p, POINTER(c_void_p), c_int32, POINTER(RuntimeContext)]),
    ("rr_chain_graph_kernel_nodes", c_int32, [c_void_p]),
    ("rr_chain_graph_destroy", None, [c_void_p]),
    ("rr_chain_graph_cache_create", Status, [c_int32, POINTER(c_void_p)]),
    ("rr_chain_graph_cache_launch", Status, [c_void_p, c_int32, c_void_p, POINTER(RuntimeContext)]),
    ("rr_chain_graph_cache_get_stats", None, [c_void_p, POINTER(ChainGraphCacheStats)]),
    ("rr_chain_graph_cache_destroy", None, [c_void_p]),
    ("rr_route_trace_read", Status, [ctypes.c_char_p, c_int32, POINTER(RouteTraceInfo), c_void_p, c_size_t]),
    ("rr_route_chain_workspace_size", c_size_t, [POINTER(RouteChainArgs)]),
    ("rr_chain_fused_launch_name", c_char_p, [POINTER(ChainArgs), c_int32, c_int32]),
    ("rr_classify_compute_capability", c_int32, [c_int32, c_int32]),
    ("rr_classify_gcn_arch_name", c_int32, [c_char_p]),
    ("rr_query_current_device_architecture", Status, [i32p]),
    ("rr_resolve_device_architecture", Status, [c_int32, i32p]),
    ("rr_select_kernel", Status, [POINTER(DispatchRequest), POINTER(DispatchDecision)]),
    ("rr_launch_dense_gemm_naive", c_int32,
     [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    ("rr_launch_topk_gate_naive", c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    ("rr_launch_histogram_naive", c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    ("rr_launch_exclusive_scan_naive", c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    ("rr_launch_token_permute_naive", c_int32,
     [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
      c_int32, c_void_p]),
    ("rr_launch_grouped_gemm_naive", c_int32,
     [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p]),
    ("rr_launch_unpermute_naive", c_int32,
     [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    ("rr_launch_cache_scrub", c_int32, [c_void_p, c_size_t, c_void_p]),
    ("rr_fill_uniform", c_int32, [c_void_p, c_size_t, c_uint64, c_uint64, c_float, c_float, c_void_p]),
    ("rr_fill_normal", c_int32, [c_void_p, c_size_t, c_uint64, c_uint64, c_float, c_float, c_void_p]),
    ("rr_capi_version", c_int32, []),
    ("rr_build_target", c_char_p, []),
]


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    """Attach restype/argtypes to every exported entry; raises if one is missing."""
    for name, restype, argtypes in PROTOTYPES:
        fn = getattr(lib, name)  # AttributeError when the symbol is absent
        fn.restype = restype
        fn.argtypes = argtypes
    return lib
