/*
 * raggedroute_capi.h - C ABI of the MI355X (gfx950) RaggedRoute routing library.
 *
 * This is the drop-in boundary. Every entry point is `extern "C"`, takes plain
 * POD structs (pointers, sizes, int32 enums) and returns an `rr_status` by
 * value. Nothing here allocates, throws or synchronises the caller's stream.
 * The C++ v0.2 surface under include/raggedroute/ is a set of inline
 * forwarders over these functions.
 *
 * Every struct mirrors the field order of the reference C++ type it replaces
 * and every enum keeps the reference ordinals; the comment on each entry names
 * the reference interface (file:line under the reference checkout).
 *
 * Conventions shared by all operator entries:
 *   - non-null pointers are HIP device pointers unless a field says otherwise;
 *   - tensors are FP32, row-major, zero strides (v0.2 contract,
 *     reference include/raggedroute/operators.h:12-17);
 *   - expert counts are capped at RR_MAX_EXPERTS (the reference caps at 64);
 *   - resets the reference performs inside the call boundary (histogram
 *     counts, permute cursors) are performed here too.
 */
#ifndef RAGGEDROUTE_CAPI_H
#define RAGGEDROUTE_CAPI_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RR_CAPI_VERSION 2
/* Largest expert count any operator accepts (reference cap: 64). */
#define RR_MAX_EXPERTS 1024
/* Implementation id of the native gfx950 kernel of every operator. */
#define RR_IMPL_GFX950_NATIVE 950u

/* reference include/raggedroute/types.h:8-17 (OperatorKind) */
enum {
  RR_OP_DENSE_GEMM = 0,
  RR_OP_TOPK_GATE = 1,
  RR_OP_HISTOGRAM = 2,
  RR_OP_EXCLUSIVE_SCAN = 3,
  RR_OP_TOKEN_PERMUTE = 4,
  RR_OP_GROUPED_GEMM = 5,
  RR_OP_UNPERMUTE = 6,
  RR_OP_HISTOGRAM_EXCLUSIVE_SCAN = 7
};

/* reference include/raggedroute/types.h:21-26 (DeviceArchitecture), with
 * RR_ARCH_GFX950 appended after the reference ordinals. */
enum {
  RR_ARCH_AUTO = 0,
  RR_ARCH_SM86 = 1,
  RR_ARCH_SM90 = 2,
  RR_ARCH_OTHER = 3,
  RR_ARCH_GFX950 = 4
};

/* reference include/raggedroute/types.h:30-34 (KernelFamily); ordinals kept. */
enum { RR_FAMILY_AUTO = 0, RR_FAMILY_NAIVE = 1, RR_FAMILY_OPTIMIZED = 2 };

/* reference include/raggedroute/types.h:46-55 (ScalarType) */
enum {
  RR_DTYPE_FP32 = 0,
  RR_DTYPE_FP16 = 1,
  RR_DTYPE_BF16 = 2,
  RR_DTYPE_FP8_E4M3 = 3,
  RR_DTYPE_FP8_E5M2 = 4,
  RR_DTYPE_FP6_E2M3 = 5,
  RR_DTYPE_FP6_E3M2 = 6,
  RR_DTYPE_FP4_E2M1 = 7
};

/* reference include/raggedroute/types.h:57-61 (TensorLayout) */
enum { RR_LAYOUT_ROW_MAJOR = 0, RR_LAYOUT_COLUMN_MAJOR = 1, RR_LAYOUT_STRIDED = 2 };

/* reference include/raggedroute/types.h:83-95 (top-k policy enums; one value each) */
enum { RR_TOPK_SELECTED_SOFTMAX = 0 };
enum { RR_TOPK_TIE_LOWER_EXPERT_ID = 0 };
enum { RR_TOPK_NAN_NEG_INF_ALL_NAN_01 = 0 };

/* reference include/raggedroute/status.h:7-16 (StatusCode); RR_STATUS_DEVICE_ERROR
 * takes the ordinal of the reference's kCudaError. */
enum {
  RR_STATUS_SUCCESS = 0,
  RR_STATUS_INVALID_ARGUMENT = 1,
  RR_STATUS_UNSUPPORTED_ARCHITECTURE = 2,
  RR_STATUS_UNSUPPORTED_DATA_TYPE = 3,
  RR_STATUS_UNSUPPORTED_LAYOUT = 4,
  RR_STATUS_UNSUPPORTED_KERNEL_VARIANT = 5,
  RR_STATUS_INSUFFICIENT_WORKSPACE = 6,
  RR_STATUS_DEVICE_ERROR = 7
};

/* reference include/raggedroute/types.h:67-71 (TensorSpec) */
typedef struct rr_tensor_spec {
  int32_t dtype;
  int32_t layout;
  int64_t strides[3];
} rr_tensor_spec;

/* reference include/raggedroute/types.h:73-81 (ConstTensorView / MutableTensorView) */
typedef struct rr_const_tensor_view {
  const void* data;
  rr_tensor_spec spec;
} rr_const_tensor_view;

typedef struct rr_mutable_tensor_view {
  void* data;
  rr_tensor_spec spec;
} rr_mutable_tensor_view;

/* reference include/raggedroute/types.h:36-41 (KernelSelection) */
typedef struct rr_kernel_selection {
  int32_t family;
  uint32_t implementation_id;
} rr_kernel_selection;

/* reference include/raggedroute/runtime.h:13-18 (RuntimeContext) */
typedef struct rr_runtime_context {
  hipStream_t stream;
  void* workspace;
  size_t workspace_bytes;
  int32_t architecture;
} rr_runtime_context;

/* reference include/raggedroute/status.h:18-24 (Status). `message` always
 * points at a static string; `hip_error` replaces the reference cuda_error. */
typedef struct rr_status {
  int32_t code;
  int32_t hip_error;
  const char* message;
} rr_status;

/* reference include/raggedroute/operators.h:19-30 (DenseGemmArgs) */
typedef struct rr_dense_gemm_args {
  rr_const_tensor_view a;
  rr_const_tensor_view b;
  rr_mutable_tensor_view c;
  int32_t m;
  int32_t n;
  int32_t k;
  float alpha;
  float beta;
  int32_t accumulator_dtype;
  rr_kernel_selection kernel;
} rr_dense_gemm_args;

/* reference include/raggedroute/operators.h:32-44 (TopKGateArgs) */
typedef struct rr_topk_gate_args {
  rr_const_tensor_view logits;
  int32_t* expert_ids;
  rr_mutable_tensor_view weights;
  int32_t tokens;
  int32_t experts;
  int32_t top_k;
  int32_t accumulator_dtype;
  int32_t normalization;
  int32_t tie_break;
  int32_t nan_policy;
  rr_kernel_selection kernel;
} rr_topk_gate_args;

/* reference include/raggedroute/operators.h:46-52 (HistogramArgs) */
typedef struct rr_histogram_args {
  const int32_t* expert_ids;
  int32_t* counts;
  int32_t route_pairs;
  int32_t experts;
  rr_kernel_selection kernel;
} rr_histogram_args;

/* reference include/raggedroute/operators.h:54-59 (ExclusiveScanArgs) */
typedef struct rr_exclusive_scan_args {
  const int32_t* counts;
  int32_t* offsets;
  int32_t experts;
  rr_kernel_selection kernel;
} rr_exclusive_scan_args;

/* reference include/raggedroute/operators.h:61-70 (HistogramExclusiveScanArgs) */
typedef struct rr_histogram_exclusive_scan_args {
  const int32_t* expert_ids;
  int32_t* counts;
  int32_t* offsets;
  int32_t route_pairs;
  int32_t experts;
  rr_kernel_selection kernel;
} rr_histogram_exclusive_scan_args;

/* reference include/raggedroute/operators.h:72-85 (TokenPermuteArgs) */
typedef struct rr_token_permute_args {
  rr_const_tensor_view x;
  const int32_t* expert_ids;
  const int32_t* offsets;
  rr_mutable_tensor_view x_permuted;
  int32_t* route_pos;
  int32_t* sorted_route; /* optional inverse map: sorted_route[route_pos[r]] == r */
  int32_t tokens;
  int32_t experts;
  int32_t top_k;
  int32_t hidden;
  rr_kernel_selection kernel;
} rr_token_permute_args;

/* reference include/raggedroute/operators.h:87-100 (GroupedGemmArgs) */
typedef struct rr_grouped_gemm_args {
  rr_const_tensor_view x_permuted;
  rr_const_tensor_view expert_weights;
  const int32_t* offsets;
  rr_mutable_tensor_view y_permuted;
  int32_t experts;
  int32_t hidden;
  int32_t output;
  int32_t max_expert_tokens; /* caller launch bound; offsets are read on device only */
  int32_t accumulator_dtype;
  rr_kernel_selection kernel;
} rr_grouped_gemm_args;

/* reference include/raggedroute/operators.h:102-112 (UnpermuteArgs) */
typedef struct rr_unpermute_args {
  rr_const_tensor_view y_permuted;
  const int32_t* route_pos;
  rr_const_tensor_view route_weights;
  rr_mutable_tensor_view y;
  int32_t tokens;
  int32_t top_k;
  int32_t output;
  int32_t accumulator_dtype;
  rr_kernel_selection kernel;
} rr_unpermute_args;

/*
 * Chain arguments. The reference exposes chain_from_tokens / chain_from_logits
 * only as benchmark suites (reference benchmarks/adapters/chain_adapter.cpp:263-467);
 * this library adds them as entry points that enqueue every stage on the
 * caller's stream with no host synchronisation.
 *   chain_from_tokens: x, router_weights -> logits (output) -> ... -> y
 *   chain_from_logits: logits (input) -> ... -> y   (router_weights unused)
 */
typedef struct rr_chain_args {
  const float* x;              /* [tokens, hidden] */
  const float* router_weights; /* [hidden, experts] (chain_from_tokens only) */
  float* logits;               /* [tokens, experts]: output of tokens, input of logits */
  int32_t* expert_ids;         /* [tokens, 2] */
  float* route_weights;        /* [tokens, 2] */
  int32_t* counts;             /* [experts] */
  int32_t* offsets;            /* [experts + 1] */
  float* x_permuted;           /* [tokens * 2, hidden] */
  int32_t* route_pos;          /* [tokens * 2] */
  int32_t* sorted_route;       /* [tokens * 2], optional */
  const float* expert_weights; /* [experts, hidden, output] */
  float* y_permuted;           /* [tokens * 2, output] */
  float* y;                    /* [tokens, output] */
  int32_t tokens;
  int32_t experts;
  int32_t top_k; /* must be 2 */
  int32_t hidden;
  int32_t output;
  rr_kernel_selection kernel; /* applied to every stage */
} rr_chain_args;

/*
 * Post-route chain arguments: prepared route ids and weights -> histogram +
 * exclusive scan -> token permute -> grouped GEMM -> unpermute. The reference
 * runs this chain only as its chain_from_route_ids research suite (reference
 * benchmarks/adapters/postroute_chain_adapter.cpp:142-230 setup, :250-356
 * stages, :357-385 validation; top_k in {2, 4, 8}, top_k <= E).
 */
typedef struct rr_route_chain_args {
  const float* x;              /* [tokens, hidden] */
  const int32_t* expert_ids;   /* [tokens, top_k], each in [0, experts) */
  const float* route_weights;  /* [tokens, top_k] */
  const float* expert_weights; /* [experts, hidden, output] */
  int32_t* counts;             /* [experts] */
  int32_t* offsets;            /* [experts + 1] */
  float* x_permuted;           /* [tokens * top_k, hidden]; optional on the auto / optimized
                                  path (NULL: rows are gathered, not materialised) */
  int32_t* route_pos;          /* [tokens * top_k] */
  int32_t* sorted_route;       /* [tokens * top_k], optional */
  float* y_permuted;           /* [tokens * top_k, output] */
  float* y;                    /* [tokens, output] */
  int32_t tokens;
  int32_t experts;
  int32_t top_k; /* 1..8, <= experts */
  int32_t hidden;
  int32_t output;
  rr_kernel_selection kernel; /* applied to every stage */
} rr_route_chain_args;

/*
 * Route trace (.rrtrace text format v1; reference
 * include/raggedroute/benchmark/adapter_utils.h:250-256 RouteTraceFrame).
 */
typedef struct rr_route_trace_info {
  int32_t tokens;
  int32_t experts; /* 1..1024 (the reference caps traces at 64) */
  int32_t top_k;
  int32_t frame_count;
  char trace_id[128];   /* truncated copies, NUL-terminated */
  char source_kind[32]; /* production | captured | synthetic_fixture */
  char frame_id[128];   /* of the frame read */
} rr_route_trace_info;

/* reference include/raggedroute/operators.h:114-122 (get_*_workspace_size) */
size_t rr_dense_gemm_workspace_size(const rr_dense_gemm_args* args);
size_t rr_topk_gate_workspace_size(const rr_topk_gate_args* args);
size_t rr_histogram_workspace_size(const rr_histogram_args* args);
size_t rr_exclusive_scan_workspace_size(const rr_exclusive_scan_args* args);
size_t rr_histogram_exclusive_scan_workspace_size(const rr_histogram_exclusive_scan_args* args);
/* reference src/permute/operator.cpp:17-19: experts * sizeof(int32) cursor words */
size_t rr_token_permute_workspace_size(const rr_token_permute_args* args);
size_t rr_grouped_gemm_workspace_size(const rr_grouped_gemm_args* args);
size_t rr_unpermute_workspace_size(const rr_unpermute_args* args);
/* no reference counterpart (chain entries are new): (experts + 2 * tokens)
 * int32 words = permute cursors + sorted_route scratch for the fused path */
size_t rr_chain_workspace_size(const rr_chain_args* args);
/* no reference counterpart (new entry): (experts + tokens * top_k) int32
 * words = permute cursors + sorted_route scratch */
size_t rr_route_chain_workspace_size(const rr_route_chain_args* args);

/* reference include/raggedroute/operators.h:127 / src/dense_gemm/operator.cpp:18-58 */
rr_status rr_dense_gemm(const rr_dense_gemm_args* args, const rr_runtime_context* context);
/* reference include/raggedroute/operators.h:128 / src/topk_gate/operator.cpp:18-60 */
rr_status rr_topk_gate(const rr_topk_gate_args* args, const rr_runtime_context* context);
/* reference include/raggedroute/operators.h:129 / src/histogram/operator.cpp:20-57 */
rr_status rr_histogram(const rr_histogram_args* args, const rr_runtime_context* context);
/* reference include/raggedroute/operators.h:130 / src/scan/operator.cpp:51-74 */
rr_status rr_exclusive_scan(const rr_exclusive_scan_args* args, const rr_runtime_context* context);
/* reference include/raggedroute/operators.h:131-132 / src/scan/operator.cpp:84-134 */
rr_status rr_histogram_exclusive_scan(const rr_histogram_exclusive_scan_args* args,
                                      const rr_runtime_context* context);
/* reference include/raggedroute/operators.h:133 / src/permute/operator.cpp:22-83 */
rr_status rr_token_permute(const rr_token_permute_args* args, const rr_runtime_context* context);
/* reference include/raggedroute/operators.h:134 / src/grouped_gemm/operator.cpp:17-49 */
rr_status rr_grouped_gemm(const rr_grouped_gemm_args* args, const rr_runtime_context* context);
/* reference include/raggedroute/operators.h:135 / src/unpermute/operator.cpp:19-57 */
rr_status rr_unpermute(const rr_unpermute_args* args, const rr_runtime_context* context);

/* Chain entries: no reference counterpart as functions; they run the stage
 * sequence of reference benchmarks/adapters/chain_adapter.cpp:263-467.
 * Auto / optimized family: y is zeroed by the first launch and both weighted
 * routes of a token are added into it with hardware FP32 atomic adds, so y
 * must be coarse-grained device memory of the running GPU (hipMalloc or an
 * allocator on it); fine-grained, host, managed or peer-mapped memory is not
 * supported for y there (use RR_FAMILY_NAIVE). Two adds into zero per
 * element: deterministic, equal to the rank-order unpermute bit for bit. */
rr_status rr_chain_from_tokens(const rr_chain_args* args, const rr_runtime_context* context);
rr_status rr_chain_from_logits(const rr_chain_args* args, const rr_runtime_context* context);
/* No reference counterpart as a function: the stage sequence of the
 * reference's chain_from_route_ids suite (reference
 * benchmarks/adapters/postroute_chain_adapter.cpp:250-356). Auto / optimized:
 * route preparation + gathered expert GEMM in one launch where the strip
 * kernel covers the shape, then the rank-order unpermute; naive: the stage
 * operators one by one (x_permuted required). Output y within the reference's
 * tolerance (atol 1e-4, rtol 4e-5 * K * top_k, :381). */
rr_status rr_chain_from_route_ids(const rr_route_chain_args* args,
                                  const rr_runtime_context* context);
/* Replaces reference include/raggedroute/benchmark/adapter_utils.h:269-322
 * (load_route_trace_frame, behind --param route_trace_path / route_trace_frame).
 * Reads the .rrtrace text v1 file at `path` (layout: schema tag, trace id,
 * source kind, "T E top_k frames", then per frame its id and T * top_k expert
 * ids), checks every frame and copies frame `frame`'s ids (token-major, host
 * memory) into expert_ids only once the whole file checked out; expert_ids =
 * NULL fills `info` alone. A file that breaks the format, or a frame index past
 * the last, returns RR_STATUS_INVALID_ARGUMENT with a static message naming
 * the rule. Host-only: no device call. */
rr_status rr_route_trace_read(const char* path, int32_t frame, rr_route_trace_info* info,
                              int32_t* expert_ids, size_t capacity);
/*
 * Chain graphs. No reference counterpart as a library interface: the
 * reference's CUDA-graph chain variants (benchmarks/adapters/chain_adapter.cpp:
 * 730-826 fixed capture and exec update, :962-1000 LRU shape cache of 16;
 * postroute_chain_adapter.cpp the same for the post-route chain) as objects.
 * `args` points at an rr_chain_args (RR_CHAIN_FROM_TOKENS / _LOGITS) or an
 * rr_route_chain_args (RR_CHAIN_FROM_ROUTE_IDS). Capture validates the call
 * like the direct entry, records it on context->stream (must not be the
 * default stream; nothing runs) and instantiates it; only the auto /
 * optimized family is capturable. Kernel arguments are baked at capture: the
 * buffers must outlive the graph, their contents are read at each replay.
 * Not thread-safe.
 */
enum { RR_CHAIN_FROM_TOKENS = 0, RR_CHAIN_FROM_LOGITS = 1, RR_CHAIN_FROM_ROUTE_IDS = 2 };
typedef struct rr_chain_graph rr_chain_graph;
typedef struct rr_chain_graph_cache rr_chain_graph_cache;
typedef struct rr_chain_graph_cache_stats {
  int32_t capacity;
  int32_t entries;
  int64_t hits;
  int64_t misses;
} rr_chain_graph_cache_stats;

rr_status rr_chain_graph_create(int32_t entry, const void* args, const rr_runtime_context* context,
                                rr_chain_graph** graph);
/* The same for `count` calls of one entry (args[i] each an rr_chain_args or
 * rr_route_chain_args as `entry` says), recorded in order into one graph:
 * e.g. the chains of every MoE layer of a model step, replayed with one
 * hipGraphLaunch. 1 <= count <= 4096. One launch of a graph has a fixed cost
 * on ROCm (about 19 us host, 5 us GPU on MI355X with ROCm 7.2): graphs of ten
 * or more chains amortise it. */
rr_status rr_chain_graph_create_sequence(int32_t entry, const void* const* args, int32_t count,
                                         const rr_runtime_context* context, rr_chain_graph** graph);
rr_status rr_chain_graph_launch(rr_chain_graph* graph, hipStream_t stream);
/* Re-captures the graph's entry with new args (same entry) and updates the
 * executable in place (hipGraphExecUpdate); a changed launch plan is
 * instantiated anew. */
rr_status rr_chain_graph_update(rr_chain_graph* graph, const void* args,
                                const rr_runtime_context* context);
/* Update of a sequence graph: the same entry and count as captured. */
rr_status rr_chain_graph_update_sequence(rr_chain_graph* graph, const void* const* args, int32_t count,
                                         const rr_runtime_context* context);
int32_t rr_chain_graph_kernel_nodes(const rr_chain_graph* graph);
void rr_chain_graph_destroy(rr_chain_graph* graph);
/* Cache of executable graphs keyed by every pointer, size and kernel field of
 * the call plus workspace and architecture; a miss captures the call, evicting
 * the least recently used entry at capacity. */
rr_status rr_chain_graph_cache_create(int32_t capacity, rr_chain_graph_cache** cache);
rr_status rr_chain_graph_cache_launch(rr_chain_graph_cache* cache, int32_t entry, const void* args,
                                      const rr_runtime_context* context);
void rr_chain_graph_cache_get_stats(const rr_chain_graph_cache* cache, rr_chain_graph_cache_stats* stats);
void rr_chain_graph_cache_destroy(rr_chain_graph_cache* cache);

/* Static device scratch of rr_chain_from_tokens_noalloc: one copy per GPU,
 * held until the process ends. */
#define RR_CHAIN_NOALLOC_SCRATCH_BYTES (1u << 20)
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): rr_chain_from_tokens with the chain workspace taken from a fixed
 * RR_CHAIN_NOALLOC_SCRATCH_BYTES device array instead of context->workspace
 * (whose fields are ignored; stream and architecture are used). Shapes with
 * rr_chain_workspace_size(args) > RR_CHAIN_NOALLOC_SCRATCH_BYTES (experts +
 * 2 * tokens > 262144) are rejected with RR_STATUS_INVALID_ARGUMENT before any
 * device call. Calls no allocating routine. Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (several streams or threads) race
 * on it. Outputs equal rr_chain_from_tokens's bit for bit. */
rr_status rr_chain_from_tokens_noalloc(const rr_chain_args* args, const rr_runtime_context* context);

/* No reference counterpart: timing hook. Runs one launch of the fused
 * (auto / optimized) chain alone so that a profiler or benchmark can time it
 * with events on the context's stream. Launches are numbered in execution
 * order; their number (2 or 3) depends on the shape, and an index past the
 * last one returns RR_STATUS_INVALID_ARGUMENT. Launch 0 is the router GEMM +
 * top-2 gate (the gate only when from_tokens is 0) and zeroes y; the last
 * launch adds into y, so repeating it alone keeps accumulating. Same argument
 * checks as the chain. */
rr_status rr_chain_fused_launch(const rr_chain_args* args, const rr_runtime_context* context,
                                int32_t from_tokens, int32_t launch);
/* No reference counterpart: name of fused launch `launch` for this shape
 * ("router_gate", "gate", "route_prep", "expert_gemm",
 * "route_prep_expert_gemm"), or NULL past the last launch. */
const char* rr_chain_fused_launch_name(const rr_chain_args* args, int32_t from_tokens,
                                       int32_t launch);

/* ---- dispatch (reference include/raggedroute/dispatch.h:12-46) ---- */

/* reference include/raggedroute/dispatch.h:12-17 (OperatorSignature): each
 * optional role is present when its has_* flag is non-zero. */
typedef struct rr_operator_signature {
  int32_t has_input;
  rr_tensor_spec input;
  int32_t has_weight;
  rr_tensor_spec weight;
  int32_t has_accumulator;
  int32_t accumulator;
  int32_t has_output;
  rr_tensor_spec output;
} rr_operator_signature;

/* reference include/raggedroute/dispatch.h:19-24 (DispatchRequest) */
typedef struct rr_dispatch_request {
  int32_t operator_kind;
  int32_t architecture;
  rr_kernel_selection requested_kernel;
  rr_operator_signature signature;
} rr_dispatch_request;

/* reference include/raggedroute/dispatch.h:26-30 (DispatchDecision) */
typedef struct rr_dispatch_decision {
  int32_t operator_kind;
  int32_t architecture;
  rr_kernel_selection kernel;
} rr_dispatch_decision;

/* reference include/raggedroute/dispatch.h:32 / src/runtime/dispatch.cpp:82-86 */
int32_t rr_classify_compute_capability(int32_t major, int32_t minor);
/* gfx950 detection by gcnArchName; no reference counterpart (reference keys on CUDA CC) */
int32_t rr_classify_gcn_arch_name(const char* gcn_arch_name);
/* reference include/raggedroute/dispatch.h:36 / src/runtime/dispatch.cpp:88-107 */
rr_status rr_query_current_device_architecture(int32_t* architecture);
/* reference include/raggedroute/dispatch.h:40-41 / src/runtime/dispatch.cpp:109-119 */
rr_status rr_resolve_device_architecture(int32_t requested, int32_t* resolved);
/* reference include/raggedroute/dispatch.h:46 / src/runtime/dispatch.cpp:121-225 */
rr_status rr_select_kernel(const rr_dispatch_request* request, rr_dispatch_decision* decision);

/* ---- low-level launchers (reference include/raggedroute/baseline_ops.h:14-42) ----
 * Naive baselines with the reference semantics: no resets (the caller zeroes
 * histogram counts and permute cursors), caller stream, hipError_t result. */
hipError_t rr_launch_dense_gemm_naive(const float* a, const float* b, float* c, int32_t m,
                                      int32_t n, int32_t k, hipStream_t stream);
hipError_t rr_launch_topk_gate_naive(const float* logits, int32_t* expert_ids, float* weights,
                                     int32_t tokens, int32_t experts, hipStream_t stream);
hipError_t rr_launch_histogram_naive(const int32_t* expert_ids, int32_t* counts,
                                     int32_t route_pairs, int32_t experts, hipStream_t stream);
hipError_t rr_launch_exclusive_scan_naive(const int32_t* counts, int32_t* offsets,
                                          int32_t experts, hipStream_t stream);
hipError_t rr_launch_token_permute_naive(const float* x, const int32_t* expert_ids,
                                         const int32_t* offsets, int32_t* cursors,
                                         float* x_permuted, int32_t* route_pos,
                                         int32_t* sorted_route, int32_t tokens, int32_t top_k,
                                         int32_t hidden, hipStream_t stream);
hipError_t rr_launch_grouped_gemm_naive(const float* x_permuted, const float* expert_weights,
                                        const int32_t* offsets, float* y_permuted,
                                        int32_t experts, int32_t hidden, int32_t output,
                                        int32_t max_expert_tokens, hipStream_t stream);
hipError_t rr_launch_unpermute_naive(const float* y_permuted, const int32_t* route_pos,
                                     const float* route_weights, float* y, int32_t tokens,
                                     int32_t top_k, int32_t output, hipStream_t stream);
/* reference include/raggedroute/baseline_ops.h:40-41 / src/benchmark/cache_scrub.cu:17-50 */
hipError_t rr_launch_cache_scrub(uint32_t* buffer, size_t elements, hipStream_t stream);

/* ---- synthetic inputs (benchmark support; reference adapter_utils.h:197-248 role) ----
 * Counter-based SplitMix64 generator: element i of sub-stream s under seed
 * `seed` uses z = splitmix64(seed * 0x9E3779B97F4A7C15 + s * 0xD1B54A32D192ED03 + i).
 * Uniform: low + (high - low) * ((z >> 40) * 2^-24).
 * Normal: Box-Muller on two 24-bit uniforms from one z (u1 in (0,1], u2 in [0,1)),
 * scaled by stddev, plus mean. */
hipError_t rr_fill_uniform(float* out, size_t count, uint64_t seed, uint64_t stream_id,
                           float low, float high, hipStream_t stream);
hipError_t rr_fill_normal(float* out, size_t count, uint64_t seed, uint64_t stream_id,
                          float mean, float stddev, hipStream_t stream);

/* Library identification: the CAPI version and the offload architecture the
 * device code was built for (static string). */
int32_t rr_capi_version(void);
const char* rr_build_target(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* RAGGEDROUTE_CAPI_H */
