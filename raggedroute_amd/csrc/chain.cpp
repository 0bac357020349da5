// Chain entries: chain_from_tokens (7 stages) and chain_from_logits (6 stages).
//
// The stage order is the one of reference benchmarks/adapters/chain_adapter.cpp:263-467:
// dense GEMM -> top-2 gate -> histogram+scan -> token permute -> grouped GEMM
// -> unpermute, all on the caller's stream, with no host synchronisation.
//
// Auto / optimized family: two or three fused launches that write every output
// of the seven stages with the same values as running them one by one:
//   1. router GEMM with the top-2 gate in its epilogue (gate kernel for
//      chain_from_logits), also zeroing y;
//   2. route preparation: counts, offsets, stable route_pos, sorted_route, cursors;
//   3. grouped GEMM gathering x rows through sorted_route, writing x_permuted
//      and y_permuted and adding both weighted routes of each token into y.
// Where the narrow-output strip kernel covers the shape (N <= 128, K <= 256,
// T <= 8192, E <= 256), 2 and 3 are one launch: every workgroup derives the
// offsets and its own rows' routes from the ids itself.
// Naive family: the seven stages through the public C ABI entries (the grouped
// GEMM gets the worst-case launch bound max_expert_tokens = R, reference
// chain_adapter.cpp:391-401).
#include <climits>
#include <cstddef>
#include <cstdint>

#include "common.h"
#include "launchers.h"

namespace rr {
namespace {

rr_const_tensor_view cview(const void* data) noexcept { return {data, default_spec()}; }
rr_mutable_tensor_view mview(void* data) noexcept { return {data, default_spec()}; }

rr_status validate_chain(const rr_chain_args* a, const rr_runtime_context* context,
                         bool from_tokens) noexcept {
  if (a == nullptr) return invalid_argument("chain args must not be null");
  if (context == nullptr) return invalid_argument("no runtime context was given");
  if (a->tokens < 0 || a->experts < 2 || a->experts > RR_MAX_EXPERTS || a->top_k != 2 ||
      a->hidden < 0 || a->output < 0) {
    return invalid_argument("chain requires T>=0, 2<=E<=1024, top_k=2, K>=0 and N>=0");
  }
  if (a->tokens > INT_MAX / 2) return invalid_argument("chain route count exceeds int32 indexing");
  if (a->tokens > 0 && a->output > 0 && a->tokens > INT_MAX / a->output) {
    return invalid_argument("chain output count exceeds int32 indexing");
  }
  if (a->tokens == 0) return ok_status();
  // (y_permuted and y have no elements at N = 0, as in grouped_gemm / unpermute)
  if (a->logits == nullptr || a->expert_ids == nullptr || a->route_weights == nullptr ||
      a->counts == nullptr || a->offsets == nullptr || a->route_pos == nullptr ||
      (a->output != 0 && (a->y_permuted == nullptr || a->y == nullptr))) {
    return invalid_argument("chain received a null device pointer");
  }
  // (expert weights [E, K, N] have no elements at K = 0 or N = 0)
  if (a->hidden != 0 && (a->x == nullptr || a->x_permuted == nullptr ||
                         (a->output != 0 && a->expert_weights == nullptr) ||
                         (from_tokens && a->router_weights == nullptr))) {
    return invalid_argument("chain received a null device pointer");
  }
  if (context->workspace == nullptr || context->workspace_bytes < rr_chain_workspace_size(a)) {
    return make_status(RR_STATUS_INSUFFICIENT_WORKSPACE,
                       "chain requires rr_chain_workspace_size bytes of int32 workspace");
  }
  if (!is_aligned(context->workspace, alignof(int32_t))) {
    return invalid_argument("chain workspace is not int32 aligned");
  }
  return ok_status();
}

// Fused path (auto / optimized family); see the file comment. Launches in
// order: 0 = router GEMM + gate (gate only for chain_from_logits); then, when
// the strip kernel covers the shape, 1 = route preparation + expert GEMM +
// unpermute in one launch; otherwise 1 = route preparation and 2 = expert GEMM
// + unpermute.
bool merged_prep(const rr_chain_args* a) noexcept {
  return kern::strip_chain_ok(a->tokens, 2, a->experts, a->hidden, a->output, a->x,
                              a->expert_weights, a->expert_ids, a->x_permuted);
}

int fused_launch_count(const rr_chain_args* a) noexcept { return merged_prep(a) ? 2 : 3; }

const char* fused_launch_name(const rr_chain_args* a, bool from_tokens, int launch) noexcept {
  const bool merged = merged_prep(a);
  if (launch == 0) return from_tokens ? "router_gate" : "gate";
  if (launch == 1) return merged ? "route_prep_expert_gemm" : "route_prep";
  if (launch == 2 && !merged) return "expert_gemm";
  return nullptr;
}

// `only` selects a single launch for per-launch timing, -1 runs all of them.
rr_status run_fused(const rr_chain_args* a, const rr_runtime_context& ctx, bool from_tokens,
                    int only = -1) noexcept {
  auto* cursors = static_cast<int32_t*>(ctx.workspace);
  int32_t* sorted_route = a->sorted_route != nullptr ? a->sorted_route : cursors + a->experts;
  const int routes = a->tokens * 2;
  const bool merged = merged_prep(a);
  hipError_t err = hipSuccess;
  if (only < 0 || only == 0) {
    // The router GEMM carries the gate in its epilogue where the strip kernel
    // covers it (K <= 256, E <= 128); longer K runs the tiled dense GEMM (its
    // best tiles need no epilogue staging) and the gate kernel.
    if (from_tokens && a->experts <= 128 &&
        kern::strip_shape_ok(a->hidden, a->experts, a->x, a->router_weights)) {
      err = kern::router_gate_mfma(a->x, a->router_weights, a->logits, a->expert_ids,
                                   a->route_weights, a->y, a->output, a->tokens, a->experts,
                                   a->hidden, ctx.stream);
    } else {
      if (from_tokens) {
        err = kern::dense_gemm_mfma(a->x, a->router_weights, a->logits, a->tokens, a->experts,
                                    a->hidden, ctx.stream);
        if (err != hipSuccess) return device_status(err, "chain router GEMM launch failed");
      }
      err = kern::topk_gate_wave(a->logits, a->expert_ids, a->route_weights, a->tokens,
                                 a->experts, ctx.stream, a->y, a->output);
    }
    if (err != hipSuccess) return device_status(err, "chain gate launch failed");
  }
  if (merged) {
    if (only < 0 || only == 1) {
      err = kern::strip_chain(a->x, a->expert_weights, a->expert_ids, a->route_weights, a->counts,
                              a->offsets, cursors, a->route_pos, a->sorted_route, a->x_permuted,
                              a->y_permuted, a->y, a->tokens, 2, a->experts, a->hidden,
                              a->output, ctx.stream);
      if (err != hipSuccess) return device_status(err, "chain expert GEMM launch failed");
    }
    return ok_status();
  }
  if (only < 0 || only == 1) {
    err = kern::route_prep(a->expert_ids, a->counts, a->offsets, cursors, a->route_pos,
                           sorted_route, routes, a->experts, ctx.stream);
    if (err != hipSuccess) return device_status(err, "chain route preparation launch failed");
  }
  if (only < 0 || only == 2) {
    err = kern::chain_grouped_mfma(a->x, a->expert_weights, a->offsets, sorted_route,
                                   a->route_weights, a->x_permuted, a->y_permuted, a->y,
                                   a->tokens, 2, a->experts, a->hidden, a->output, ctx.stream);
    if (err != hipSuccess) return device_status(err, "chain grouped GEMM launch failed");
    // N = 0: the GEMM has no column tiles to gather x_permuted in
    if (a->output == 0 && a->hidden > 0) {
      err = kern::permute_copy(a->x, a->route_pos, a->x_permuted, a->tokens, 2, a->hidden,
                               ctx.stream);
      if (err != hipSuccess) return device_status(err, "chain permute copy launch failed");
    }
  }
  return ok_status();
}

rr_status run_chain(const rr_chain_args* a, const rr_runtime_context* context,
                    bool from_tokens) noexcept {
  rr_status status = validate_chain(a, context, from_tokens);
  if (status.code != RR_STATUS_SUCCESS || a->tokens == 0) return status;

  rr_runtime_context ctx = *context;
  status = rr_resolve_device_architecture(context->architecture, &ctx.architecture);
  if (status.code != RR_STATUS_SUCCESS) return status;
  const int32_t routes = a->tokens * 2;
  // An optimized request selects the native kernel of every stage (operator-local
  // ids do not carry across stages); auto and naive pass through unchanged.
  rr_kernel_selection kernel = a->kernel;
  if (kernel.family == RR_FAMILY_OPTIMIZED) kernel.implementation_id = RR_IMPL_GFX950_NATIVE;
  // Same dispatch checks as the stages (architecture, family / id) before the fused path.
  rr_dispatch_decision decision{};
  status = dispatch_operator(RR_OP_HISTOGRAM_EXCLUSIVE_SCAN, {}, kernel, ctx.architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (decision.kernel.family == RR_FAMILY_OPTIMIZED) return run_fused(a, ctx, from_tokens);

  if (from_tokens) {
    rr_dense_gemm_args dense{};
    dense.a = cview(a->x);
    dense.b = cview(a->router_weights);
    dense.c = mview(a->logits);
    dense.m = a->tokens;
    dense.n = a->experts;
    dense.k = a->hidden;
    dense.alpha = 1.0F;
    dense.beta = 0.0F;
    dense.accumulator_dtype = RR_DTYPE_FP32;
    dense.kernel = kernel;
    status = rr_dense_gemm(&dense, &ctx);
    if (status.code != RR_STATUS_SUCCESS) return status;
  }

  rr_topk_gate_args gate{};
  gate.logits = cview(a->logits);
  gate.expert_ids = a->expert_ids;
  gate.weights = mview(a->route_weights);
  gate.tokens = a->tokens;
  gate.experts = a->experts;
  gate.top_k = 2;
  gate.accumulator_dtype = RR_DTYPE_FP32;
  gate.kernel = kernel;
  status = rr_topk_gate(&gate, &ctx);
  if (status.code != RR_STATUS_SUCCESS) return status;

  rr_histogram_exclusive_scan_args meta{};
  meta.expert_ids = a->expert_ids;
  meta.counts = a->counts;
  meta.offsets = a->offsets;
  meta.route_pairs = routes;
  meta.experts = a->experts;
  meta.kernel = kernel;
  status = rr_histogram_exclusive_scan(&meta, &ctx);
  if (status.code != RR_STATUS_SUCCESS) return status;

  rr_token_permute_args permute{};
  permute.x = cview(a->x);
  permute.expert_ids = a->expert_ids;
  permute.offsets = a->offsets;
  permute.x_permuted = mview(a->x_permuted);
  permute.route_pos = a->route_pos;
  permute.sorted_route = a->sorted_route;
  permute.tokens = a->tokens;
  permute.experts = a->experts;
  permute.top_k = 2;
  permute.hidden = a->hidden;
  permute.kernel = kernel;
  status = rr_token_permute(&permute, &ctx);
  if (status.code != RR_STATUS_SUCCESS) return status;

  rr_grouped_gemm_args grouped{};
  grouped.x_permuted = cview(a->x_permuted);
  grouped.expert_weights = cview(a->expert_weights);
  grouped.offsets = a->offsets;
  grouped.y_permuted = mview(a->y_permuted);
  grouped.experts = a->experts;
  grouped.hidden = a->hidden;
  grouped.output = a->output;
  grouped.max_expert_tokens = routes;
  grouped.accumulator_dtype = RR_DTYPE_FP32;
  grouped.kernel = kernel;
  status = rr_grouped_gemm(&grouped, &ctx);
  if (status.code != RR_STATUS_SUCCESS) return status;

  rr_unpermute_args unpermute{};
  unpermute.y_permuted = cview(a->y_permuted);
  unpermute.route_pos = a->route_pos;
  unpermute.route_weights = cview(a->route_weights);
  unpermute.y = mview(a->y);
  unpermute.tokens = a->tokens;
  unpermute.top_k = 2;
  unpermute.output = a->output;
  unpermute.accumulator_dtype = RR_DTYPE_FP32;
  unpermute.kernel = kernel;
  return rr_unpermute(&unpermute, &ctx);
}

// ---- post-route chain (chain_from_route_ids) ----
// Stage order of reference benchmarks/adapters/postroute_chain_adapter.cpp:240-356
// (histogram -> scan -> token permute -> grouped GEMM -> unpermute); the shape
// limits are the intersection of the stage operators' (token_permute:
// 1 <= top_k <= E <= 1024; unpermute: top_k <= 64).
rr_status validate_route_chain(const rr_route_chain_args* a,
                               const rr_runtime_context* context) noexcept {
  if (a == nullptr) return invalid_argument("route chain args must not be null");
  if (context == nullptr) return invalid_argument("no runtime context was given");
  if (a->tokens < 0 || a->experts < 1 || a->experts > RR_MAX_EXPERTS || a->top_k < 1 ||
      a->top_k > a->experts || a->top_k > 64 || a->hidden < 0 || a->output < 0) {
    return invalid_argument(
        "route chain requires T>=0, 1<=top_k<=E<=1024, top_k<=64, K>=0 and N>=0");
  }
  if (a->tokens > INT_MAX / a->top_k) {
    return invalid_argument("route chain route count exceeds int32 indexing");
  }
  if (a->tokens > 0 && a->output > 0 && a->tokens > INT_MAX / a->output) {
    return invalid_argument("route chain output count exceeds int32 indexing");
  }
  if (a->tokens == 0) return ok_status();
  if (a->expert_ids == nullptr || a->counts == nullptr || a->offsets == nullptr ||
      a->route_pos == nullptr ||
      (a->output != 0 && (a->route_weights == nullptr || a->y_permuted == nullptr || a->y == nullptr)) ||
      (a->hidden != 0 && (a->x == nullptr ||
                          (a->output != 0 && a->expert_weights == nullptr)))) {
    return invalid_argument("route chain received a null device pointer");
  }
  if (context->workspace == nullptr ||
      context->workspace_bytes < rr_route_chain_workspace_size(a)) {
    return make_status(RR_STATUS_INSUFFICIENT_WORKSPACE,
                       "route chain requires rr_route_chain_workspace_size bytes of int32 workspace");
  }
  if (!is_aligned(context->workspace, alignof(int32_t))) {
    return invalid_argument("route chain workspace is not int32 aligned");
  }
  return ok_status();
}

// Fused path: routing metadata and the expert GEMM over rows gathered from x
// through sorted_route in one launch where the strip kernel covers the shape
// (route_prep + gathered grouped GEMM otherwise), then the unpermute gather in
// route order per token. x_permuted is written only when the caller passes it.
rr_status run_route_chain_fused(const rr_route_chain_args* a,
                                const rr_runtime_context& ctx) noexcept {
  auto* cursors = static_cast<int32_t*>(ctx.workspace);
  int32_t* sorted_route = a->sorted_route != nullptr ? a->sorted_route : cursors + a->experts;
  const int routes = a->tokens * a->top_k;
  hipError_t err = hipSuccess;
  if (kern::strip_chain_ok(a->tokens, a->top_k, a->experts, a->hidden, a->output, a->x,
                           a->expert_weights, a->expert_ids, a->x_permuted)) {
    err = kern::strip_chain(a->x, a->expert_weights, a->expert_ids, a->route_weights, a->counts,
                            a->offsets, cursors, a->route_pos, a->sorted_route, a->x_permuted,
                            a->y_permuted, nullptr, a->tokens, a->top_k, a->experts, a->hidden,
                            a->output, ctx.stream);
    if (err != hipSuccess) return device_status(err, "route chain expert GEMM launch failed");
  } else {
    err = kern::route_prep(a->expert_ids, a->counts, a->offsets, cursors, a->route_pos,
                           sorted_route, routes, a->experts, ctx.stream);
    if (err != hipSuccess) return device_status(err, "route chain preparation launch failed");
    err = kern::chain_grouped_mfma(a->x, a->expert_weights, a->offsets, sorted_route,
                                   a->route_weights, a->x_permuted, a->y_permuted, nullptr,
                                   a->tokens, a->top_k, a->experts, a->hidden, a->output,
                                   ctx.stream);
    if (err != hipSuccess) return device_status(err, "route chain grouped GEMM launch failed");
    // N = 0: the GEMM has no column tiles to gather x_permuted in
    if (a->output == 0 && a->hidden > 0 && a->x_permuted != nullptr) {
      err = kern::permute_copy(a->x, a->route_pos, a->x_permuted, a->tokens, a->top_k, a->hidden,
                               ctx.stream);
      if (err != hipSuccess) return device_status(err, "route chain permute copy launch failed");
    }
  }
  err = kern::unpermute_gather(a->y_permuted, a->route_pos, a->route_weights, a->y, a->tokens,
                               a->top_k, a->output, ctx.stream);
  if (err != hipSuccess) return device_status(err, "route chain unpermute launch failed");
  return ok_status();
}

rr_status run_route_chain(const rr_route_chain_args* a,
                          const rr_runtime_context* context) noexcept {
  rr_status status = validate_route_chain(a, context);
  if (status.code != RR_STATUS_SUCCESS || a->tokens == 0) return status;

  rr_runtime_context ctx = *context;
  status = rr_resolve_device_architecture(context->architecture, &ctx.architecture);
  if (status.code != RR_STATUS_SUCCESS) return status;
  const int32_t routes = a->tokens * a->top_k;
  rr_kernel_selection kernel = a->kernel;
  if (kernel.family == RR_FAMILY_OPTIMIZED) kernel.implementation_id = RR_IMPL_GFX950_NATIVE;
  rr_dispatch_decision decision{};
  status = dispatch_operator(RR_OP_HISTOGRAM_EXCLUSIVE_SCAN, {}, kernel, ctx.architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (decision.kernel.family == RR_FAMILY_OPTIMIZED) return run_route_chain_fused(a, ctx);
  if (a->hidden != 0 && a->x_permuted == nullptr) {
    return invalid_argument("the naive route chain requires x_permuted");
  }

  rr_histogram_args histogram{};
  histogram.expert_ids = a->expert_ids;
  histogram.counts = a->counts;
  histogram.route_pairs = routes;
  histogram.experts = a->experts;
  histogram.kernel = kernel;
  status = rr_histogram(&histogram, &ctx);
  if (status.code != RR_STATUS_SUCCESS) return status;

  rr_exclusive_scan_args scan{};
  scan.counts = a->counts;
  scan.offsets = a->offsets;
  scan.experts = a->experts;
  scan.kernel = kernel;
  status = rr_exclusive_scan(&scan, &ctx);
  if (status.code != RR_STATUS_SUCCESS) return status;

  rr_token_permute_args permute{};
  permute.x = cview(a->x);
  permute.expert_ids = a->expert_ids;
  permute.offsets = a->offsets;
  permute.x_permuted = mview(a->x_permuted);
  permute.route_pos = a->route_pos;
  permute.sorted_route = a->sorted_route;
  permute.tokens = a->tokens;
  permute.experts = a->experts;
  permute.top_k = a->top_k;
  permute.hidden = a->hidden;
  permute.kernel = kernel;
  status = rr_token_permute(&permute, &ctx);
  if (status.code != RR_STATUS_SUCCESS) return status;

  rr_grouped_gemm_args grouped{};
  grouped.x_permuted = cview(a->x_permuted);
  grouped.expert_weights = cview(a->expert_weights);
  grouped.offsets = a->offsets;
  grouped.y_permuted = mview(a->y_permuted);
  grouped.experts = a->experts;
  grouped.hidden = a->hidden;
  grouped.output = a->output;
  grouped.max_expert_tokens = routes;
  grouped.accumulator_dtype = RR_DTYPE_FP32;
  grouped.kernel = kernel;
  status = rr_grouped_gemm(&grouped, &ctx);
  if (status.code != RR_STATUS_SUCCESS) return status;

  rr_unpermute_args unpermute{};
  unpermute.y_permuted = cview(a->y_permuted);
  unpermute.route_pos = a->route_pos;
  unpermute.route_weights = cview(a->route_weights);
  unpermute.y = mview(a->y);
  unpermute.tokens = a->tokens;
  unpermute.top_k = a->top_k;
  unpermute.output = a->output;
  unpermute.accumulator_dtype = RR_DTYPE_FP32;
  unpermute.kernel = kernel;
  return rr_unpermute(&unpermute, &ctx);
}

}  // namespace
}  // namespace rr

extern "C" {

rr_status rr_chain_from_route_ids(const rr_route_chain_args* args,
                                  const rr_runtime_context* context) {
  return rr::run_route_chain(args, context);
}

rr_status rr_chain_from_tokens(const rr_chain_args* args, const rr_runtime_context* context) {
  return rr::run_chain(args, context, true);
}

rr_status rr_chain_from_logits(const rr_chain_args* args, const rr_runtime_context* context) {
  return rr::run_chain(args, context, false);
}

rr_status rr_chain_fused_launch(const rr_chain_args* args, const rr_runtime_context* context,
                                int32_t from_tokens, int32_t launch) {
  rr_status status = rr::validate_chain(args, context, from_tokens != 0);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (launch < 0 || launch >= rr::fused_launch_count(args)) {
    return rr::invalid_argument("fused chain launch index out of range for this shape");
  }
  if (args->tokens == 0) return status;
  return rr::run_fused(args, *context, from_tokens != 0, launch);
}

const char* rr_chain_fused_launch_name(const rr_chain_args* args, int32_t from_tokens,
                                       int32_t launch) {
  if (args == nullptr) return nullptr;
  return rr::fused_launch_name(args, from_tokens != 0, launch);
}

}  // extern "C"
