// C ABI operator wrappers: argument validation -> dispatch -> launch.
//
// Each wrapper keeps the check order and status codes of the reference
// wrapper it replaces (cited per function), with the expert cap raised from
// 64 to RR_MAX_EXPERTS. Wrappers never allocate and never synchronise.
#include <hip/hip_runtime_api.h>

#include <climits>
#include <cstddef>
#include <cstdint>

#include "common.h"
#include "launchers.h"

namespace rr {
namespace {

rr_operator_signature compute_signature(const rr_const_tensor_view& input,
                                        const rr_const_tensor_view& weight, int32_t accumulator,
                                        const rr_mutable_tensor_view& output) noexcept {
  rr_operator_signature s{};
  s.has_input = 1;
  s.input = input.spec;
  s.has_weight = 1;
  s.weight = weight.spec;
  s.has_accumulator = 1;
  s.accumulator = accumulator;
  s.has_output = 1;
  s.output = output.spec;
  return s;
}

rr_status unknown_family(const char* message) noexcept {
  return make_status(RR_STATUS_UNSUPPORTED_KERNEL_VARIANT, message);
}

rr_status null_context() noexcept { return invalid_argument("no runtime context was given"); }

}  // namespace
}  // namespace rr

extern "C" {

size_t rr_dense_gemm_workspace_size(const rr_dense_gemm_args*) { return 0; }
size_t rr_topk_gate_workspace_size(const rr_topk_gate_args*) { return 0; }
size_t rr_histogram_workspace_size(const rr_histogram_args*) { return 0; }
size_t rr_exclusive_scan_workspace_size(const rr_exclusive_scan_args*) { return 0; }
size_t rr_histogram_exclusive_scan_workspace_size(const rr_histogram_exclusive_scan_args*) {
  return 0;
}
// reference src/permute/operator.cpp:17-19
size_t rr_token_permute_workspace_size(const rr_token_permute_args* args) {
  if (args == nullptr || args->experts <= 0) return 0;
  return static_cast<size_t>(args->experts) * sizeof(int32_t);
}
size_t rr_grouped_gemm_workspace_size(const rr_grouped_gemm_args*) { return 0; }
size_t rr_unpermute_workspace_size(const rr_unpermute_args*) { return 0; }
// Chain workspace: E int32 cursor words, then 2T int32 words that hold
// sorted_route when the caller passes none (used by the fused path).
size_t rr_chain_workspace_size(const rr_chain_args* args) {
  if (args == nullptr || args->experts <= 0 || args->tokens < 0) return 0;
  return (static_cast<size_t>(args->experts) + 2 * static_cast<size_t>(args->tokens)) *
         sizeof(int32_t);
}
// Route chain workspace: E cursor words, then T * top_k words that hold
// sorted_route when the caller passes none.
size_t rr_route_chain_workspace_size(const rr_route_chain_args* args) {
  if (args == nullptr || args->experts <= 0 || args->tokens < 0 || args->top_k <= 0) return 0;
  return (static_cast<size_t>(args->experts) +
          static_cast<size_t>(args->tokens) * static_cast<size_t>(args->top_k)) *
         sizeof(int32_t);
}

// reference src/dense_gemm/operator.cpp:18-58
rr_status rr_dense_gemm(const rr_dense_gemm_args* args, const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("dense_gemm: no argument struct was given");
  if (context == nullptr) return rr::null_context();
  if (args->m < 0 || args->n < 0 || args->k < 0) {
    return rr::invalid_argument("dense_gemm: m, n and k must be >= 0");
  }
  if (args->alpha != 1.0F || args->beta != 0.0F) {
    return rr::invalid_argument("dense_gemm: only alpha = 1 with beta = 0 is implemented");
  }
  rr_dispatch_decision decision{};
  rr_status status = rr::dispatch_operator(
      RR_OP_DENSE_GEMM, rr::compute_signature(args->a, args->b, args->accumulator_dtype, args->c),
      args->kernel, context->architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (args->m == 0 || args->n == 0) return rr::ok_status();
  if (args->c.data == nullptr ||
      (args->k != 0 && (args->a.data == nullptr || args->b.data == nullptr))) {
    return rr::invalid_argument("dense_gemm: a buffer the call reads or writes is a null pointer");
  }
  if (!rr::is_aligned(args->a.data, alignof(float)) ||
      !rr::is_aligned(args->b.data, alignof(float)) ||
      !rr::is_aligned(args->c.data, alignof(float))) {
    return rr::invalid_argument("dense_gemm: every buffer must start on a 4-byte boundary");
  }
  const auto* a = static_cast<const float*>(args->a.data);
  const auto* b = static_cast<const float*>(args->b.data);
  auto* c = static_cast<float*>(args->c.data);
  if (decision.kernel.family == RR_FAMILY_NAIVE) {
    return rr::device_status(rr::kern::dense_gemm_naive(a, b, c, args->m, args->n, args->k,
                                                        context->stream),
                             "dense_gemm: the naive kernel did not launch");
  }
  if (rr::is_native(decision)) {
    return rr::device_status(
        rr::kern::dense_gemm_mfma(a, b, c, args->m, args->n, args->k, context->stream),
        "dense_gemm: the gfx950 kernel did not launch");
  }
  return rr::unknown_family("dense_gemm: no kernel exists for the selected family");
}

// reference src/topk_gate/operator.cpp:18-60
rr_status rr_topk_gate(const rr_topk_gate_args* args, const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("topk_gate: no argument struct was given");
  if (context == nullptr) return rr::null_context();
  if (args->tokens < 0 || args->experts < 2 || args->experts > RR_MAX_EXPERTS ||
      args->top_k != 2) {
    return rr::invalid_argument("topk_gate: needs tokens >= 0, 2 <= experts <= 1024 and top_k == 2");
  }
  if (args->normalization != RR_TOPK_SELECTED_SOFTMAX ||
      args->tie_break != RR_TOPK_TIE_LOWER_EXPERT_ID ||
      args->nan_policy != RR_TOPK_NAN_NEG_INF_ALL_NAN_01) {
    return rr::invalid_argument("topk_gate: only the reference tie, NaN and normalisation policies are implemented");
  }
  rr_operator_signature signature{};
  signature.has_input = 1;
  signature.input = args->logits.spec;
  signature.has_accumulator = 1;
  signature.accumulator = args->accumulator_dtype;
  signature.has_output = 1;
  signature.output = args->weights.spec;
  rr_dispatch_decision decision{};
  rr_status status = rr::dispatch_operator(RR_OP_TOPK_GATE, signature, args->kernel,
                                           context->architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (args->tokens == 0) return rr::ok_status();
  if (args->logits.data == nullptr || args->expert_ids == nullptr ||
      args->weights.data == nullptr) {
    return rr::invalid_argument("topk_gate: a buffer the call reads or writes is a null pointer");
  }
  if (!rr::is_aligned(args->logits.data, alignof(float)) ||
      !rr::is_aligned(args->weights.data, alignof(float))) {
    return rr::invalid_argument("topk_gate: every buffer must start on a 4-byte boundary");
  }
  const auto* logits = static_cast<const float*>(args->logits.data);
  auto* weights = static_cast<float*>(args->weights.data);
  hipError_t error = hipErrorInvalidValue;
  if (decision.kernel.family == RR_FAMILY_NAIVE) {
    error = rr::kern::topk_gate_naive(logits, args->expert_ids, weights, args->tokens,
                                      args->experts, context->stream);
  } else if (rr::is_native(decision)) {
    error = rr::kern::topk_gate_wave(logits, args->expert_ids, weights, args->tokens,
                                     args->experts, context->stream);
  } else {
    return rr::unknown_family("topk_gate: no kernel exists for the selected family");
  }
  return rr::device_status(error, "topk_gate: a kernel did not launch");
}

// reference src/histogram/operator.cpp:20-57
rr_status rr_histogram(const rr_histogram_args* args, const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("histogram: no argument struct was given");
  if (context == nullptr) return rr::null_context();
  if (args->route_pairs < 0 || args->experts <= 0 || args->experts > RR_MAX_EXPERTS) {
    return rr::invalid_argument("histogram: needs route_pairs >= 0 and 1 <= experts <= 1024");
  }
  rr_dispatch_decision decision{};
  rr_status status = rr::dispatch_operator(RR_OP_HISTOGRAM, {}, args->kernel,
                                           context->architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (args->counts == nullptr || (args->route_pairs != 0 && args->expert_ids == nullptr)) {
    return rr::invalid_argument("histogram: a buffer the call reads or writes is a null pointer");
  }
  if (!rr::is_aligned(args->counts, alignof(int32_t)) ||
      !rr::is_aligned(args->expert_ids, alignof(int32_t))) {
    return rr::invalid_argument("histogram: every buffer must start on a 4-byte boundary");
  }
  if (decision.kernel.family == RR_FAMILY_NAIVE) {
    // The naive launcher accumulates, so the wrapper owns the reset.
    status = rr::device_status(
        hipMemsetAsync(args->counts, 0, static_cast<size_t>(args->experts) * sizeof(int32_t),
                       context->stream),
        "histogram: clearing the counts failed");
    if (status.code != RR_STATUS_SUCCESS) return status;
    return rr::device_status(rr::kern::histogram_naive(args->expert_ids, args->counts,
                                                       args->route_pairs, args->experts,
                                                       context->stream),
                             "histogram: a kernel did not launch");
  }
  if (rr::is_native(decision)) {
    return rr::device_status(rr::kern::histogram_native(args->expert_ids, args->counts,
                                                        args->route_pairs, args->experts,
                                                        context->stream),
                             "histogram: a kernel did not launch");
  }
  return rr::unknown_family("histogram: no kernel exists for the selected family");
}

// reference src/scan/operator.cpp:51-74
rr_status rr_exclusive_scan(const rr_exclusive_scan_args* args,
                            const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("exclusive_scan: no argument struct was given");
  if (context == nullptr) return rr::null_context();
  if (args->experts <= 0 || args->experts > RR_MAX_EXPERTS) {
    return rr::invalid_argument("exclusive_scan: needs 1 <= experts <= 1024");
  }
  rr_dispatch_decision decision{};
  rr_status status = rr::dispatch_operator(RR_OP_EXCLUSIVE_SCAN, {}, args->kernel,
                                           context->architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (args->counts == nullptr || args->offsets == nullptr) {
    return rr::invalid_argument("exclusive_scan: a buffer the call reads or writes is a null pointer");
  }
  if (!rr::is_aligned(args->counts, alignof(int32_t)) ||
      !rr::is_aligned(args->offsets, alignof(int32_t))) {
    return rr::invalid_argument("exclusive_scan: every buffer must start on a 4-byte boundary");
  }
  if (decision.kernel.family == RR_FAMILY_NAIVE) {
    return rr::device_status(rr::kern::exclusive_scan_naive(args->counts, args->offsets,
                                                            args->experts, context->stream),
                             "exclusive_scan: the naive kernel did not launch");
  }
  if (rr::is_native(decision)) {
    return rr::device_status(rr::kern::exclusive_scan_native(args->counts, args->offsets,
                                                             args->experts, context->stream),
                             "exclusive_scan: a kernel did not launch");
  }
  return rr::unknown_family("exclusive_scan: no kernel exists for the selected family");
}

// reference src/scan/operator.cpp:84-134
rr_status rr_histogram_exclusive_scan(const rr_histogram_exclusive_scan_args* args,
                                      const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("histogram_exclusive_scan: no argument struct was given");
  if (context == nullptr) return rr::null_context();
  if (args->route_pairs < 0 || args->experts <= 0 || args->experts > RR_MAX_EXPERTS) {
    return rr::invalid_argument("histogram_exclusive_scan: needs route_pairs >= 0 and 1 <= experts <= 1024");
  }
  if (args->counts == nullptr || args->offsets == nullptr ||
      (args->route_pairs != 0 && args->expert_ids == nullptr)) {
    return rr::invalid_argument("histogram_exclusive_scan: a buffer the call reads or writes is a null pointer");
  }
  if (!rr::is_aligned(args->expert_ids, alignof(int32_t)) ||
      !rr::is_aligned(args->counts, alignof(int32_t)) ||
      !rr::is_aligned(args->offsets, alignof(int32_t))) {
    return rr::invalid_argument("histogram_exclusive_scan: every buffer must start on a 4-byte boundary");
  }
  const size_t ids_bytes = static_cast<size_t>(args->route_pairs) * sizeof(int32_t);
  const size_t counts_bytes = static_cast<size_t>(args->experts) * sizeof(int32_t);
  const size_t offsets_bytes = static_cast<size_t>(args->experts + 1) * sizeof(int32_t);
  if (rr::ranges_overlap(args->expert_ids, ids_bytes, args->counts, counts_bytes) ||
      rr::ranges_overlap(args->expert_ids, ids_bytes, args->offsets, offsets_bytes) ||
      rr::ranges_overlap(args->counts, counts_bytes, args->offsets, offsets_bytes)) {
    return rr::invalid_argument(
        "histogram_exclusive_scan: ids, counts and offsets must not overlap");
  }
  rr_dispatch_decision decision{};
  rr_status status = rr::dispatch_operator(RR_OP_HISTOGRAM_EXCLUSIVE_SCAN, {}, args->kernel,
                                           context->architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (decision.kernel.family == RR_FAMILY_NAIVE) {
    // Separate path: reset + naive histogram, then naive scan.
    status = rr::device_status(hipMemsetAsync(args->counts, 0, counts_bytes, context->stream),
                               "histogram: clearing the counts failed");
    if (status.code != RR_STATUS_SUCCESS) return status;
    status = rr::device_status(rr::kern::histogram_naive(args->expert_ids, args->counts,
                                                         args->route_pairs, args->experts,
                                                         context->stream),
                               "histogram: a kernel did not launch");
    if (status.code != RR_STATUS_SUCCESS) return status;
    return rr::device_status(rr::kern::exclusive_scan_naive(args->counts, args->offsets,
                                                            args->experts, context->stream),
                             "exclusive_scan: the naive kernel did not launch");
  }
  if (rr::is_native(decision)) {
    return rr::device_status(
        rr::kern::histogram_exclusive_scan_native(args->expert_ids, args->counts, args->offsets,
                                                  args->route_pairs, args->experts,
                                                  context->stream),
        "histogram_exclusive_scan: a kernel did not launch");
  }
  return rr::unknown_family("histogram_exclusive_scan: no kernel exists for the selected family");
}

// reference src/permute/operator.cpp:22-83
rr_status rr_token_permute(const rr_token_permute_args* args, const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("token_permute: no argument struct was given");
  if (context == nullptr) return rr::null_context();
  if (args->tokens < 0 || args->experts <= 0 || args->experts > RR_MAX_EXPERTS ||
      args->top_k <= 0 || args->top_k > args->experts || args->hidden < 0) {
    return rr::invalid_argument(
        "token_permute: needs tokens >= 0, 1 <= top_k <= experts <= 1024 and hidden >= 0");
  }
  if (args->tokens > 0 && args->tokens > INT_MAX / args->top_k) {
    return rr::invalid_argument("token_permute: tokens * top_k does not fit in int32");
  }
  rr_operator_signature signature{};
  signature.has_input = 1;
  signature.input = args->x.spec;
  signature.has_output = 1;
  signature.output = args->x_permuted.spec;
  rr_dispatch_decision decision{};
  rr_status status = rr::dispatch_operator(RR_OP_TOKEN_PERMUTE, signature, args->kernel,
                                           context->architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (args->tokens == 0) return rr::ok_status();
  if (args->expert_ids == nullptr || args->offsets == nullptr || args->route_pos == nullptr ||
      (args->hidden != 0 && (args->x.data == nullptr || args->x_permuted.data == nullptr))) {
    return rr::invalid_argument("token_permute: a buffer the call reads or writes is a null pointer");
  }
  if (!rr::is_aligned(args->x.data, alignof(float)) ||
      !rr::is_aligned(args->x_permuted.data, alignof(float))) {
    return rr::invalid_argument("token_permute: every buffer must start on a 4-byte boundary");
  }
  const size_t workspace_bytes = static_cast<size_t>(args->experts) * sizeof(int32_t);
  if (context->workspace == nullptr || context->workspace_bytes < workspace_bytes) {
    return rr::make_status(RR_STATUS_INSUFFICIENT_WORKSPACE,
                           "token_permute: the workspace must hold one int32 cursor per expert");
  }
  if (!rr::is_aligned(context->workspace, alignof(int32_t))) {
    return rr::invalid_argument("token_permute: the workspace must start on a 4-byte boundary");
  }
  const auto* x = static_cast<const float*>(args->x.data);
  auto* x_permuted = static_cast<float*>(args->x_permuted.data);
  auto* cursors = static_cast<int32_t*>(context->workspace);
  if (decision.kernel.family == RR_FAMILY_NAIVE) {
    // The naive launcher increments cursors atomically; the wrapper resets them.
    status = rr::device_status(hipMemsetAsync(cursors, 0, workspace_bytes, context->stream),
                               "token_permute: clearing the cursors failed");
    if (status.code != RR_STATUS_SUCCESS) return status;
    return rr::device_status(
        rr::kern::token_permute_naive(x, args->expert_ids, args->offsets, cursors, x_permuted,
                                      args->route_pos, args->sorted_route, args->tokens,
                                      args->top_k, args->hidden, args->experts, context->stream),
        "token_permute: the naive kernel did not launch");
  }
  if (rr::is_native(decision)) {
    // The stable kernel writes the final cursor values itself (no reset pass).
    return rr::device_status(
        rr::kern::token_permute_stable(x, args->expert_ids, args->offsets, cursors, x_permuted,
                                       args->route_pos, args->sorted_route, args->tokens,
                                       args->experts, args->top_k, args->hidden,
                                       context->stream),
        "token_permute: a kernel did not launch");
  }
  return rr::unknown_family("token_permute: no kernel exists for the selected family");
}

// reference src/grouped_gemm/operator.cpp:17-49
rr_status rr_grouped_gemm(const rr_grouped_gemm_args* args, const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("grouped_gemm: no argument struct was given");
  if (context == nullptr) return rr::null_context();
  if (args->experts <= 0 || args->experts > RR_MAX_EXPERTS || args->hidden < 0 ||
      args->output < 0 || args->max_expert_tokens < 0) {
    return rr::invalid_argument("grouped_gemm: needs 1 <= experts <= 1024 and hidden, output, max_expert_tokens >= 0");
  }
  rr_dispatch_decision decision{};
  rr_status status = rr::dispatch_operator(
      RR_OP_GROUPED_GEMM,
      rr::compute_signature(args->x_permuted, args->expert_weights, args->accumulator_dtype,
                            args->y_permuted),
      args->kernel, context->architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (args->max_expert_tokens == 0 || args->output == 0) return rr::ok_status();
  if (args->offsets == nullptr || args->y_permuted.data == nullptr ||
      (args->hidden != 0 &&
       (args->x_permuted.data == nullptr || args->expert_weights.data == nullptr))) {
    return rr::invalid_argument("grouped_gemm: a buffer the call reads or writes is a null pointer");
  }
  if (!rr::is_aligned(args->x_permuted.data, alignof(float)) ||
      !rr::is_aligned(args->expert_weights.data, alignof(float)) ||
      !rr::is_aligned(args->y_permuted.data, alignof(float))) {
    return rr::invalid_argument("grouped_gemm: every buffer must start on a 4-byte boundary");
  }
  const auto* x = static_cast<const float*>(args->x_permuted.data);
  const auto* w = static_cast<const float*>(args->expert_weights.data);
  auto* y = static_cast<float*>(args->y_permuted.data);
  if (decision.kernel.family == RR_FAMILY_NAIVE) {
    return rr::device_status(
        rr::kern::grouped_gemm_naive(x, w, args->offsets, y, args->experts, args->hidden,
                                     args->output, args->max_expert_tokens, context->stream),
        "grouped_gemm: a kernel did not launch");
  }
  if (rr::is_native(decision)) {
    return rr::device_status(
        rr::kern::grouped_gemm_mfma(x, w, args->offsets, y, args->experts, args->hidden,
                                    args->output, args->max_expert_tokens, context->stream),
        "grouped_gemm: a kernel did not launch");
  }
  return rr::unknown_family("grouped_gemm: no kernel exists for the selected family");
}

// reference src/unpermute/operator.cpp:19-57
rr_status rr_unpermute(const rr_unpermute_args* args, const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("unpermute: no argument struct was given");
  if (context == nullptr) return rr::null_context();
  if (args->tokens < 0 || args->top_k <= 0 || args->top_k > 64 || args->output < 0) {
    return rr::invalid_argument("unpermute: needs tokens >= 0, 1 <= top_k <= 64 and output >= 0");
  }
  if (args->tokens > 0 && args->tokens > INT_MAX / args->top_k) {
    return rr::invalid_argument("unpermute: tokens * top_k does not fit in int32");
  }
  if (args->tokens > 0 && args->output > 0 && args->tokens > INT_MAX / args->output) {
    return rr::invalid_argument("unpermute: tokens * output does not fit in int32");
  }
  rr_dispatch_decision decision{};
  rr_status status = rr::dispatch_operator(
      RR_OP_UNPERMUTE,
      rr::compute_signature(args->y_permuted, args->route_weights, args->accumulator_dtype,
                            args->y),
      args->kernel, context->architecture, &decision);
  if (status.code != RR_STATUS_SUCCESS) return status;
  if (args->tokens == 0 || args->output == 0) return rr::ok_status();
  if (args->y_permuted.data == nullptr || args->route_pos == nullptr ||
      args->route_weights.data == nullptr || args->y.data == nullptr) {
    return rr::invalid_argument("unpermute: a buffer the call reads or writes is a null pointer");
  }
  if (!rr::is_aligned(args->y_permuted.data, alignof(float)) ||
      !rr::is_aligned(args->route_weights.data, alignof(float)) ||
      !rr::is_aligned(args->y.data, alignof(float))) {
    return rr::invalid_argument("unpermute: every buffer must start on a 4-byte boundary");
  }
  const auto* yp = static_cast<const float*>(args->y_permuted.data);
  const auto* w = static_cast<const float*>(args->route_weights.data);
  auto* y = static_cast<float*>(args->y.data);
  if (decision.kernel.family == RR_FAMILY_NAIVE) {
    return rr::device_status(rr::kern::unpermute_naive(yp, args->route_pos, w, y, args->tokens,
                                                       args->top_k, args->output,
                                                       context->stream),
                             "unpermute: a kernel did not launch");
  }
  if (rr::is_native(decision)) {
    return rr::device_status(rr::kern::unpermute_gather(yp, args->route_pos, w, y, args->tokens,
                                                        args->top_k, args->output,
                                                        context->stream),
                             "unpermute: a kernel did not launch");
  }
  return rr::unknown_family("unpermute: no kernel exists for the selected family");
}

}  // extern "C"
