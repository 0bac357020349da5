// raggedroute/baseline_ops.h - naive HIP launchers (reference include/raggedroute/baseline_ops.h:14-42).
// Simple baselines with the reference semantics: device pointers, caller
// stream, no resets (callers zero histogram counts and permute cursors).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

#include "raggedroute_capi.h"

namespace raggedroute::ops {

inline hipError_t launch_dense_gemm_naive(const float* a, const float* b, float* c, int m, int n,
                                          int k, hipStream_t caller_stream) {
  return rr_launch_dense_gemm_naive(a, b, c, m, n, k, caller_stream);
}

inline hipError_t launch_topk_gate_naive(const float* logits, std::int32_t* expert_ids,
                                         float* weights, int tokens, int experts,
                                         hipStream_t caller_stream) {
  return rr_launch_topk_gate_naive(logits, expert_ids, weights, tokens, experts, caller_stream);
}

inline hipError_t launch_histogram_naive(const std::int32_t* expert_ids, std::int32_t* counts,
                                         int route_pairs, int experts, hipStream_t caller_stream) {
  return rr_launch_histogram_naive(expert_ids, counts, route_pairs, experts, caller_stream);
}

inline hipError_t launch_exclusive_scan_naive(const std::int32_t* counts, std::int32_t* offsets,
                                              int experts, hipStream_t caller_stream) {
  return rr_launch_exclusive_scan_naive(counts, offsets, experts, caller_stream);
}

inline hipError_t launch_token_permute_naive(const float* x, const std::int32_t* expert_ids,
                                             const std::int32_t* offsets, std::int32_t* cursors,
                                             float* x_permuted, std::int32_t* route_pos,
                                             std::int32_t* sorted_route, int tokens, int top_k,
                                             int hidden, hipStream_t caller_stream) {
  return rr_launch_token_permute_naive(x, expert_ids, offsets, cursors, x_permuted, route_pos,
                                       sorted_route, tokens, top_k, hidden, caller_stream);
}

inline hipError_t launch_grouped_gemm_naive(const float* x_permuted, const float* expert_weights,
                                            const std::int32_t* offsets, float* y_permuted,
                                            int experts, int hidden, int output,
                                            int max_expert_tokens, hipStream_t caller_stream) {
  return rr_launch_grouped_gemm_naive(x_permuted, expert_weights, offsets, y_permuted, experts,
                                      hidden, output, max_expert_tokens, caller_stream);
}

inline hipError_t launch_unpermute_naive(const float* y_permuted, const std::int32_t* route_pos,
                                         const float* route_weights, float* y, int tokens,
                                         int top_k, int output, hipStream_t caller_stream) {
  return rr_launch_unpermute_naive(y_permuted, route_pos, route_weights, y, tokens, top_k, output,
                                   caller_stream);
}

inline hipError_t launch_cache_scrub(std::uint32_t* buffer, std::size_t elements,
                                     hipStream_t caller_stream) {
  return rr_launch_cache_scrub(buffer, elements, caller_stream);
}

}  // namespace raggedroute::ops
