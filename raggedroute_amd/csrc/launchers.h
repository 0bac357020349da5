// Host-side launchers of the gfx950 kernels (defined in the *.hip files).
// Shapes are validated by the callers; every launcher returns the launch error.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace rr::kern {

// ---- dense / grouped GEMM on FP32 MFMA (gemm.hip) ----
// c[m, n] = a[m, k] * b[k, n]
hipError_t dense_gemm_mfma(const float* a, const float* b, float* c, int m, int n, int k,
                           hipStream_t stream);
// y[r, :] = x[r, :] * w[e] for r in [offsets[e], offsets[e + 1]); offsets read on device.
hipError_t grouped_gemm_mfma(const float* x, const float* w, const int32_t* offsets, float* y,
                             int experts, int hidden, int output, int max_expert_tokens,
                             hipStream_t stream);

// ---- fused chain forms (gemm.hip) ----
// logits = x * router_weights with each row's top-2 ids / weights taken in the
// epilogue; rows [0, tokens) of y_zero ([tokens, y_cols]) are zeroed. Strip
// shapes only (E <= 128, K <= 256); hipErrorInvalidValue otherwise.
hipError_t router_gate_mfma(const float* x, const float* router_weights, float* logits,
                            int32_t* ids, float* gate_weights, float* y_zero, int y_cols,
                            int tokens, int experts, int hidden, hipStream_t stream);
// Grouped GEMM over x rows gathered through sorted_route (route = top_k *
// token + rank): writes x_permuted (optional) and y_permuted and, when y is
// given (top_k = 2 only), adds w[route] * y_permuted[row] into the zeroed
// y[token] (the unpermute).
hipError_t chain_grouped_mfma(const float* x, const float* expert_weights, const int32_t* offsets,
                              const int32_t* sorted_route, const float* route_weights,
                              float* x_permuted, float* y_permuted, float* y, int tokens,
                              int top_k, int experts, int hidden, int output, hipStream_t stream);

// ---- narrow-output strip GEMMs (strip.hip): N <= 128, K <= 256 ----
// Shape / alignment test shared by the strip entries (K and N multiples of 4,
// 16-byte aligned A and W).
bool strip_shape_ok(int k, int n, const void* a, const void* w);
// Grouped strips take up to 256 segments.
bool strip_segments_ok(int segments);
// The fused route preparation + expert GEMM also needs T <= 8192, E <= 256 and
// the route-id stage to fit in LDS.
bool strip_chain_ok(int tokens, int top_k, int experts, int k, int n, const void* x,
                    const void* w, const void* ids, const void* x_permuted);
hipError_t strip_dense(const float* a, const float* b, float* c, int m, int n, int k,
                       hipStream_t stream);
// rows_bound: upper bound on the total segment rows (sizes the grid only).
hipError_t strip_grouped(const float* x, const float* w, const int32_t* offsets, float* y,
                         int experts, int hidden, int output, long rows_bound, hipStream_t stream);
hipError_t strip_router_gate(const float* x, const float* router_weights, float* logits,
                             int32_t* ids, float* gate_weights, float* y_zero, int y_cols,
                             int tokens, int experts, int hidden, hipStream_t stream);
// ids (top_k routes of every token, all in [0, experts)) -> counts, offsets,
// cursors, stable route_pos, sorted_route (optional), x_permuted (optional),
// y_permuted and, when y is given (top_k = 2 only), y += w * y_permuted with
// y zeroed beforehand, in one launch.
hipError_t strip_chain(const float* x, const float* expert_weights, const int32_t* ids,
                       const float* route_weights, int32_t* counts, int32_t* offsets,
                       int32_t* cursors, int32_t* route_pos, int32_t* sorted_route,
                       float* x_permuted, float* y_permuted, float* y, int tokens, int top_k,
                       int experts, int hidden, int output, hipStream_t stream);

// ---- routing kernels (routing.hip) ----
// y_zero (optional): [tokens, y_cols] rows zeroed by the same launch (chain fusion).
hipError_t topk_gate_wave(const float* logits, int32_t* ids, float* weights, int tokens,
                          int experts, hipStream_t stream, float* y_zero = nullptr,
                          int y_cols = 0);
// counts[e] = #{ids == e}; overwrites counts (no external reset needed).
hipError_t histogram_native(const int32_t* ids, int32_t* counts, int route_pairs, int experts,
                            hipStream_t stream);
// offsets[0..E] exclusive prefix of counts; in-place safe (counts == offsets).
hipError_t exclusive_scan_native(const int32_t* counts, int32_t* offsets, int experts,
                                 hipStream_t stream);
hipError_t histogram_exclusive_scan_native(const int32_t* ids, int32_t* counts, int32_t* offsets,
                                           int route_pairs, int experts, hipStream_t stream);
// Stable placement (route index ascending inside each expert segment) and
// token-owned row copy; cursors end equal to the per-expert route counts.
hipError_t token_permute_stable(const float* x, const int32_t* ids, const int32_t* offsets,
                                int32_t* cursors, float* x_permuted, int32_t* route_pos,
                                int32_t* sorted_route, int tokens, int experts, int top_k,
                                int hidden, hipStream_t stream);
// Fused-chain route preparation: ids -> counts, offsets, stable route_pos,
// sorted_route (required here) and cursors in one launch.
hipError_t route_prep(const int32_t* ids, int32_t* counts, int32_t* offsets, int32_t* cursors,
                      int32_t* route_pos, int32_t* sorted_route, int routes, int experts,
                      hipStream_t stream);
// Token-owned row copy x -> x_permuted through route_pos (second half of token_permute).
hipError_t permute_copy(const float* x, const int32_t* route_pos, float* x_permuted, int tokens,
                        int top_k, int hidden, hipStream_t stream);
hipError_t unpermute_gather(const float* y_permuted, const int32_t* route_pos,
                            const float* route_weights, float* y, int tokens, int top_k,
                            int output, hipStream_t stream);

// ---- naive baselines (naive.hip): reference semantics, no resets ----
hipError_t dense_gemm_naive(const float* a, const float* b, float* c, int m, int n, int k,
                            hipStream_t stream);
hipError_t topk_gate_naive(const float* logits, int32_t* ids, float* weights, int tokens,
                           int experts, hipStream_t stream);
hipError_t histogram_naive(const int32_t* ids, int32_t* counts, int route_pairs, int experts,
                           hipStream_t stream);
hipError_t exclusive_scan_naive(const int32_t* counts, int32_t* offsets, int experts,
                                hipStream_t stream);
// experts bounds the ids used to index offsets (INT_MAX: trust the ids).
hipError_t token_permute_naive(const float* x, const int32_t* ids, const int32_t* offsets,
                               int32_t* cursors, float* x_permuted, int32_t* route_pos,
                               int32_t* sorted_route, int tokens, int top_k, int hidden,
                               int experts, hipStream_t stream);
hipError_t grouped_gemm_naive(const float* x, const float* w, const int32_t* offsets, float* y,
                              int experts, int hidden, int output, int max_expert_tokens,
                              hipStream_t stream);
hipError_t unpermute_naive(const float* y_permuted, const int32_t* route_pos,
                           const float* route_weights, float* y, int tokens, int top_k,
                           int output, hipStream_t stream);

// ---- support (support.hip) ----
hipError_t cache_scrub(uint32_t* buffer, std::size_t elements, hipStream_t stream);
hipError_t fill_uniform(float* out, std::size_t count, uint64_t seed, uint64_t stream_id,
                        float low, float high, hipStream_t stream);
hipError_t fill_normal(float* out, std::size_t count, uint64_t seed, uint64_t stream_id,
                       float mean, float stddev, hipStream_t stream);

}  // namespace rr::kern
