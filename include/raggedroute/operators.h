// raggedroute/operators.h - v0.2 operator API (reference include/raggedroute/operators.h:10-137).
//
// Same names, Args fields and signatures as the reference. Each function is an
// inline forwarder to the C ABI in raggedroute_capi.h; the work runs in the
// gfx950 library. Unless a field says otherwise, non-null pointers are HIP
// device pointers. v0.2 requires zero-stride contiguous row-major FP32 storage,
// valid route ids in [0, experts), monotonic offsets with offsets[experts]
// equal to the route count, and non-overlapping input/output buffers. Expert
// counts up to 1024 are accepted (the reference caps at 64).
#pragma once

#include <cstddef>
#include <cstdint>

#include "raggedroute/detail/capi_bridge.h"
#include "raggedroute/runtime.h"
#include "raggedroute/status.h"
#include "raggedroute/types.h"

namespace raggedroute {

struct DenseGemmArgs {
  ConstTensorView a;
  ConstTensorView b;
  MutableTensorView c;
  int m = 0;
  int n = 0;
  int k = 0;
  float alpha = 1.0F;
  float beta = 0.0F;
  ScalarType accumulator_dtype = ScalarType::kFp32;
  KernelSelection kernel;
};

struct TopKGateArgs {
  ConstTensorView logits;
  std::int32_t* expert_ids = nullptr;
  MutableTensorView weights;
  int tokens = 0;
  int experts = 0;
  int top_k = 2;
  ScalarType accumulator_dtype = ScalarType::kFp32;
  TopKNormalization normalization = TopKNormalization::kSelectedSoftmax;
  TopKTieBreak tie_break = TopKTieBreak::kLowerExpertId;
  TopKNaNPolicy nan_policy = TopKNaNPolicy::kNegativeInfinityAllNaNFallback01;
  KernelSelection kernel;
};

struct HistogramArgs {
  const std::int32_t* expert_ids = nullptr;
  std::int32_t* counts = nullptr;
  int route_pairs = 0;
  int experts = 0;
  KernelSelection kernel;
};

struct ExclusiveScanArgs {
  const std::int32_t* counts = nullptr;
  std::int32_t* offsets = nullptr;
  int experts = 0;
  KernelSelection kernel;
};

// Fused routing-metadata primitive; input and both outputs pairwise non-overlapping.
struct HistogramExclusiveScanArgs {
  const std::int32_t* expert_ids = nullptr;
  std::int32_t* counts = nullptr;
  std::int32_t* offsets = nullptr;
  int route_pairs = 0;
  int experts = 0;
  KernelSelection kernel;
};

struct TokenPermuteArgs {
  ConstTensorView x;
  const std::int32_t* expert_ids = nullptr;
  const std::int32_t* offsets = nullptr;
  MutableTensorView x_permuted;
  std::int32_t* route_pos = nullptr;
  // Optional inverse mapping: sorted_route[route_pos[r]] == r.
  std::int32_t* sorted_route = nullptr;
  int tokens = 0;
  int experts = 0;
  int top_k = 0;
  int hidden = 0;
  KernelSelection kernel;
};

struct GroupedGemmArgs {
  ConstTensorView x_permuted;
  ConstTensorView expert_weights;
  const std::int32_t* offsets = nullptr;
  MutableTensorView y_permuted;
  int experts = 0;
  int hidden = 0;
  int output = 0;
  // Caller-provided launch bound; offsets are never read on the host.
  int max_expert_tokens = 0;
  ScalarType accumulator_dtype = ScalarType::kFp32;
  KernelSelection kernel;
};

struct UnpermuteArgs {
  ConstTensorView y_permuted;
  const std::int32_t* route_pos = nullptr;
  ConstTensorView route_weights;
  MutableTensorView y;
  int tokens = 0;
  int top_k = 0;
  int output = 0;
  ScalarType accumulator_dtype = ScalarType::kFp32;
  KernelSelection kernel;
};

namespace detail {

inline rr_dense_gemm_args to_c(const DenseGemmArgs& a) noexcept {
  return {to_c(a.a), to_c(a.b), to_c(a.c), a.m, a.n, a.k, a.alpha, a.beta,
          static_cast<int32_t>(a.accumulator_dtype), to_c(a.kernel)};
}
inline rr_topk_gate_args to_c(const TopKGateArgs& a) noexcept {
  return {to_c(a.logits), a.expert_ids, to_c(a.weights), a.tokens, a.experts, a.top_k,
          static_cast<int32_t>(a.accumulator_dtype), static_cast<int32_t>(a.normalization),
          static_cast<int32_t>(a.tie_break), static_cast<int32_t>(a.nan_policy),
          to_c(a.kernel)};
}
inline rr_histogram_args to_c(const HistogramArgs& a) noexcept {
  return {a.expert_ids, a.counts, a.route_pairs, a.experts, to_c(a.kernel)};
}
inline rr_exclusive_scan_args to_c(const ExclusiveScanArgs& a) noexcept {
  return {a.counts, a.offsets, a.experts, to_c(a.kernel)};
}
inline rr_histogram_exclusive_scan_args to_c(const HistogramExclusiveScanArgs& a) noexcept {
  return {a.expert_ids, a.counts, a.offsets, a.route_pairs, a.experts, to_c(a.kernel)};
}
inline rr_token_permute_args to_c(const TokenPermuteArgs& a) noexcept {
  return {to_c(a.x),  a.expert_ids, a.offsets, to_c(a.x_permuted), a.route_pos, a.sorted_route,
          a.tokens,   a.experts,    a.top_k,   a.hidden,           to_c(a.kernel)};
}
inline rr_grouped_gemm_args to_c(const GroupedGemmArgs& a) noexcept {
  return {to_c(a.x_permuted), to_c(a.expert_weights), a.offsets, to_c(a.y_permuted),
          a.experts, a.hidden, a.output, a.max_expert_tokens,
          static_cast<int32_t>(a.accumulator_dtype), to_c(a.kernel)};
}
inline rr_unpermute_args to_c(const UnpermuteArgs& a) noexcept {
  return {to_c(a.y_permuted), a.route_pos, to_c(a.route_weights), to_c(a.y), a.tokens, a.top_k,
          a.output, static_cast<int32_t>(a.accumulator_dtype), to_c(a.kernel)};
}

}  // namespace detail

// Workspace queries (reference operators.h:114-122): zero for every operator
// except token_permute, which needs experts * sizeof(int32) cursor words.
inline std::size_t get_dense_gemm_workspace_size(const DenseGemmArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_dense_gemm_workspace_size(&c);
}
inline std::size_t get_topk_gate_workspace_size(const TopKGateArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_topk_gate_workspace_size(&c);
}
inline std::size_t get_histogram_workspace_size(const HistogramArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_histogram_workspace_size(&c);
}
inline std::size_t get_exclusive_scan_workspace_size(const ExclusiveScanArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_exclusive_scan_workspace_size(&c);
}
inline std::size_t get_histogram_exclusive_scan_workspace_size(
    const HistogramExclusiveScanArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_histogram_exclusive_scan_workspace_size(&c);
}
inline std::size_t get_token_permute_workspace_size(const TokenPermuteArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_token_permute_workspace_size(&c);
}
inline std::size_t get_grouped_gemm_workspace_size(const GroupedGemmArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_grouped_gemm_workspace_size(&c);
}
inline std::size_t get_unpermute_workspace_size(const UnpermuteArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_unpermute_workspace_size(&c);
}

// Complete operator wrappers (reference operators.h:124-135): caller stream, no
// hot-path allocation, no unconditional synchronisation, mandatory device-side
// resets inside the call boundary.
inline Status dense_gemm(const DenseGemmArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_dense_gemm(&a, &c));
}
inline Status topk_gate(const TopKGateArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_topk_gate(&a, &c));
}
inline Status histogram(const HistogramArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_histogram(&a, &c));
}
inline Status exclusive_scan(const ExclusiveScanArgs& args,
                             const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_exclusive_scan(&a, &c));
}
inline Status histogram_exclusive_scan(const HistogramExclusiveScanArgs& args,
                                       const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_histogram_exclusive_scan(&a, &c));
}
inline Status token_permute(const TokenPermuteArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_token_permute(&a, &c));
}
inline Status grouped_gemm(const GroupedGemmArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_grouped_gemm(&a, &c));
}
inline Status unpermute(const UnpermuteArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_unpermute(&a, &c));
}

}  // namespace raggedroute
