// raggedroute/chain.h - chain entries. The reference defines chain_from_tokens
// and chain_from_logits only as benchmark suites (reference
// benchmarks/adapters/chain_adapter.cpp:263-467); this build adds them as
// library entries that enqueue every stage on the caller's stream.
//
// Memory contract of `y` (auto / optimized family): the fused chain zeroes y
// in its first launch and adds both weighted routes of each token into it
// with hardware FP32 atomic adds. y must be device memory of the GPU that runs
// the chain, from hipMalloc or an allocator built on it (coarse-grained). Not
// supported for y on that path: fine-grained device memory, host memory
// (hipHostMalloc, registered, managed) and peer memory mapped over xGMI. Use
// KernelFamily::kNaive or chain_from_route_ids (plain stores) for those. Every
// element gets exactly two adds into zero, so the result is deterministic and
// bit-identical to the rank-order unpermute, subnormal products included.
#pragma once

#include <cstddef>
#include <cstdint>

#include "raggedroute/detail/capi_bridge.h"
#include "raggedroute/runtime.h"
#include "raggedroute/status.h"
#include "raggedroute/types.h"

namespace raggedroute {

struct ChainArgs {
  const float* x = nullptr;               // [tokens, hidden]
  const float* router_weights = nullptr;  // [hidden, experts]; chain_from_tokens only
  float* logits = nullptr;                // [tokens, experts]; output (tokens) / input (logits)
  std::int32_t* expert_ids = nullptr;     // [tokens, 2]
  float* route_weights = nullptr;         // [tokens, 2]
  std::int32_t* counts = nullptr;         // [experts]
  std::int32_t* offsets = nullptr;        // [experts + 1]
  float* x_permuted = nullptr;            // [tokens * 2, hidden]
  std::int32_t* route_pos = nullptr;      // [tokens * 2]
  std::int32_t* sorted_route = nullptr;   // [tokens * 2], optional
  const float* expert_weights = nullptr;  // [experts, hidden, output]
  float* y_permuted = nullptr;            // [tokens * 2, output]
  float* y = nullptr;                     // [tokens, output]
  int tokens = 0;
  int experts = 0;
  int top_k = 2;
  int hidden = 0;
  int output = 0;
  KernelSelection kernel;
};

namespace detail {
inline rr_chain_args to_c(const ChainArgs& a) noexcept {
  rr_chain_args c{};
  c.x = a.x;
  c.router_weights = a.router_weights;
  c.logits = a.logits;
  c.expert_ids = a.expert_ids;
  c.route_weights = a.route_weights;
  c.counts = a.counts;
  c.offsets = a.offsets;
  c.x_permuted = a.x_permuted;
  c.route_pos = a.route_pos;
  c.sorted_route = a.sorted_route;
  c.expert_weights = a.expert_weights;
  c.y_permuted = a.y_permuted;
  c.y = a.y;
  c.tokens = a.tokens;
  c.experts = a.experts;
  c.top_k = a.top_k;
  c.hidden = a.hidden;
  c.output = a.output;
  c.kernel = to_c(a.kernel);
  return c;
}
}  // namespace detail

inline std::size_t get_chain_workspace_size(const ChainArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_chain_workspace_size(&c);
}

inline Status chain_from_tokens(const ChainArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_chain_from_tokens(&a, &c));
}

inline Status chain_from_logits(const ChainArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_chain_from_logits(&a, &c));
}

// Post-route chain (reference chain_from_route_ids suite,
// benchmarks/adapters/postroute_chain_adapter.cpp:250-356).
struct RouteChainArgs {
  const float* x = nullptr;               // [tokens, hidden]
  const std::int32_t* expert_ids = nullptr;  // [tokens, top_k]
  const float* route_weights = nullptr;   // [tokens, top_k]
  const float* expert_weights = nullptr;  // [experts, hidden, output]
  std::int32_t* counts = nullptr;         // [experts]
  std::int32_t* offsets = nullptr;        // [experts + 1]
  float* x_permuted = nullptr;            // [tokens * top_k, hidden]; optional (auto / optimized)
  std::int32_t* route_pos = nullptr;      // [tokens * top_k]
  std::int32_t* sorted_route = nullptr;   // [tokens * top_k], optional
  float* y_permuted = nullptr;            // [tokens * top_k, output]
  float* y = nullptr;                     // [tokens, output]
  int tokens = 0;
  int experts = 0;
  int top_k = 2;
  int hidden = 0;
  int output = 0;
  KernelSelection kernel;
};

namespace detail {
inline rr_route_chain_args to_c(const RouteChainArgs& a) noexcept {
  rr_route_chain_args c{};
  c.x = a.x;
  c.expert_ids = a.expert_ids;
  c.route_weights = a.route_weights;
  c.expert_weights = a.expert_weights;
  c.counts = a.counts;
  c.offsets = a.offsets;
  c.x_permuted = a.x_permuted;
  c.route_pos = a.route_pos;
  c.sorted_route = a.sorted_route;
  c.y_permuted = a.y_permuted;
  c.y = a.y;
  c.tokens = a.tokens;
  c.experts = a.experts;
  c.top_k = a.top_k;
  c.hidden = a.hidden;
  c.output = a.output;
  c.kernel = to_c(a.kernel);
  return c;
}
}  // namespace detail

inline std::size_t get_route_chain_workspace_size(const RouteChainArgs& args) noexcept {
  const auto c = detail::to_c(args);
  return rr_route_chain_workspace_size(&c);
}

inline Status chain_from_route_ids(const RouteChainArgs& args, const RuntimeContext& context) noexcept {
  const auto a = detail::to_c(args);
  const auto c = detail::to_c(context);
  return detail::from_c(rr_chain_from_route_ids(&a, &c));
}

// One chain call captured into an executable HIP graph (auto / optimized
// family). Move-only owner of an rr_chain_graph.
class ChainGraph {
 public:
  ChainGraph() = default;
  ChainGraph(const ChainGraph&) = delete;
  ChainGraph& operator=(const ChainGraph&) = delete;
  ChainGraph(ChainGraph&& other) noexcept : graph_(other.graph_) { other.graph_ = nullptr; }
  ChainGraph& operator=(ChainGraph&& other) noexcept {
    if (this != &other) {
      rr_chain_graph_destroy(graph_);
      graph_ = other.graph_;
      other.graph_ = nullptr;
    }
    return *this;
  }
  ~ChainGraph() { rr_chain_graph_destroy(graph_); }

  Status capture_from_tokens(const ChainArgs& args, const RuntimeContext& context) noexcept {
    return capture(RR_CHAIN_FROM_TOKENS, detail::to_c(args), context);
  }
  Status capture_from_logits(const ChainArgs& args, const RuntimeContext& context) noexcept {
    return capture(RR_CHAIN_FROM_LOGITS, detail::to_c(args), context);
  }
  Status capture_from_route_ids(const RouteChainArgs& args, const RuntimeContext& context) noexcept {
    return capture(RR_CHAIN_FROM_ROUTE_IDS, detail::to_c(args), context);
  }
  Status launch(hipStream_t stream) noexcept {
    return detail::from_c(rr_chain_graph_launch(graph_, stream));
  }
  int kernel_nodes() const noexcept { return rr_chain_graph_kernel_nodes(graph_); }

 private:
  template <class CArgs>
  Status capture(int entry, const CArgs& c_args, const RuntimeContext& context) noexcept {
    rr_chain_graph_destroy(graph_);
    graph_ = nullptr;
    const auto c = detail::to_c(context);
    return detail::from_c(rr_chain_graph_create(entry, &c_args, &c, &graph_));
  }
  rr_chain_graph* graph_ = nullptr;
};

}  // namespace raggedroute
