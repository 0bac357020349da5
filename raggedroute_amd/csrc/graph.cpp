// Chain graphs: one chain call, or a sequence of chain calls (one per MoE
// layer of a model step, say), captured into an executable HIP graph and
// replayed with a single hipGraphLaunch (the reference's CUDA-graph chain variants,
// benchmarks/adapters/chain_adapter.cpp:730-826 fixed capture / exec update,
// :962-1000 shape cache; postroute_chain_adapter.cpp the same for the
// post-route chain).
//
// Only the auto / optimized family is captured: its launches are kernels
// only. The naive family resets counters with hipMemsetAsync, and memset
// nodes are kept out of graphs. A graph bakes every kernel argument (pointers,
// sizes) at capture; the device buffers must outlive it, and their contents
// are read at replay time. Graph and cache objects are not thread-safe.
//
// On ROCm 7.2 one hipGraphLaunch has a fixed cost (measured on MI355X: about
// 19 us of host time and 5 us of GPU time before the first node) that a graph
// of one headline chain (two kernels, ~20 us) does not win back; a sequence
// of ten or more chains per graph runs at the direct calls' GPU time with a
// fraction of their host submission time. A graph of at most kDirectCalls
// chains is therefore replayed by launching its recorded kernel nodes one by
// one (same kernels, grids and argument values, in capture order) instead of
// through hipGraphLaunch (RR_CHAIN_GRAPH_DIRECT=off keeps hipGraphLaunch).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "common.h"

struct rr_chain_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int32_t entry = 0;
  int32_t calls = 1;  // chain calls recorded, in order
  int32_t kernel_nodes = 0;
  // short sequences: the kernel nodes in launch order, replayed directly
  // (their argument buffers belong to `graph`); empty: hipGraphLaunch
  std::vector<hipKernelNodeParams> direct;
};

namespace rr {
namespace {

bool optimized_family(const rr_kernel_selection& k) noexcept {
  return k.family == RR_FAMILY_AUTO || k.family == RR_FAMILY_OPTIMIZED;
}

rr_status check_call(int32_t entry, const void* args, const rr_runtime_context* context) noexcept {
  if (args == nullptr) return invalid_argument("chain graph args must not be null");
  if (context == nullptr) return invalid_argument("no runtime context was given");
  if (context->stream == nullptr) {
    return invalid_argument("chain graph capture needs a non-default stream");
  }
  if (entry == RR_CHAIN_FROM_TOKENS || entry == RR_CHAIN_FROM_LOGITS) {
    if (!optimized_family(static_cast<const rr_chain_args*>(args)->kernel)) {
      return invalid_argument("chain graphs capture the auto / optimized family only");
    }
  } else if (entry == RR_CHAIN_FROM_ROUTE_IDS) {
    if (!optimized_family(static_cast<const rr_route_chain_args*>(args)->kernel)) {
      return invalid_argument("chain graphs capture the auto / optimized family only");
    }
  } else {
    return invalid_argument("unknown chain entry");
  }
  return ok_status();
}

rr_status run_entry(int32_t entry, const void* args, const rr_runtime_context* context) noexcept {
  switch (entry) {
    case RR_CHAIN_FROM_TOKENS:
      return rr_chain_from_tokens(static_cast<const rr_chain_args*>(args), context);
    case RR_CHAIN_FROM_LOGITS:
      return rr_chain_from_logits(static_cast<const rr_chain_args*>(args), context);
    default:
      return rr_chain_from_route_ids(static_cast<const rr_route_chain_args*>(args), context);
  }
}

// Records `count` calls of one entry, in order, on context->stream
// (thread-local capture) into *graph.
rr_status capture(int32_t entry, const void* const* args, int32_t count,
                  const rr_runtime_context* context, hipGraph_t* graph) noexcept {
  *graph = nullptr;
  hipError_t err = hipStreamBeginCapture(context->stream, hipStreamCaptureModeThreadLocal);
  if (err != hipSuccess) return device_status(err, "chain graph capture could not begin");
  rr_status status = ok_status();
  for (int32_t i = 0; i < count && status.code == RR_STATUS_SUCCESS; ++i) {
    status = run_entry(entry, args[i], context);
  }
  hipGraph_t captured = nullptr;
  err = hipStreamEndCapture(context->stream, &captured);
  if (status.code != RR_STATUS_SUCCESS) {
    if (captured != nullptr) (void)hipGraphDestroy(captured);
    return status;
  }
  if (err != hipSuccess) {
    if (captured != nullptr) (void)hipGraphDestroy(captured);
    return device_status(err, "chain graph capture failed");
  }
  *graph = captured;
  return ok_status();
}

rr_status check_calls(int32_t entry, const void* const* args, int32_t count,
                      const rr_runtime_context* context) noexcept {
  if (args == nullptr || count < 1 || count > 4096) {
    return invalid_argument("chain graph needs 1 to 4096 calls and their args");
  }
  for (int32_t i = 0; i < count; ++i) {
    const rr_status status = check_call(entry, args[i], context);
    if (status.code != RR_STATUS_SUCCESS) return status;
  }
  return ok_status();
}

int32_t count_kernel_nodes(hipGraph_t graph) noexcept {
  size_t count = 0;
  if (hipGraphGetNodes(graph, nullptr, &count) != hipSuccess || count == 0) return 0;
  std::vector<hipGraphNode_t> nodes(count);
  if (hipGraphGetNodes(graph, nodes.data(), &count) != hipSuccess) return 0;
  int32_t kernels = 0;
  for (size_t i = 0; i < count; ++i) {
    hipGraphNodeType type{};
    if (hipGraphNodeGetType(nodes[i], &type) == hipSuccess && type == hipGraphNodeTypeKernel) {
      ++kernels;
    }
  }
  return kernels;
}

constexpr int32_t kDirectCalls = 2;

bool direct_allowed() noexcept {
  static const bool allowed = [] {
    const char* v = std::getenv("RR_CHAIN_GRAPH_DIRECT");
    return v == nullptr || std::strcmp(v, "off") != 0;
  }();
  return allowed;
}

// The kernel nodes of a captured single-stream sequence in launch order: one
// root, each node with at most one dependent, every node a kernel node. Any
// other shape leaves `out` empty (the graph is then replayed by hipGraphLaunch).
void collect_direct(hipGraph_t graph, std::vector<hipKernelNodeParams>* out) noexcept {
  out->clear();
  size_t total = 0;
  size_t roots = 0;
  if (hipGraphGetNodes(graph, nullptr, &total) != hipSuccess || total == 0) return;
  if (hipGraphGetRootNodes(graph, nullptr, &roots) != hipSuccess || roots != 1) return;
  hipGraphNode_t node = nullptr;
  if (hipGraphGetRootNodes(graph, &node, &roots) != hipSuccess) return;
  std::vector<hipKernelNodeParams> order;
  while (node != nullptr && order.size() < total) {
    hipGraphNodeType type{};
    hipKernelNodeParams p{};
    if (hipGraphNodeGetType(node, &type) != hipSuccess || type != hipGraphNodeTypeKernel ||
        hipGraphKernelNodeGetParams(node, &p) != hipSuccess || p.extra != nullptr) {
      return;
    }
    order.push_back(p);
    size_t deps = 0;
    if (hipGraphNodeGetDependentNodes(node, nullptr, &deps) != hipSuccess || deps > 1) return;
    hipGraphNode_t next = nullptr;
    if (deps == 1 && hipGraphNodeGetDependentNodes(node, &next, &deps) != hipSuccess) return;
    node = deps == 1 ? next : nullptr;
  }
  if (node != nullptr || order.size() != total) return;
  *out = std::move(order);
}

rr_status instantiate(rr_chain_graph* g, hipStream_t stream) noexcept {
  hipError_t err = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (err != hipSuccess) {
    g->exec = nullptr;
    return device_status(err, "chain graph instantiation failed");
  }
  err = hipGraphUpload(g->exec, stream);
  if (err != hipSuccess) return device_status(err, "chain graph upload failed");
  return ok_status();
}

void release(rr_chain_graph* g) noexcept {
  if (g == nullptr) return;
  if (g->exec != nullptr) (void)hipGraphExecDestroy(g->exec);
  if (g->graph != nullptr) (void)hipGraphDestroy(g->graph);
  g->exec = nullptr;
  g->graph = nullptr;
}

rr_status create(int32_t entry, const void* const* args, int32_t count,
                 const rr_runtime_context* context, rr_chain_graph** out) noexcept {
  if (out == nullptr) return invalid_argument("chain graph output handle must not be null");
  *out = nullptr;
  rr_status status = check_calls(entry, args, count, context);
  if (status.code != RR_STATUS_SUCCESS) return status;
  auto* g = new (std::nothrow) rr_chain_graph;
  if (g == nullptr) return make_status(RR_STATUS_DEVICE_ERROR, "chain graph allocation failed");
  g->entry = entry;
  g->calls = count;
  status = capture(entry, args, count, context, &g->graph);
  if (status.code == RR_STATUS_SUCCESS) status = instantiate(g, context->stream);
  if (status.code != RR_STATUS_SUCCESS) {
    release(g);
    delete g;
    return status;
  }
  g->kernel_nodes = count_kernel_nodes(g->graph);
  if (count <= kDirectCalls && direct_allowed()) collect_direct(g->graph, &g->direct);
  *out = g;
  return ok_status();
}

// New arguments for an existing graph (same entry, same number of calls):
// capture them and update the executable in place when the topology
// matches, else instantiate anew.
rr_status update(rr_chain_graph* g, const void* const* args, int32_t count,
                 const rr_runtime_context* context) noexcept {
  if (g == nullptr) return invalid_argument("chain graph must not be null");
  if (count != g->calls) return invalid_argument("chain graph update needs as many calls as were captured");
  rr_status status = check_calls(g->entry, args, count, context);
  if (status.code != RR_STATUS_SUCCESS) return status;
  hipGraph_t fresh = nullptr;
  status = capture(g->entry, args, count, context, &fresh);
  if (status.code != RR_STATUS_SUCCESS) return status;
  hipGraphNode_t error_node = nullptr;
  hipGraphExecUpdateResult result = hipGraphExecUpdateError;
  const hipError_t err = hipGraphExecUpdate(g->exec, fresh, &error_node, &result);
  g->direct.clear();  // (its argument buffers belong to the graph destroyed here)
  (void)hipGraphDestroy(g->graph);
  g->graph = fresh;
  g->kernel_nodes = count_kernel_nodes(fresh);
  if (count <= kDirectCalls && direct_allowed()) collect_direct(fresh, &g->direct);
  if (err == hipSuccess && result == hipGraphExecUpdateSuccess) return ok_status();
  (void)hipGetLastError();  // a rejected update is not a device error
  (void)hipGraphExecDestroy(g->exec);
  g->exec = nullptr;
  return instantiate(g, context->stream);
}

// ---- shape cache ----
struct CacheEntry {
  std::vector<int64_t> key;
  rr_chain_graph* graph = nullptr;
  uint64_t last_use = 0;
};

void push_view(std::vector<int64_t>& key, const void* p) {
  key.push_back(static_cast<int64_t>(reinterpret_cast<std::uintptr_t>(p)));
}

// Every field that shapes the captured launches: pointers, sizes, kernel
// selection, workspace and architecture (the stream is not part of a graph).
std::vector<int64_t> cache_key(int32_t entry, const void* args, const rr_runtime_context* c) {
  std::vector<int64_t> key;
  key.push_back(entry);
  if (entry == RR_CHAIN_FROM_ROUTE_IDS) {
    const auto* a = static_cast<const rr_route_chain_args*>(args);
    for (const void* p : {static_cast<const void*>(a->x), static_cast<const void*>(a->expert_ids),
                          static_cast<const void*>(a->route_weights),
                          static_cast<const void*>(a->expert_weights), static_cast<const void*>(a->counts),
                          static_cast<const void*>(a->offsets), static_cast<const void*>(a->x_permuted),
                          static_cast<const void*>(a->route_pos), static_cast<const void*>(a->sorted_route),
                          static_cast<const void*>(a->y_permuted), static_cast<const void*>(a->y)}) {
      push_view(key, p);
    }
    for (int64_t v : {a->tokens, a->experts, a->top_k, a->hidden, a->output}) key.push_back(v);
    key.push_back(a->kernel.family);
    key.push_back(a->kernel.implementation_id);
  } else {
    const auto* a = static_cast<const rr_chain_args*>(args);
    for (const void* p : {static_cast<const void*>(a->x), static_cast<const void*>(a->router_weights),
                          static_cast<const void*>(a->logits), static_cast<const void*>(a->expert_ids),
                          static_cast<const void*>(a->route_weights), static_cast<const void*>(a->counts),
                          static_cast<const void*>(a->offsets), static_cast<const void*>(a->x_permuted),
                          static_cast<const void*>(a->route_pos), static_cast<const void*>(a->sorted_route),
                          static_cast<const void*>(a->expert_weights), static_cast<const void*>(a->y_permuted),
                          static_cast<const void*>(a->y)}) {
      push_view(key, p);
    }
    for (int64_t v : {a->tokens, a->experts, a->top_k, a->hidden, a->output}) key.push_back(v);
    key.push_back(a->kernel.family);
    key.push_back(a->kernel.implementation_id);
  }
  push_view(key, c->workspace);
  key.push_back(static_cast<int64_t>(c->workspace_bytes));
  key.push_back(c->architecture);
  return key;
}

}  // namespace
}  // namespace rr

struct rr_chain_graph_cache {
  std::vector<rr::CacheEntry> entries;
  int32_t capacity = 16;
  uint64_t clock = 0;
  int64_t hits = 0;
  int64_t misses = 0;
};

extern "C" {

rr_status rr_chain_graph_create(int32_t entry, const void* args, const rr_runtime_context* context,
                                rr_chain_graph** graph) {
  return rr::create(entry, &args, 1, context, graph);
}

rr_status rr_chain_graph_create_sequence(int32_t entry, const void* const* args, int32_t count,
                                         const rr_runtime_context* context, rr_chain_graph** graph) {
  return rr::create(entry, args, count, context, graph);
}

rr_status rr_chain_graph_launch(rr_chain_graph* graph, hipStream_t stream) {
  if (graph == nullptr || graph->exec == nullptr) return rr::invalid_argument("chain graph must not be null");
  if (!graph->direct.empty()) {
    for (const hipKernelNodeParams& p : graph->direct) {
      const hipError_t err = hipLaunchKernel(p.func, p.gridDim, p.blockDim, p.kernelParams, p.sharedMemBytes, stream);
      if (err != hipSuccess) return rr::device_status(err, "chain graph launch failed");
    }
    return rr::ok_status();
  }
  return rr::device_status(hipGraphLaunch(graph->exec, stream), "chain graph launch failed");
}

rr_status rr_chain_graph_update(rr_chain_graph* graph, const void* args,
                                const rr_runtime_context* context) {
  return rr::update(graph, &args, 1, context);
}

rr_status rr_chain_graph_update_sequence(rr_chain_graph* graph, const void* const* args, int32_t count,
                                         const rr_runtime_context* context) {
  return rr::update(graph, args, count, context);
}

int32_t rr_chain_graph_kernel_nodes(const rr_chain_graph* graph) {
  return graph == nullptr ? 0 : graph->kernel_nodes;
}

void rr_chain_graph_destroy(rr_chain_graph* graph) {
  rr::release(graph);
  delete graph;
}

rr_status rr_chain_graph_cache_create(int32_t capacity, rr_chain_graph_cache** cache) {
  if (cache == nullptr) return rr::invalid_argument("chain graph cache output handle must not be null");
  *cache = nullptr;
  if (capacity < 1 || capacity > 4096) return rr::invalid_argument("chain graph cache capacity must be in [1, 4096]");
  auto* c = new (std::nothrow) rr_chain_graph_cache;
  if (c == nullptr) return rr::make_status(RR_STATUS_DEVICE_ERROR, "chain graph cache allocation failed");
  c->capacity = capacity;
  *cache = c;
  return rr::ok_status();
}

rr_status rr_chain_graph_cache_launch(rr_chain_graph_cache* cache, int32_t entry, const void* args,
                                      const rr_runtime_context* context) {
  if (cache == nullptr) return rr::invalid_argument("chain graph cache must not be null");
  rr_status status = rr::check_call(entry, args, context);
  if (status.code != RR_STATUS_SUCCESS) return status;
  std::vector<int64_t> key;
  try {
    key = rr::cache_key(entry, args, context);
  } catch (...) {
    return rr::make_status(RR_STATUS_DEVICE_ERROR, "chain graph cache allocation failed");
  }
  ++cache->clock;
  for (auto& e : cache->entries) {
    if (e.key == key) {
      e.last_use = cache->clock;
      ++cache->hits;
      return rr_chain_graph_launch(e.graph, context->stream);
    }
  }
  rr_chain_graph* g = nullptr;
  status = rr::create(entry, &args, 1, context, &g);
  if (status.code != RR_STATUS_SUCCESS) return status;
  ++cache->misses;
  try {
    if (static_cast<int32_t>(cache->entries.size()) == cache->capacity) {
      auto lru = cache->entries.begin();
      for (auto it = cache->entries.begin(); it != cache->entries.end(); ++it) {
        if (it->last_use < lru->last_use) lru = it;
      }
      rr_chain_graph_destroy(lru->graph);
      lru->graph = g;
      lru->key = std::move(key);
      lru->last_use = cache->clock;
    } else {
      cache->entries.push_back(rr::CacheEntry{std::move(key), g, cache->clock});
    }
  } catch (...) {
    rr_chain_graph_destroy(g);
    return rr::make_status(RR_STATUS_DEVICE_ERROR, "chain graph cache allocation failed");
  }
  return rr_chain_graph_launch(g, context->stream);
}

void rr_chain_graph_cache_get_stats(const rr_chain_graph_cache* cache, rr_chain_graph_cache_stats* out) {
  if (out == nullptr) return;
  std::memset(out, 0, sizeof(*out));
  if (cache == nullptr) return;
  out->capacity = cache->capacity;
  out->entries = static_cast<int32_t>(cache->entries.size());
  out->hits = cache->hits;
  out->misses = cache->misses;
}

void rr_chain_graph_cache_destroy(rr_chain_graph_cache* cache) {
  if (cache == nullptr) return;
  for (auto& e : cache->entries) rr_chain_graph_destroy(e.graph);
  delete cache;
}

}  // extern "C"
