// Naive gfx950 baselines with the semantics of the reference cuda_naive
// launchers (reference src/*/cuda_naive/baseline.cu). They are the semantic
// floor behind KernelFamily::kNaive and the ops::launch_*_naive entries: one
// thread per output element, sequential FP32 accumulation, atomic placement in
// the permute. None of them resets its outputs; the operator wrappers do.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstddef>
#include <cstdint>

#include "launchers.h"

namespace rr::kern {
namespace {

constexpr unsigned kThreads = 256;
constexpr unsigned kMaxBlocks = 65535;

unsigned grid_for(std::size_t elements) {
  const std::size_t blocks = (elements + kThreads - 1) / kThreads;
  return static_cast<unsigned>(blocks < kMaxBlocks ? blocks : kMaxBlocks);
}

// reference src/dense_gemm/cuda_naive/baseline.cu:16-32
__global__ void rr_dense_gemm_naive_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                           float* __restrict__ c, int m, int n, int k) {
  const std::size_t total = static_cast<std::size_t>(m) * n;
  const std::size_t stride = static_cast<std::size_t>(blockDim.x) * gridDim.x;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += stride) {
    const std::size_t row = i / n;
    const std::size_t col = i % n;
    float acc = 0.0F;
    for (int p = 0; p < k; ++p) {
      acc = __fadd_rn(acc, __fmul_rn(a[row * k + p], b[static_cast<std::size_t>(p) * n + col]));
    }
    c[i] = acc;
  }
}

// reference src/topk_gate/cuda_naive/baseline.cu:18-22: (value desc, id asc) order.
__device__ inline bool precedes(float value, int id, float incumbent, int incumbent_id) {
  return incumbent_id < 0 || value > incumbent || (value == incumbent && id < incumbent_id);
}

// reference src/topk_gate/cuda_naive/baseline.cu:24-80
__global__ void rr_topk_gate_naive_kernel(const float* __restrict__ logits, int32_t* __restrict__ ids,
                                          float* __restrict__ weights, int tokens, int experts) {
  const std::size_t stride = static_cast<std::size_t>(blockDim.x) * gridDim.x;
  for (std::size_t t = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       t < static_cast<std::size_t>(tokens); t += stride) {
    float v1 = -INFINITY, v2 = -INFINITY;
    int e1 = -1, e2 = -1;
    bool saw_non_nan = false;
    const float* row = logits + t * experts;
    for (int e = 0; e < experts; ++e) {
      const float raw = row[e];
      const bool nan = isnan(raw);
      const float v = nan ? -INFINITY : raw;
      saw_non_nan = saw_non_nan || !nan;
      if (precedes(v, e, v1, e1)) {
        v2 = v1;
        e2 = e1;
        v1 = v;
        e1 = e;
      } else if (precedes(v, e, v2, e2)) {
        v2 = v;
        e2 = e;
      }
    }
    float w1, w2;
    if (!saw_non_nan || v1 == v2) {
      if (!saw_non_nan) {
        e1 = 0;
        e2 = 1;
      }
      w1 = 0.5F;
      w2 = 0.5F;
    } else if (v1 == INFINITY || v2 == -INFINITY) {
      w1 = 1.0F;
      w2 = 0.0F;
    } else {
      const float r = expf(v2 - v1);
      w1 = 1.0F / (1.0F + r);
      w2 = r * w1;
    }
    ids[2 * t] = e1;
    ids[2 * t + 1] = e2;
    weights[2 * t] = w1;
    weights[2 * t + 1] = w2;
  }
}

// reference src/histogram/cuda_naive/baseline.cu:17-27: out-of-range ids are ignored.
__global__ void rr_histogram_naive_kernel(const int32_t* __restrict__ ids, int32_t* counts,
                                          int route_pairs, int experts) {
  const std::size_t stride = static_cast<std::size_t>(blockDim.x) * gridDim.x;
  for (std::size_t r = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       r < static_cast<std::size_t>(route_pairs); r += stride) {
    const int32_t e = ids[r];
    if (e >= 0 && e < experts) atomicAdd(counts + e, 1);
  }
}

// reference src/scan/cuda_naive/baseline.cu:12-26: reads each count before
// writing its offset, so counts and offsets may alias (in-place scan).
__global__ void rr_exclusive_scan_naive_kernel(const int32_t* counts, int32_t* offsets,
                                               int experts) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  int32_t running = 0;
  for (int e = 0; e < experts; ++e) {
    const int32_t c = counts[e];
    offsets[e] = running;
    running += c;
  }
  offsets[experts] = running;
}

// reference src/permute/cuda_naive/baseline.cu:13-34: one block per route,
// destination = offsets[e] + atomic cursor (placement order is unspecified).
// Routes whose id lies outside [0, experts) or whose destination lies outside
// [0, routes) are not placed (route_pos = -1) instead of being dereferenced.
__global__ void rr_token_permute_naive_kernel(const float* __restrict__ x,
                                              const int32_t* __restrict__ ids,
                                              const int32_t* __restrict__ offsets, int32_t* cursors,
                                              float* __restrict__ x_permuted,
                                              int32_t* __restrict__ route_pos,
                                              int32_t* __restrict__ sorted_route, int routes,
                                              int top_k, int hidden, int experts) {
  const int route = static_cast<int>(blockIdx.x);
  if (route >= routes) return;
  __shared__ int destination;
  if (threadIdx.x == 0) {
    const int e = ids[route];
    int dest = -1;
    if (e >= 0 && e < experts) {
      dest = offsets[e] + atomicAdd(cursors + e, 1);
      if (dest < 0 || dest >= routes) dest = -1;
    }
    destination = dest;
    route_pos[route] = dest;
    if (sorted_route != nullptr && dest >= 0) sorted_route[dest] = route;
  }
  __syncthreads();
  if (destination < 0) return;
  const std::size_t token = static_cast<std::size_t>(route / top_k);
  for (int col = threadIdx.x; col < hidden; col += blockDim.x) {
    x_permuted[static_cast<std::size_t>(destination) * hidden + col] = x[token * hidden + col];
  }
}

// reference src/grouped_gemm/cuda_naive/baseline.cu:11-31: z = expert, y strides
// over the expert's rows, x = output column.
__global__ void rr_grouped_gemm_naive_kernel(const float* __restrict__ x,
                                             const float* __restrict__ w,
                                             const int32_t* __restrict__ offsets,
                                             float* __restrict__ y, int hidden, int output) {
  const int expert = static_cast<int>(blockIdx.z);
  const int col = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  const int begin = offsets[expert];
  const int end = offsets[expert + 1];
  if (col >= output) return;
  const int row_stride = static_cast<int>(gridDim.y * blockDim.y);
  const float* we = w + static_cast<std::size_t>(expert) * hidden * output;
  for (int local = static_cast<int>(blockIdx.y * blockDim.y + threadIdx.y); local < end - begin;
       local += row_stride) {
    const std::size_t row = static_cast<std::size_t>(begin + local);
    float acc = 0.0F;
    for (int p = 0; p < hidden; ++p) {
      acc = __fadd_rn(acc, __fmul_rn(x[row * hidden + p],
                                     we[static_cast<std::size_t>(p) * output + col]));
    }
    y[row * output + col] = acc;
  }
}

// reference src/unpermute/cuda_naive/baseline.cu:13-29
__global__ void rr_unpermute_naive_kernel(const float* __restrict__ y_permuted,
                                          const int32_t* __restrict__ route_pos,
                                          const float* __restrict__ route_weights,
                                          float* __restrict__ y, int tokens, int top_k,
                                          int output) {
  const int linear = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  if (linear >= tokens * output) return;
  const int token = linear / output;
  const int col = linear % output;
  const int routes = tokens * top_k;
  float acc = 0.0F;
  for (int j = 0; j < top_k; ++j) {
    const int route = token * top_k + j;
    const int32_t src = route_pos[route];
    if (src < 0 || src >= routes) continue;  // never dereference an out-of-range row
    acc = __fadd_rn(acc, __fmul_rn(route_weights[route],
                                   y_permuted[static_cast<std::size_t>(src) * output + col]));
  }
  y[linear] = acc;
}

}  // namespace

hipError_t dense_gemm_naive(const float* a, const float* b, float* c, int m, int n, int k,
                            hipStream_t stream) {
  if (m < 0 || n < 0 || k < 0) return hipErrorInvalidValue;
  if (m == 0 || n == 0) return hipSuccess;
  if (c == nullptr || (k != 0 && (a == nullptr || b == nullptr))) return hipErrorInvalidValue;
  rr_dense_gemm_naive_kernel<<<grid_for(static_cast<std::size_t>(m) * n), kThreads, 0, stream>>>(
      a, b, c, m, n, k);
  return hipGetLastError();
}

hipError_t topk_gate_naive(const float* logits, int32_t* ids, float* weights, int tokens,
                           int experts, hipStream_t stream) {
  if (tokens < 0 || experts < 2) return hipErrorInvalidValue;
  if (tokens == 0) return hipSuccess;
  if (logits == nullptr || ids == nullptr || weights == nullptr) return hipErrorInvalidValue;
  rr_topk_gate_naive_kernel<<<grid_for(tokens), kThreads, 0, stream>>>(logits, ids, weights,
                                                                        tokens, experts);
  return hipGetLastError();
}

hipError_t histogram_naive(const int32_t* ids, int32_t* counts, int route_pairs, int experts,
                           hipStream_t stream) {
  if (route_pairs < 0 || experts <= 0) return hipErrorInvalidValue;
  if (route_pairs == 0) return hipSuccess;
  if (ids == nullptr || counts == nullptr) return hipErrorInvalidValue;
  rr_histogram_naive_kernel<<<grid_for(route_pairs), kThreads, 0, stream>>>(ids, counts,
                                                                             route_pairs, experts);
  return hipGetLastError();
}

hipError_t exclusive_scan_naive(const int32_t* counts, int32_t* offsets, int experts,
                                hipStream_t stream) {
  if (experts <= 0 || counts == nullptr || offsets == nullptr) return hipErrorInvalidValue;
  rr_exclusive_scan_naive_kernel<<<1, 1, 0, stream>>>(counts, offsets, experts);
  return hipGetLastError();
}

hipError_t token_permute_naive(const float* x, const int32_t* ids, const int32_t* offsets,
                               int32_t* cursors, float* x_permuted, int32_t* route_pos,
                               int32_t* sorted_route, int tokens, int top_k, int hidden,
                               int experts, hipStream_t stream) {
  if (tokens < 0 || top_k <= 0 || hidden < 0) return hipErrorInvalidValue;
  if (tokens == 0) return hipSuccess;
  if (tokens > INT_MAX / top_k) return hipErrorInvalidValue;
  if (ids == nullptr || offsets == nullptr || cursors == nullptr || route_pos == nullptr ||
      (hidden != 0 && (x == nullptr || x_permuted == nullptr))) {
    return hipErrorInvalidValue;
  }
  const int routes = tokens * top_k;
  rr_token_permute_naive_kernel<<<routes, 128, 0, stream>>>(x, ids, offsets, cursors, x_permuted,
                                                            route_pos, sorted_route, routes, top_k,
                                                            hidden, experts);
  return hipGetLastError();
}

hipError_t grouped_gemm_naive(const float* x, const float* w, const int32_t* offsets, float* y,
                              int experts, int hidden, int output, int max_expert_tokens,
                              hipStream_t stream) {
  if (experts <= 0 || hidden < 0 || output < 0 || max_expert_tokens < 0) {
    return hipErrorInvalidValue;
  }
  if (max_expert_tokens == 0 || output == 0) return hipSuccess;
  if (offsets == nullptr || y == nullptr || (hidden != 0 && (x == nullptr || w == nullptr))) {
    return hipErrorInvalidValue;
  }
  const dim3 block(16, 16, 1);
  const unsigned grid_x = static_cast<unsigned>((static_cast<std::size_t>(output) + 15) / 16);
  const std::size_t rows_y = (static_cast<std::size_t>(max_expert_tokens) + 15) / 16;
  const dim3 grid(grid_x, static_cast<unsigned>(rows_y < kMaxBlocks ? rows_y : kMaxBlocks),
                  static_cast<unsigned>(experts));
  rr_grouped_gemm_naive_kernel<<<grid, block, 0, stream>>>(x, w, offsets, y, hidden, output);
  return hipGetLastError();
}

hipError_t unpermute_naive(const float* y_permuted, const int32_t* route_pos,
                           const float* route_weights, float* y, int tokens, int top_k,
                           int output, hipStream_t stream) {
  if (tokens < 0 || top_k <= 0 || output < 0) return hipErrorInvalidValue;
  if (tokens == 0 || output == 0) return hipSuccess;
  if (tokens > INT_MAX / top_k || tokens > INT_MAX / output) return hipErrorInvalidValue;
  if (y_permuted == nullptr || route_pos == nullptr || route_weights == nullptr || y == nullptr) {
    return hipErrorInvalidValue;
  }
  const std::size_t elements = static_cast<std::size_t>(tokens) * output;
  const unsigned blocks = static_cast<unsigned>((elements + kThreads - 1) / kThreads);
  rr_unpermute_naive_kernel<<<blocks, kThreads, 0, stream>>>(y_permuted, route_pos, route_weights,
                                                             y, tokens, top_k, output);
  return hipGetLastError();
}

}  // namespace rr::kern

extern "C" {

hipError_t rr_launch_dense_gemm_naive(const float* a, const float* b, float* c, int32_t m,
                                      int32_t n, int32_t k, hipStream_t stream) {
  return rr::kern::dense_gemm_naive(a, b, c, m, n, k, stream);
}
hipError_t rr_launch_topk_gate_naive(const float* logits, int32_t* expert_ids, float* weights,
                                     int32_t tokens, int32_t experts, hipStream_t stream) {
  return rr::kern::topk_gate_naive(logits, expert_ids, weights, tokens, experts, stream);
}
hipError_t rr_launch_histogram_naive(const int32_t* expert_ids, int32_t* counts,
                                     int32_t route_pairs, int32_t experts, hipStream_t stream) {
  return rr::kern::histogram_naive(expert_ids, counts, route_pairs, experts, stream);
}
hipError_t rr_launch_exclusive_scan_naive(const int32_t* counts, int32_t* offsets,
                                          int32_t experts, hipStream_t stream) {
  return rr::kern::exclusive_scan_naive(counts, offsets, experts, stream);
}
hipError_t rr_launch_token_permute_naive(const float* x, const int32_t* expert_ids,
                                         const int32_t* offsets, int32_t* cursors,
                                         float* x_permuted, int32_t* route_pos,
                                         int32_t* sorted_route, int32_t tokens, int32_t top_k,
                                         int32_t hidden, hipStream_t stream) {
  // The raw launcher has no expert count (reference signature); ids are trusted
  // to index offsets, destinations are still range-checked.
  return rr::kern::token_permute_naive(x, expert_ids, offsets, cursors, x_permuted, route_pos,
                                       sorted_route, tokens, top_k, hidden, INT_MAX, stream);
}
hipError_t rr_launch_grouped_gemm_naive(const float* x_permuted, const float* expert_weights,
                                        const int32_t* offsets, float* y_permuted,
                                        int32_t experts, int32_t hidden, int32_t output,
                                        int32_t max_expert_tokens, hipStream_t stream) {
  return rr::kern::grouped_gemm_naive(x_permuted, expert_weights, offsets, y_permuted, experts,
                                      hidden, output, max_expert_tokens, stream);
}
hipError_t rr_launch_unpermute_naive(const float* y_permuted, const int32_t* route_pos,
                                     const float* route_weights, float* y, int32_t tokens,
                                     int32_t top_k, int32_t output, hipStream_t stream) {
  return rr::kern::unpermute_naive(y_permuted, route_pos, route_weights, y, tokens, top_k, output,
                                   stream);
}

}  // extern "C"
