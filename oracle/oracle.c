/*
 * oracle.c - CPU restatement of the reference RaggedRoute CPU oracles.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline); see oracle.h.
 * Compiled with -O2 -ffp-contract=off: every FP32 `acc += a * b` below is a
 * rounded multiply followed by a rounded add, as in the reference's loops.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* reference src/dense_gemm/cpu_reference/reference.cpp:10-35 (alpha = 1, beta = 0) */
int rro_dense_gemm_f64(const double* a, const double* b, double* c, int m, int n, int k) {
  if (m < 0 || n < 0 || k < 0) return RRO_EINVAL;
  for (int row = 0; row < m; ++row) {
    for (int col = 0; col < n; ++col) {
      double sum = 0.0;
      for (int p = 0; p < k; ++p) sum += a[(int64_t)row * k + p] * b[(int64_t)p * n + col];
      c[(int64_t)row * n + col] = sum;
    }
  }
  return RRO_OK;
}

/* reference benchmarks/adapters/chain_adapter.cpp:197-206: FP32 router logits,
 * sequential k for each (token, expert). */
void rro_dense_gemm_f32_seq(const float* a, const float* b, float* c, int m, int n, int k) {
  for (int row = 0; row < m; ++row) {
    for (int col = 0; col < n; ++col) {
      float sum = 0.0F;
      for (int p = 0; p < k; ++p) sum += a[(int64_t)row * k + p] * b[(int64_t)p * n + col];
      c[(int64_t)row * n + col] = sum;
    }
  }
}

/* reference include/raggedroute/benchmark/adapter_utils.h:367-370 and
 * src/topk_gate/cpu_reference/reference.cpp:22-24: value desc, then lower id. */
static int precedes_f32(float value, int id, float incumbent, int incumbent_id) {
  return incumbent_id < 0 || value > incumbent || (value == incumbent && id < incumbent_id);
}

static int precedes_f64(double value, int id, double incumbent, int incumbent_id) {
  return incumbent_id < 0 || value > incumbent || (value == incumbent && id < incumbent_id);
}

/* reference include/raggedroute/benchmark/adapter_utils.h:363-418 (FP32 top-2). */
int rro_top2_f32(const float* logits, int tokens, int experts, int32_t* ids, float* weights) {
  if (tokens < 0 || experts < 2) return RRO_EINVAL;
  for (int t = 0; t < tokens; ++t) {
    float first = -INFINITY, second = -INFINITY;
    int first_id = -1, second_id = -1;
    int saw_non_nan = 0;
    for (int e = 0; e < experts; ++e) {
      const float raw = logits[(int64_t)t * experts + e];
      const int is_nan = isnan(raw);
      const float value = is_nan ? -INFINITY : raw;
      saw_non_nan = saw_non_nan || !is_nan;
      if (precedes_f32(value, e, first, first_id)) {
        second = first;
        second_id = first_id;
        first = value;
        first_id = e;
      } else if (precedes_f32(value, e, second, second_id)) {
        second = value;
        second_id = e;
      }
    }
    float w1 = 0.5F, w2 = 0.5F;
    if (!saw_non_nan) {
      first_id = 0;
      second_id = 1;
    } else if (first != second) {
      if (first == INFINITY || second == -INFINITY) {
        w1 = 1.0F;
        w2 = 0.0F;
      } else {
        const float relative = expf(second - first);
        w1 = 1.0F / (1.0F + relative);
        w2 = relative * w1;
      }
    }
    ids[2 * (int64_t)t] = first_id;
    ids[2 * (int64_t)t + 1] = second_id;
    weights[2 * (int64_t)t] = w1;
    weights[2 * (int64_t)t + 1] = w2;
  }
  return RRO_OK;
}

/* reference src/topk_gate/cpu_reference/reference.cpp:12-72 (double top-2). */
int rro_top2_f64(const double* logits, int tokens, int experts, int32_t* ids, double* weights) {
  if (tokens < 0 || experts < 2) return RRO_EINVAL;
  for (int t = 0; t < tokens; ++t) {
    double first = -INFINITY, second = -INFINITY;
    int first_id = -1, second_id = -1;
    int saw_non_nan = 0;
    for (int e = 0; e < experts; ++e) {
      const double raw = logits[(int64_t)t * experts + e];
      const int is_nan = isnan(raw);
      const double value = is_nan ? -INFINITY : raw;
      saw_non_nan = saw_non_nan || !is_nan;
      if (precedes_f64(value, e, first, first_id)) {
        second = first;
        second_id = first_id;
        first = value;
        first_id = e;
      } else if (precedes_f64(value, e, second, second_id)) {
        second = value;
        second_id = e;
      }
    }
    double w1 = 0.5, w2 = 0.5;
    if (!saw_non_nan) {
      first_id = 0;
      second_id = 1;
    } else if (first != second) {
      if (first == INFINITY || second == -INFINITY) {
        w1 = 1.0;
        w2 = 0.0;
      } else {
        const double relative = exp(second - first);
        w1 = 1.0 / (1.0 + relative);
        w2 = relative * w1;
      }
    }
    ids[2 * (int64_t)t] = first_id;
    ids[2 * (int64_t)t + 1] = second_id;
    weights[2 * (int64_t)t] = w1;
    weights[2 * (int64_t)t + 1] = w2;
  }
  return RRO_OK;
}

/* reference src/histogram/cpu_reference/reference.cpp:11-22: ids out of range
 * and count overflow are errors (the device kernels ignore out-of-range ids). */
int rro_histogram(const int32_t* ids, int64_t routes, int experts, int32_t* counts) {
  if (experts < 1) return RRO_EINVAL;
  memset(counts, 0, sizeof(int32_t) * (size_t)experts);
  for (int64_t r = 0; r < routes; ++r) {
    const int32_t id = ids[r];
    if (id < 0 || id >= experts) return RRO_EINVAL;
    if (counts[id] == INT32_MAX) return RRO_EOVERFLOW;
    ++counts[id];
  }
  return RRO_OK;
}

/* reference src/scan/cpu_reference/reference.cpp:9-20: offsets[0] = 0,
 * offsets[e + 1] = offsets[e] + counts[e]; negative counts and int32 overflow
 * are errors. */
int rro_exclusive_scan(const int32_t* counts, int experts, int32_t* offsets) {
  if (experts < 0) return RRO_EINVAL;
  int64_t total = 0;
  for (int e = 0; e < experts; ++e) {
    if (counts[e] < 0) return RRO_EINVAL;
    offsets[e] = (int32_t)total;
    total += counts[e];
    if (total > INT32_MAX) return RRO_EOVERFLOW;
  }
  offsets[experts] = (int32_t)total;
  return RRO_OK;
}

/* reference benchmarks/adapters/unpermute_adapter.cpp:47-53: stable map,
 * route_pos[r] = offsets[e] + #{r' < r : ids[r'] == e}. */
int rro_stable_route_pos(const int32_t* ids, int64_t routes, const int32_t* offsets, int experts,
                         int32_t* route_pos) {
  if (experts < 1) return RRO_EINVAL;
  int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)experts);
  if (cursor == NULL) return RRO_EINVAL;
  memcpy(cursor, offsets, sizeof(int32_t) * (size_t)experts);
  for (int64_t r = 0; r < routes; ++r) {
    const int32_t e = ids[r];
    if (e < 0 || e >= experts) {
      free(cursor);
      return RRO_EINVAL;
    }
    route_pos[r] = cursor[e]++;
  }
  free(cursor);
  return RRO_OK;
}

/* Inverse map sorted_route[route_pos[r]] = r (reference operators.h:78-79). */
int rro_inverse_route(const int32_t* route_pos, int64_t routes, int32_t* sorted_route) {
  for (int64_t r = 0; r < routes; ++r) {
    const int32_t p = route_pos[r];
    if (p < 0 || p >= routes) return RRO_EINVAL;
    sorted_route[p] = (int32_t)r;
  }
  return RRO_OK;
}

/* x_permuted[route_pos[r], :] = x[r / top_k, :] (reference
 * src/permute/cpu_reference/reference.cpp:65-71 checks exactly this copy). */
void rro_permute_rows(const float* x, const int32_t* route_pos, int tokens, int top_k, int hidden,
                      float* x_permuted) {
  const int64_t routes = (int64_t)tokens * top_k;
  for (int64_t r = 0; r < routes; ++r) {
    const int64_t t = r / top_k;
    memcpy(x_permuted + (int64_t)route_pos[r] * hidden, x + t * hidden, sizeof(float) * (size_t)hidden);
  }
}

/* reference src/permute/cpu_reference/reference.cpp:22-81: returns a bitmask of
 * the failed invariants (0 = valid). Row copies compare bitwise as floats
 * (NaN == NaN). */
int rro_validate_permute(const float* x, const int32_t* ids, const int32_t* offsets, int experts,
                         const float* x_permuted, const int32_t* route_pos,
                         const int32_t* sorted_route, int tokens, int top_k, int hidden) {
  if (tokens < 0 || top_k < 1 || hidden < 0 || experts < 1) return RRO_PERM_ID_RANGE;
  const int64_t routes = (int64_t)tokens * top_k;
  int failures = 0;
  unsigned char* seen = (unsigned char*)calloc((size_t)(routes > 0 ? routes : 1), 1);
  if (seen == NULL) return RRO_PERM_BIJECTION;
  for (int64_t r = 0; r < routes; ++r) {
    const int e = ids[r];
    if (e < 0 || e >= experts) {
      failures |= RRO_PERM_ID_RANGE;
      continue;
    }
    const int p = route_pos[r];
    if (p < 0 || p >= routes) {
      failures |= RRO_PERM_POSITION_RANGE;
      continue;
    }
    if (p < offsets[e] || p >= offsets[e + 1]) failures |= RRO_PERM_EXPERT_SEGMENT;
    if (seen[p]) failures |= RRO_PERM_BIJECTION;
    seen[p] = 1;
    if (sorted_route != NULL && sorted_route[p] != (int32_t)r) failures |= RRO_PERM_INVERSE;
    const int64_t t = r / top_k;
    for (int c = 0; c < hidden; ++c) {
      const float actual = x_permuted[(int64_t)p * hidden + c];
      const float expected = x[t * hidden + c];
      if (actual != expected && !(isnan(actual) && isnan(expected))) {
        failures |= RRO_PERM_ROW_COPY;
        break;
      }
    }
  }
  for (int64_t p = 0; p < routes; ++p) {
    if (!seen[p]) {
      failures |= RRO_PERM_BIJECTION;
      break;
    }
  }
  if (offsets[0] != 0 || offsets[experts] != (int32_t)routes) failures |= RRO_PERM_OFFSETS;
  free(seen);
  return failures;
}

/* reference src/grouped_gemm/cpu_reference/reference.cpp:10-44 (double). */
int rro_grouped_gemm_f64(const double* x, const double* w, const int32_t* offsets, int experts,
                         int hidden, int output, double* y) {
  if (experts < 1 || hidden < 0 || output < 0) return RRO_EINVAL;
  for (int e = 0; e < experts; ++e) {
    if (offsets[e] < 0 || offsets[e] > offsets[e + 1]) return RRO_EINVAL;
  }
  const int64_t rows = offsets[experts];
  memset(y, 0, sizeof(double) * (size_t)(rows * output));
  for (int e = 0; e < experts; ++e) {
    const double* we = w + (int64_t)e * hidden * output;
    for (int64_t row = offsets[e]; row < offsets[e + 1]; ++row) {
      for (int col = 0; col < output; ++col) {
        double sum = 0.0;
        for (int p = 0; p < hidden; ++p) sum += x[row * hidden + p] * we[(int64_t)p * output + col];
        y[row * output + col] = sum;
      }
    }
  }
  return RRO_OK;
}

/* FP32 grouped GEMM with sequential k (loop order of reference
 * src/grouped_gemm/cuda_naive/baseline.cu:22-29). */
int rro_grouped_gemm_f32_seq(const float* x, const float* w, const int32_t* offsets, int experts,
                             int hidden, int output, float* y) {
  if (experts < 1 || hidden < 0 || output < 0) return RRO_EINVAL;
  for (int e = 0; e < experts; ++e) {
    if (offsets[e] < 0 || offsets[e] > offsets[e + 1]) return RRO_EINVAL;
    const float* we = w + (int64_t)e * hidden * output;
    for (int64_t row = offsets[e]; row < offsets[e + 1]; ++row) {
      for (int col = 0; col < output; ++col) {
        float sum = 0.0F;
        for (int p = 0; p < hidden; ++p) sum += x[row * hidden + p] * we[(int64_t)p * output + col];
        y[row * output + col] = sum;
      }
    }
  }
  return RRO_OK;
}

/* reference src/unpermute/cpu_reference/reference.cpp:10-36 (double). */
int rro_unpermute_f64(const double* y_permuted, const int32_t* route_pos,
                      const double* route_weights, int tokens, int top_k, int output, double* y) {
  if (tokens < 0 || top_k < 1 || output < 0) return RRO_EINVAL;
  const int64_t routes = (int64_t)tokens * top_k;
  for (int t = 0; t < tokens; ++t) {
    for (int c = 0; c < output; ++c) {
      double sum = 0.0;
      for (int j = 0; j < top_k; ++j) {
        const int64_t route = (int64_t)t * top_k + j;
        const int32_t src = route_pos[route];
        if (src < 0 || src >= routes) return RRO_EINVAL;
        sum += route_weights[route] * y_permuted[(int64_t)src * output + c];
      }
      y[(int64_t)t * output + c] = sum;
    }
  }
  return RRO_OK;
}

/* reference benchmarks/adapters/unpermute_adapter.cpp:63-73 (FP32, rank order). */
int rro_unpermute_f32(const float* y_permuted, const int32_t* route_pos, const float* route_weights,
                      int tokens, int top_k, int output, float* y) {
  if (tokens < 0 || top_k < 1 || output < 0) return RRO_EINVAL;
  const int64_t routes = (int64_t)tokens * top_k;
  for (int t = 0; t < tokens; ++t) {
    for (int c = 0; c < output; ++c) {
      float sum = 0.0F;
      for (int j = 0; j < top_k; ++j) {
        const int64_t route = (int64_t)t * top_k + j;
        const int32_t src = route_pos[route];
        if (src < 0 || src >= routes) return RRO_EINVAL;
        sum += route_weights[route] * y_permuted[(int64_t)src * output + c];
      }
      y[(int64_t)t * output + c] = sum;
    }
  }
  return RRO_OK;
}

/* reference benchmarks/adapters/chain_adapter.cpp:858-879: direct per-token
 * expert projection (sequential k) and weighted top-2 combine in FP32. */
/* Combined expert output of top_k routes per token, FP32 in the reference's
 * loop order: per token and column, combined = 0; for each rank in order,
 * projection = sequential FP32 dot of x[t] with column c of W[id]; combined +=
 * weight * projection (reference benchmarks/adapters/chain_adapter.cpp:858-879
 * for top-2, benchmarks/adapters/postroute_chain_adapter.cpp:655-676 for any
 * top_k). */
void rro_route_chain_output_f32(const float* x, const float* expert_weights, const int32_t* ids,
                                const float* route_weights, int tokens, int top_k, int hidden,
                                int output, float* y) {
  for (int t = 0; t < tokens; ++t) {
    for (int c = 0; c < output; ++c) {
      float combined = 0.0F;
      for (int rank = 0; rank < top_k; ++rank) {
        const int64_t route = (int64_t)t * top_k + rank;
        const int64_t e = ids[route];
        float projection = 0.0F;
        for (int p = 0; p < hidden; ++p) {
          projection += x[(int64_t)t * hidden + p] * expert_weights[(e * hidden + p) * output + c];
        }
        combined += route_weights[route] * projection;
      }
      y[(int64_t)t * output + c] = combined;
    }
  }
}

void rro_chain_output_f32(const float* x, const float* expert_weights, const int32_t* ids,
                          const float* route_weights, int tokens, int hidden, int output,
                          float* y) {
  rro_route_chain_output_f32(x, expert_weights, ids, route_weights, tokens, 2, hidden, output, y);
}

/* The reference chain oracle in order (reference chain_adapter.cpp:188-239):
 * FP32 router logits (when from_tokens) -> FP32 top-2 -> counts -> offsets ->
 * stable route map -> FP32 combined output. */
int rro_chain(const float* x, const float* router_weights, float* logits, int from_tokens,
              const float* expert_weights, int tokens, int experts, int hidden, int output,
              int32_t* ids, float* route_weights, int32_t* counts, int32_t* offsets,
              int32_t* route_pos, float* y) {
  if (from_tokens) rro_dense_gemm_f32_seq(x, router_weights, logits, tokens, experts, hidden);
  int rc = rro_top2_f32(logits, tokens, experts, ids, route_weights);
  if (rc != RRO_OK) return rc;
  rc = rro_histogram(ids, (int64_t)tokens * 2, experts, counts);
  if (rc != RRO_OK) return rc;
  rc = rro_exclusive_scan(counts, experts, offsets);
  if (rc != RRO_OK) return rc;
  rc = rro_stable_route_pos(ids, (int64_t)tokens * 2, offsets, experts, route_pos);
  if (rc != RRO_OK) return rc;
  rro_chain_output_f32(x, expert_weights, ids, route_weights, tokens, hidden, output, y);
  return RRO_OK;
}

/* reference src/correctness/reference_validation.cpp:20-26 */
static int same_class(double actual, double expected) {
  if (isnan(expected)) return isnan(actual);
  if (isinf(expected)) return isinf(actual) && (signbit(actual) == signbit(expected));
  return isfinite(actual);
}

/* reference src/correctness/reference_validation.cpp:32-68: element fails when
 * its class differs or |a - e| > atol + rtol * max(|e|, 1e-30). Returns the
 * number of failing elements. */
int64_t rro_compare_floating(const double* actual, const double* expected, int64_t n, double atol,
                             double rtol, double* max_abs, double* max_rel) {
  int64_t failures = 0;
  double worst_abs = 0.0, worst_rel = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    if (!same_class(actual[i], expected[i])) {
      ++failures;
      continue;
    }
    if (!isfinite(expected[i])) continue;
    const double absolute = fabs(actual[i] - expected[i]);
    const double denominator = fmax(fabs(expected[i]), 1.0e-30);
    if (absolute > worst_abs) worst_abs = absolute;
    if (absolute / denominator > worst_rel) worst_rel = absolute / denominator;
    if (absolute > atol + rtol * denominator) ++failures;
  }
  if (max_abs) *max_abs = worst_abs;
  if (max_rel) *max_rel = worst_rel;
  return failures;
}

/* reference src/correctness/reference_validation.cpp:70-115 with FP32
 * accumulation (u = 2^-24) and FP32 output: element (i, j) fails when
 * |a - e| > 4 * gamma_K * sum_p |A[i,p] * B[p,j]| + 1e-7, gamma_K = K u / (1 - K u).
 * worst_ratio receives max |a - e| / bound. */
int64_t rro_compare_gemm(const double* actual, const double* expected, const double* a,
                         const double* b, int m, int n, int k, double* max_abs,
                         double* worst_ratio) {
  const double u = ldexp(1.0, -24);
  const double ku = (double)k * u;
  const double gamma = ku < 1.0 ? ku / (1.0 - ku) : INFINITY;
  int64_t failures = 0;
  double worst_abs = 0.0, ratio = 0.0;
  for (int row = 0; row < m; ++row) {
    for (int col = 0; col < n; ++col) {
      const int64_t idx = (int64_t)row * n + col;
      if (!same_class(actual[idx], expected[idx])) {
        ++failures;
        continue;
      }
      if (!isfinite(expected[idx])) continue;
      double sum_abs = 0.0;
      for (int p = 0; p < k; ++p) sum_abs += fabs(a[(int64_t)row * k + p] * b[(int64_t)p * n + col]);
      const double allowed = 4.0 * gamma * sum_abs + 1.0e-7;
      const double absolute = fabs(actual[idx] - expected[idx]);
      if (absolute > worst_abs) worst_abs = absolute;
      if (absolute / allowed > ratio) ratio = absolute / allowed;
      if (absolute > allowed) ++failures;
    }
  }
  if (max_abs) *max_abs = worst_abs;
  if (worst_ratio) *worst_ratio = ratio;
  return failures;
}
