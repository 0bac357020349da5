/*
 * oracle.h - CPU restatement of the reference RaggedRoute CPU oracles.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker: it may be
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, and nothing in the product (raggedroute_amd/, include/) links, loads or
 * calls it. Build: `make -C oracle` (gcc -O2 -ffp-contract=off, single thread).
 *
 * Every function restates the reference file:line named on it. Integer results
 * are exact; FP32 functions use the reference's loop order with separately
 * rounded multiply and add (no contraction), FP64 functions are the reference's
 * double-precision oracles.
 *
 * Return codes: 0 = ok, negative = the reference oracle would throw
 * (RRO_EINVAL: invalid shape / id out of range; RRO_EOVERFLOW: int32 overflow).
 */
#ifndef RAGGEDROUTE_ORACLE_H
#define RAGGEDROUTE_ORACLE_H

#include <stdint.h>

#define RRO_OK 0
#define RRO_EINVAL (-1)
#define RRO_EOVERFLOW (-2)

/* failure bits of rro_validate_permute (reference permute reference.cpp:43-79) */
#define RRO_PERM_ID_RANGE 1
#define RRO_PERM_POSITION_RANGE 2
#define RRO_PERM_EXPERT_SEGMENT 4
#define RRO_PERM_BIJECTION 8
#define RRO_PERM_INVERSE 16
#define RRO_PERM_ROW_COPY 32
#define RRO_PERM_OFFSETS 64

#ifdef __cplusplus
extern "C" {
#endif

int rro_dense_gemm_f64(const double* a, const double* b, double* c, int m, int n, int k);
void rro_dense_gemm_f32_seq(const float* a, const float* b, float* c, int m, int n, int k);
int rro_top2_f32(const float* logits, int tokens, int experts, int32_t* ids, float* weights);
int rro_top2_f64(const double* logits, int tokens, int experts, int32_t* ids, double* weights);
int rro_histogram(const int32_t* ids, int64_t routes, int experts, int32_t* counts);
int rro_exclusive_scan(const int32_t* counts, int experts, int32_t* offsets);
int rro_stable_route_pos(const int32_t* ids, int64_t routes, const int32_t* offsets, int experts,
                         int32_t* route_pos);
int rro_inverse_route(const int32_t* route_pos, int64_t routes, int32_t* sorted_route);
void rro_permute_rows(const float* x, const int32_t* route_pos, int tokens, int top_k, int hidden,
                      float* x_permuted);
int rro_validate_permute(const float* x, const int32_t* ids, const int32_t* offsets, int experts,
                         const float* x_permuted, const int32_t* route_pos,
                         const int32_t* sorted_route, int tokens, int top_k, int hidden);
int rro_grouped_gemm_f64(const double* x, const double* w, const int32_t* offsets, int experts,
                         int hidden, int output, double* y);
int rro_grouped_gemm_f32_seq(const float* x, const float* w, const int32_t* offsets, int experts,
                             int hidden, int output, float* y);
int rro_unpermute_f64(const double* y_permuted, const int32_t* route_pos,
                      const double* route_weights, int tokens, int top_k, int output, double* y);
int rro_unpermute_f32(const float* y_permuted, const int32_t* route_pos, const float* route_weights,
                      int tokens, int top_k, int output, float* y);
void rro_route_chain_output_f32(const float* x, const float* expert_weights, const int32_t* ids,
                                const float* route_weights, int tokens, int top_k, int hidden,
                                int output, float* y);
void rro_chain_output_f32(const float* x, const float* expert_weights, const int32_t* ids,
                          const float* route_weights, int tokens, int hidden, int output,
                          float* y);
int rro_chain(const float* x, const float* router_weights, float* logits, int from_tokens,
              const float* expert_weights, int tokens, int experts, int hidden, int output,
              int32_t* ids, float* route_weights, int32_t* counts, int32_t* offsets,
              int32_t* route_pos, float* y);
int64_t rro_compare_floating(const double* actual, const double* expected, int64_t n, double atol,
                             double rtol, double* max_abs, double* max_rel);
int64_t rro_compare_gemm(const double* actual, const double* expected, const double* a,
                         const double* b, int m, int n, int k, double* max_abs,
                         double* worst_ratio);

#ifdef __cplusplus
}
#endif

#endif /* RAGGEDROUTE_ORACLE_H */
