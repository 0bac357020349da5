// Top-2 selected-softmax helpers shared by the gate kernel and the router
// GEMM's fused gate epilogue.
//
// Semantics of reference src/topk_gate/cuda_naive/baseline.cu:18-80: order by
// (value desc, expert asc); NaN ranks as -Inf; -0 and +0 tie (lower id wins);
// equal selected values -> {0.5, 0.5}; +Inf first or -Inf second -> {1, 0};
// else r = exp(v2 - v1), w1 = 1 / (1 + r), w2 = r * w1. An all-NaN row
// therefore yields ids {0, 1} with weights {0.5, 0.5} without a special case.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "wave.h"

namespace rr::dev {

// Packed key: larger key = better candidate. High word: order-preserving bits
// of the value (NaN -> -Inf, -0 -> +0); low word: ~expert so ties prefer the
// lower expert id. A zero key is below every real key.
__device__ __forceinline__ uint64_t gate_key(float value, int expert) {
  uint32_t bits = __float_as_uint(isnan(value) ? -INFINITY : value);
  if ((bits << 1) == 0u) bits = 0u;
  const uint32_t ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return (static_cast<uint64_t>(ordered) << 32) |
         static_cast<uint32_t>(~static_cast<uint32_t>(expert));
}

__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t ordered = static_cast<uint32_t>(key >> 32);
  const uint32_t bits = (ordered & 0x80000000u) ? (ordered & 0x7FFFFFFFu) : ~ordered;
  return __uint_as_float(bits);
}

__device__ __forceinline__ int key_expert(uint64_t key) {
  return static_cast<int>(~static_cast<uint32_t>(key));
}

// Selects instead of an if / else that assigns one of two references: the
// compiler turns the latter into a store through a selected address and moves
// the pair to scratch memory.
__device__ __forceinline__ void insert_key(uint64_t key, uint64_t& k1, uint64_t& k2) {
  const bool above1 = key > k1;
  const bool above2 = key > k2;
  const uint64_t second = above1 ? k1 : (above2 ? key : k2);
  k1 = above1 ? key : k1;
  k2 = second;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const int lo = __shfl_xor(static_cast<int>(static_cast<uint32_t>(v)), mask, 64);
  const int hi = __shfl_xor(static_cast<int>(static_cast<uint32_t>(v >> 32)), mask, 64);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// Merge the top-2 pairs of lanes that differ in the bits of LPR / 2 .. 1
// (xor butterfly inside groups of LPR lanes). Keys are distinct except zeros.
template <int LPR>
__device__ __forceinline__ void merge_top2(uint64_t& k1, uint64_t& k2) {
#pragma unroll
  for (int d = LPR / 2; d >= 1; d >>= 1) {
    const uint64_t o1 = shfl_xor_u64(k1, d);
    const uint64_t o2 = shfl_xor_u64(k2, d);
    const uint64_t hi = k1 > o1 ? k1 : o1;
    const uint64_t lo = k1 > o1 ? o1 : k1;
    const uint64_t m2 = k2 > o2 ? k2 : o2;
    k2 = lo > m2 ? lo : m2;
    k1 = hi;
  }
}

// Top-2 merge of a lane's pair with a partner lane's pair (the two pairs hold
// distinct keys, zeros aside).
__device__ __forceinline__ void merge_pair(uint64_t& k1, uint64_t& k2, uint64_t o1, uint64_t o2) {
  const uint64_t hi = k1 > o1 ? k1 : o1;
  const uint64_t lo = k1 > o1 ? o1 : k1;
  const uint64_t m2 = k2 > o2 ? k2 : o2;
  k2 = lo > m2 ? lo : m2;
  k1 = hi;
}

template <int kCtrl>
__device__ __forceinline__ uint64_t dpp_move_u64(uint64_t v) {
  const uint32_t lo = rr::dev::dpp_move<kCtrl>(static_cast<uint32_t>(v));
  const uint32_t hi = rr::dev::dpp_move<kCtrl>(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Top-2 over the 16 lanes of each DPP row (lanes 16r .. 16r + 15) with
// register moves only: partners xor 1 and xor 2 inside quads, then the mirror
// inside each half row (pairs the two quads) and inside the row (pairs the
// two halves). Every pairing joins disjoint lane sets, so every lane ends with
// the top-2 of its row.
__device__ __forceinline__ void merge_top2_row16(uint64_t& k1, uint64_t& k2) {
  constexpr int kQuadXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
  constexpr int kQuadXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
  constexpr int kRowHalfMirror = 0x141;  // lane i <-> 7 - i inside 8
  constexpr int kRowMirror = 0x140;      // lane i <-> 15 - i inside 16
  merge_pair(k1, k2, dpp_move_u64<kQuadXor1>(k1), dpp_move_u64<kQuadXor1>(k2));
  merge_pair(k1, k2, dpp_move_u64<kQuadXor2>(k1), dpp_move_u64<kQuadXor2>(k2));
  merge_pair(k1, k2, dpp_move_u64<kRowHalfMirror>(k1), dpp_move_u64<kRowHalfMirror>(k2));
  merge_pair(k1, k2, dpp_move_u64<kRowMirror>(k1), dpp_move_u64<kRowMirror>(k2));
}

// Selected-softmax weights of the two chosen keys.
__device__ __forceinline__ void gate_weights(uint64_t k1, uint64_t k2, float* w1, float* w2) {
  const float v1 = key_value(k1);
  const float v2 = key_value(k2);
  if (v1 == v2) {
    *w1 = 0.5F;
    *w2 = 0.5F;
  } else if (v1 == INFINITY || v2 == -INFINITY) {
    *w1 = 1.0F;
    *w2 = 0.0F;
  } else {
    const float r = expf(v2 - v1);
    *w1 = 1.0F / (1.0F + r);
    *w2 = __fmul_rn(r, *w1);
  }
}

}  // namespace rr::dev
