// Wave64 device helpers for gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rr::dev {

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return static_cast<int>(__lane_id()); }

__device__ __forceinline__ uint64_t lanemask_lt() {
  return (uint64_t{1} << lane_id()) - 1;  // lane 0 -> 0
}

// Mask of the active lanes whose `key` equals this lane's key, for keys in
// [0, 2^bits). `bits` ballots replace a match-any instruction (CDNA has none).
__device__ __forceinline__ uint64_t match_mask(uint32_t key, int bits, uint64_t active) {
  uint64_t mask = active;
  for (int b = 0; b < bits; ++b) {
    const bool bit = (key >> b) & 1u;
    const uint64_t set = __ballot(bit);
    mask &= bit ? set : ~set;
  }
  return mask;
}

__host__ __device__ __forceinline__ int bits_for(int experts) {
  int bits = 0;
  while ((1 << bits) < experts) ++bits;
  return bits;
}

// Inclusive wave scan of int32 values (wraps like the reference's int32 sums).
__device__ __forceinline__ int32_t wave_inclusive_scan(int32_t x) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int32_t y = __shfl_up(x, d, kWave);
    if (lane >= d) x = static_cast<int32_t>(static_cast<uint32_t>(x) + static_cast<uint32_t>(y));
  }
  return x;
}

}  // namespace rr::dev
