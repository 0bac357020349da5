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

// Orders one wave's LDS accesses on either side of it for the compiler. The
// hardware already runs a wave's LDS instructions in issue order, so a lane's
// read after this sees what other lanes of the same wave wrote before it.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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

// DPP lane moves (gfx9 encodings). A lane whose source is out of range, or
// whose row is masked off, receives 0.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ uint32_t dpp_move(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, kRowMask, 0xf, false));
}
constexpr int kDppRowShr1 = 0x111;
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142;  // lane 15 of each row -> the next row
constexpr int kDppRowBcast31 = 0x143;  // lane 31 -> rows 2 and 3

// Inclusive wave scan of int32 values (wraps like the reference's int32 sums):
// shifts of 1, 2, 4, 8 inside rows of 16 lanes, then the row totals are
// carried across rows. Register-to-register moves, no LDS round trips.
__device__ __forceinline__ int32_t wave_inclusive_scan(int32_t v) {
  uint32_t x = static_cast<uint32_t>(v);
  x += dpp_move<kDppRowShr1>(x);
  x += dpp_move<kDppRowShr2>(x);
  x += dpp_move<kDppRowShr4>(x);
  x += dpp_move<kDppRowShr8>(x);
  x += dpp_move<kDppRowBcast15, 0xa>(x);
  x += dpp_move<kDppRowBcast31, 0xc>(x);
  return static_cast<int32_t>(x);
}

}  // namespace rr::dev
