// Internal helpers shared by the host-side wrappers of libraggedroute_amd.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <limits>

#include "raggedroute_capi.h"

namespace rr {

inline rr_status make_status(int32_t code, const char* message,
                             hipError_t error = hipSuccess) noexcept {
  return {code, static_cast<int32_t>(error), message};
}

inline rr_status ok_status() noexcept { return {RR_STATUS_SUCCESS, 0, "success"}; }

inline rr_status invalid_argument(const char* message) noexcept {
  return make_status(RR_STATUS_INVALID_ARGUMENT, message);
}

inline rr_status device_status(hipError_t error, const char* message) noexcept {
  return error == hipSuccess ? ok_status() : make_status(RR_STATUS_DEVICE_ERROR, message, error);
}

inline bool is_aligned(const void* pointer, std::size_t alignment) noexcept {
  return pointer == nullptr || reinterpret_cast<std::uintptr_t>(pointer) % alignment == 0;
}

inline bool ranges_overlap(const void* left, std::size_t left_bytes, const void* right,
                           std::size_t right_bytes) noexcept {
  if (left_bytes == 0 || right_bytes == 0) return false;
  const auto l = reinterpret_cast<std::uintptr_t>(left);
  const auto r = reinterpret_cast<std::uintptr_t>(right);
  return l < r + right_bytes && r < l + left_bytes;
}

inline rr_tensor_spec default_spec() noexcept {
  rr_tensor_spec s{};
  s.dtype = RR_DTYPE_FP32;
  s.layout = RR_LAYOUT_ROW_MAJOR;
  return s;
}

// Resolves the architecture and runs select_kernel for one operator call.
rr_status dispatch_operator(int32_t operator_kind, const rr_operator_signature& signature,
                            rr_kernel_selection requested, int32_t architecture,
                            rr_dispatch_decision* decision) noexcept;

// True when the decision names the native gfx950 kernel (any accepted
// optimized id); false for the naive family.
inline bool is_native(const rr_dispatch_decision& decision) noexcept {
  return decision.kernel.family == RR_FAMILY_OPTIMIZED;
}

}  // namespace rr
