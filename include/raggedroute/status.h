// raggedroute/status.h - fail-closed status (reference include/raggedroute/status.h:7-29).
// kDeviceError keeps the ordinal of the reference's kCudaError; the error field
// is a hipError_t.
#pragma once

#include <hip/hip_runtime_api.h>

namespace raggedroute {

enum class StatusCode {
  kSuccess = 0,
  kInvalidArgument,
  kUnsupportedArchitecture,
  kUnsupportedDataType,
  kUnsupportedLayout,
  kUnsupportedKernelVariant,
  kInsufficientWorkspace,
  kDeviceError,
};

// Status owns no memory: `message` points at a static string.
struct Status {
  StatusCode code = StatusCode::kSuccess;
  hipError_t hip_error = hipSuccess;
  const char* message = "success";

  constexpr bool ok() const noexcept { return code == StatusCode::kSuccess; }
  constexpr explicit operator bool() const noexcept { return ok(); }
};

constexpr Status success_status() noexcept { return {}; }

}  // namespace raggedroute
