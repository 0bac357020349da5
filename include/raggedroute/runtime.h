// raggedroute/runtime.h - per-call resources (reference include/raggedroute/runtime.h:13-18).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>

#include "raggedroute/types.h"

namespace raggedroute {

// Workspace allocation and device discovery belong outside steady-state timing:
// callers cache the resolved architecture here.
struct RuntimeContext {
  hipStream_t stream = nullptr;
  void* workspace = nullptr;
  std::size_t workspace_bytes = 0;
  DeviceArchitecture architecture = DeviceArchitecture::kAuto;
};

}  // namespace raggedroute
