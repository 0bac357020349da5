// raggedroute/dispatch.h - architecture resolution and kernel selection
// (reference include/raggedroute/dispatch.h:12-46). Inline forwarders to the C ABI.
#pragma once

#include <optional>

#include "raggedroute/detail/capi_bridge.h"
#include "raggedroute/status.h"
#include "raggedroute/types.h"

namespace raggedroute {

// Floating operand roles used as the dispatch key; std::nullopt means the role
// is not part of the operator contract (Histogram and Scan have no roles).
struct OperatorSignature {
  std::optional<TensorSpec> input;
  std::optional<TensorSpec> weight;
  std::optional<ScalarType> accumulator;
  std::optional<TensorSpec> output;
};

struct DispatchRequest {
  OperatorKind operator_kind = OperatorKind::kDenseGemm;
  DeviceArchitecture architecture = DeviceArchitecture::kAuto;
  KernelSelection requested_kernel;
  OperatorSignature signature;
};

struct DispatchDecision {
  OperatorKind operator_kind = OperatorKind::kDenseGemm;
  DeviceArchitecture architecture = DeviceArchitecture::kOther;
  KernelSelection kernel;
};

// CUDA compute capabilities still classify (8.6 -> kSm86, 9.0 -> kSm90) but
// never execute here.
inline DeviceArchitecture classify_compute_capability(int major, int minor) noexcept {
  return static_cast<DeviceArchitecture>(rr_classify_compute_capability(major, minor));
}

// Queries the current HIP device once (gcnArchName). Callers that benchmark
// steady-state operators cache the result in RuntimeContext::architecture.
inline Status query_current_device_architecture(DeviceArchitecture* architecture) noexcept {
  int32_t raw = 0;
  const rr_status status = rr_query_current_device_architecture(architecture ? &raw : nullptr);
  if (status.code == RR_STATUS_SUCCESS && architecture) {
    *architecture = static_cast<DeviceArchitecture>(raw);
  }
  return detail::from_c(status);
}

// Resolves kAuto through the current device; explicit values need no query.
inline Status resolve_device_architecture(DeviceArchitecture requested,
                                          DeviceArchitecture* resolved) noexcept {
  int32_t raw = 0;
  const rr_status status =
      rr_resolve_device_architecture(static_cast<int32_t>(requested), resolved ? &raw : nullptr);
  if (status.code == RR_STATUS_SUCCESS && resolved) *resolved = static_cast<DeviceArchitecture>(raw);
  return detail::from_c(status);
}

// Pure dispatch after architecture resolution; check order roles -> layout ->
// dtype -> architecture -> family/id, as in the reference.
inline Status select_kernel(const DispatchRequest& request, DispatchDecision* decision) noexcept {
  rr_dispatch_request c{};
  c.operator_kind = static_cast<int32_t>(request.operator_kind);
  c.architecture = static_cast<int32_t>(request.architecture);
  c.requested_kernel = detail::to_c(request.requested_kernel);
  const OperatorSignature& s = request.signature;
  c.signature.has_input = s.input.has_value();
  if (s.input) c.signature.input = detail::to_c(*s.input);
  c.signature.has_weight = s.weight.has_value();
  if (s.weight) c.signature.weight = detail::to_c(*s.weight);
  c.signature.has_accumulator = s.accumulator.has_value();
  if (s.accumulator) c.signature.accumulator = static_cast<int32_t>(*s.accumulator);
  c.signature.has_output = s.output.has_value();
  if (s.output) c.signature.output = detail::to_c(*s.output);
  rr_dispatch_decision out{};
  const rr_status status = rr_select_kernel(&c, decision ? &out : nullptr);
  if (status.code == RR_STATUS_SUCCESS && decision) {
    decision->operator_kind = static_cast<OperatorKind>(out.operator_kind);
    decision->architecture = static_cast<DeviceArchitecture>(out.architecture);
    decision->kernel = detail::from_c(out.kernel);
  }
  return detail::from_c(status);
}

}  // namespace raggedroute
