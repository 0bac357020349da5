// raggedroute/detail/capi_bridge.h - conversions between the C++ v0.2 types and
// the C ABI structs of raggedroute_capi.h. Header-only; no allocation.
#pragma once

#include "raggedroute/runtime.h"
#include "raggedroute/status.h"
#include "raggedroute/types.h"
#include "raggedroute_capi.h"

namespace raggedroute::detail {

inline rr_tensor_spec to_c(const TensorSpec& spec) noexcept {
  rr_tensor_spec out{};
  out.dtype = static_cast<int32_t>(spec.dtype);
  out.layout = static_cast<int32_t>(spec.layout);
  out.strides[0] = spec.strides[0];
  out.strides[1] = spec.strides[1];
  out.strides[2] = spec.strides[2];
  return out;
}

inline TensorSpec from_c(const rr_tensor_spec& spec) noexcept {
  TensorSpec out;
  out.dtype = static_cast<ScalarType>(spec.dtype);
  out.layout = static_cast<TensorLayout>(spec.layout);
  out.strides = {spec.strides[0], spec.strides[1], spec.strides[2]};
  return out;
}

inline rr_const_tensor_view to_c(const ConstTensorView& view) noexcept {
  return {view.data, to_c(view.spec)};
}

inline rr_mutable_tensor_view to_c(const MutableTensorView& view) noexcept {
  return {view.data, to_c(view.spec)};
}

inline rr_kernel_selection to_c(const KernelSelection& kernel) noexcept {
  return {static_cast<int32_t>(kernel.family), kernel.implementation_id};
}

inline KernelSelection from_c(const rr_kernel_selection& kernel) noexcept {
  return {static_cast<KernelFamily>(kernel.family), kernel.implementation_id};
}

inline rr_runtime_context to_c(const RuntimeContext& context) noexcept {
  return {context.stream, context.workspace, context.workspace_bytes,
          static_cast<int32_t>(context.architecture)};
}

inline Status from_c(const rr_status& status) noexcept {
  return {static_cast<StatusCode>(status.code), static_cast<hipError_t>(status.hip_error),
          status.message};
}

}  // namespace raggedroute::detail
