// Dispatch runtime: architecture resolution and kernel selection.
//
// Follows the check order of reference src/runtime/dispatch.cpp:121-225
// (roles -> layout -> dtype -> architecture -> family/id), with gfx950 as the
// only executing architecture. Pure host code; select_kernel touches no device.
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstring>

#include "common.h"

namespace rr {
namespace {

bool has_zero_strides(const rr_tensor_spec& spec) noexcept {
  return spec.strides[0] == 0 && spec.strides[1] == 0 && spec.strides[2] == 0;
}

// reference dispatch.cpp:25-27
bool has_v02_layout(int32_t present, const rr_tensor_spec& spec) noexcept {
  return !present || (spec.layout == RR_LAYOUT_ROW_MAJOR && has_zero_strides(spec));
}

bool is_storage_type(int32_t type) noexcept {
  return type == RR_DTYPE_FP32 || type == RR_DTYPE_FP16 || type == RR_DTYPE_BF16;
}

bool has_roles(const rr_operator_signature& s, bool input, bool weight, bool accumulator,
               bool output) noexcept {
  return (s.has_input != 0) == input && (s.has_weight != 0) == weight &&
         (s.has_accumulator != 0) == accumulator && (s.has_output != 0) == output;
}

bool roles_valid(int32_t kind, const rr_operator_signature& s) noexcept {
  switch (kind) {
    case RR_OP_DENSE_GEMM:
    case RR_OP_GROUPED_GEMM:
    case RR_OP_UNPERMUTE:
      return has_roles(s, true, true, true, true);
    case RR_OP_TOPK_GATE:
      return has_roles(s, true, false, true, true);
    case RR_OP_TOKEN_PERMUTE:
      return has_roles(s, true, false, false, true);
    case RR_OP_HISTOGRAM:
    case RR_OP_EXCLUSIVE_SCAN:
    case RR_OP_HISTOGRAM_EXCLUSIVE_SCAN:
      return has_roles(s, false, false, false, false);
    default:
      return false;
  }
}

// reference dispatch.cpp:39-71: which storage combinations form a valid
// signature for the operator (whether or not a kernel exists for it).
bool dtype_signature_valid(int32_t kind, const rr_operator_signature& s) noexcept {
  switch (kind) {
    case RR_OP_DENSE_GEMM:
    case RR_OP_GROUPED_GEMM: {
      const int32_t in = s.input.dtype;
      return is_storage_type(in) && s.weight.dtype == in && s.accumulator == RR_DTYPE_FP32 &&
             (s.output.dtype == in || s.output.dtype == RR_DTYPE_FP32);
    }
    case RR_OP_TOPK_GATE:
      return s.input.dtype == RR_DTYPE_FP32 && s.accumulator == RR_DTYPE_FP32 &&
             s.output.dtype == RR_DTYPE_FP32;
    case RR_OP_HISTOGRAM:
    case RR_OP_EXCLUSIVE_SCAN:
    case RR_OP_HISTOGRAM_EXCLUSIVE_SCAN:
      return true;
    case RR_OP_TOKEN_PERMUTE:
      return is_storage_type(s.input.dtype) && s.output.dtype == s.input.dtype;
    case RR_OP_UNPERMUTE: {
      const int32_t in = s.input.dtype;
      return is_storage_type(in) && s.weight.dtype == RR_DTYPE_FP32 &&
             s.accumulator == RR_DTYPE_FP32 &&
             (s.output.dtype == in || s.output.dtype == RR_DTYPE_FP32);
    }
    default:
      return false;
  }
}

// reference dispatch.cpp:73-78
bool all_fp32(const rr_operator_signature& s) noexcept {
  return (!s.has_input || s.input.dtype == RR_DTYPE_FP32) &&
         (!s.has_weight || s.weight.dtype == RR_DTYPE_FP32) &&
         (!s.has_accumulator || s.accumulator == RR_DTYPE_FP32) &&
         (!s.has_output || s.output.dtype == RR_DTYPE_FP32);
}

// Optimized implementation ids accepted per operator. 950 names the native
// gfx950 kernel everywhere; the reference's public optimized ids are accepted
// as aliases of it so that callers passing them keep working (reference ids:
// dense 1-7, top-k 1-4, histogram 101, fused histogram-scan 2, permute 1-10;
// exclusive_scan, grouped_gemm and unpermute expose none).
bool optimized_id_accepted(int32_t kind, uint32_t id) noexcept {
  if (id == RR_IMPL_GFX950_NATIVE) return true;
  switch (kind) {
    case RR_OP_DENSE_GEMM:
      return id >= 1 && id <= 7;
    case RR_OP_TOPK_GATE:
      return id >= 1 && id <= 4;
    case RR_OP_HISTOGRAM:
      return id == 101;
    case RR_OP_HISTOGRAM_EXCLUSIVE_SCAN:
      return id == 2;
    case RR_OP_TOKEN_PERMUTE:
      return id >= 1 && id <= 10;
    default:
      return false;
  }
}

constexpr int kMaxCachedDevices = 64;
// Per-device architecture cache holding architecture + 1 (0 = not yet queried).
// With the per-device CU-count cache in gemm.hip this is the only mutable
// static state of the library; both are idempotent, so races are benign.
std::atomic<int32_t> g_arch_cache[kMaxCachedDevices] = {};

}  // namespace

rr_status dispatch_operator(int32_t operator_kind, const rr_operator_signature& signature,
                            rr_kernel_selection requested, int32_t architecture,
                            rr_dispatch_decision* decision) noexcept {
  int32_t resolved = RR_ARCH_OTHER;
  rr_status status = rr_resolve_device_architecture(architecture, &resolved);
  if (status.code != RR_STATUS_SUCCESS) return status;
  rr_dispatch_request request{};
  request.operator_kind = operator_kind;
  request.architecture = resolved;
  request.requested_kernel = requested;
  request.signature = signature;
  return rr_select_kernel(&request, decision);
}

}  // namespace rr

extern "C" {

int32_t rr_capi_version(void) { return RR_CAPI_VERSION; }

int32_t rr_classify_compute_capability(int32_t major, int32_t minor) {
  if (major == 8 && minor == 6) return RR_ARCH_SM86;
  if (major == 9 && minor == 0) return RR_ARCH_SM90;
  return RR_ARCH_OTHER;
}

int32_t rr_classify_gcn_arch_name(const char* name) {
  if (name == nullptr) return RR_ARCH_OTHER;
  // gcnArchName looks like "gfx950:sramecc+:xnack-".
  if (std::strncmp(name, "gfx950", 6) == 0 && (name[6] == '\0' || name[6] == ':')) {
    return RR_ARCH_GFX950;
  }
  return RR_ARCH_OTHER;
}

rr_status rr_query_current_device_architecture(int32_t* architecture) {
  if (architecture == nullptr) {
    return rr::invalid_argument("no architecture output pointer was given");
  }
  int device = 0;
  hipError_t error = hipGetDevice(&device);
  if (error != hipSuccess) {
    return rr::device_status(error, "resolving the architecture: hipGetDevice failed");
  }
  if (device >= 0 && device < rr::kMaxCachedDevices) {
    const int32_t cached = rr::g_arch_cache[device].load(std::memory_order_acquire);
    if (cached > 0) {
      *architecture = cached - 1;
      return rr::ok_status();
    }
  }
  hipDeviceProp_t properties{};
  error = hipGetDeviceProperties(&properties, device);
  if (error != hipSuccess) {
    return rr::device_status(error, "resolving the architecture: hipGetDeviceProperties failed");
  }
  const int32_t arch = rr_classify_gcn_arch_name(properties.gcnArchName);
  if (device >= 0 && device < rr::kMaxCachedDevices) {
    rr::g_arch_cache[device].store(arch + 1, std::memory_order_release);
  }
  *architecture = arch;
  return rr::ok_status();
}

rr_status rr_resolve_device_architecture(int32_t requested, int32_t* resolved) {
  if (resolved == nullptr) {
    return rr::invalid_argument("no resolved-architecture output pointer was given");
  }
  if (requested == RR_ARCH_AUTO) return rr_query_current_device_architecture(resolved);
  *resolved = requested;
  return rr::ok_status();
}

rr_status rr_select_kernel(const rr_dispatch_request* request, rr_dispatch_decision* decision) {
  if (decision == nullptr) return rr::invalid_argument("select_kernel: no decision output pointer was given");
  if (request == nullptr) return rr::invalid_argument("select_kernel: no request was given");
  const int32_t kind = request->operator_kind;
  if (kind < RR_OP_DENSE_GEMM || kind > RR_OP_HISTOGRAM_EXCLUSIVE_SCAN) {
    return rr::invalid_argument("select_kernel: the operator kind is not one of the eight operators");
  }
  const rr_operator_signature& s = request->signature;
  if (!rr::roles_valid(kind, s)) {
    return rr::invalid_argument("select_kernel: the signature's input / weight / accumulator / output roles do not fit the operator");
  }
  if (!rr::has_v02_layout(s.has_input, s.input) || !rr::has_v02_layout(s.has_weight, s.weight) ||
      !rr::has_v02_layout(s.has_output, s.output)) {
    return rr::make_status(RR_STATUS_UNSUPPORTED_LAYOUT,
                           "select_kernel: tensors must be contiguous row-major with zero strides");
  }
  if (!rr::dtype_signature_valid(kind, s) || !rr::all_fp32(s)) {
    return rr::make_status(RR_STATUS_UNSUPPORTED_DATA_TYPE,
                           "select_kernel: only all-FP32 signatures have kernels");
  }
  if (request->architecture == RR_ARCH_AUTO) {
    return rr::invalid_argument("select_kernel: resolve the architecture (kAuto) before selecting");
  }
  if (request->architecture != RR_ARCH_GFX950) {
    return rr::make_status(RR_STATUS_UNSUPPORTED_ARCHITECTURE,
                           "select_kernel: kernels exist for gfx950 (MI355X) only");
  }
  const rr_kernel_selection requested = request->requested_kernel;
  if (requested.family == RR_FAMILY_AUTO && requested.implementation_id != 0) {
    return rr::make_status(RR_STATUS_UNSUPPORTED_KERNEL_VARIANT,
                           "select_kernel: the auto family takes implementation id 0 only");
  }
  if (requested.family == RR_FAMILY_NAIVE && requested.implementation_id != 0) {
    return rr::make_status(RR_STATUS_UNSUPPORTED_KERNEL_VARIANT,
                           "select_kernel: the naive family takes implementation id 0 only");
  }
  decision->operator_kind = kind;
  decision->architecture = RR_ARCH_GFX950;
  if (requested.family == RR_FAMILY_OPTIMIZED) {
    if (!rr::optimized_id_accepted(kind, requested.implementation_id)) {
      return rr::make_status(RR_STATUS_UNSUPPORTED_KERNEL_VARIANT,
                             "select_kernel: no optimized kernel has that implementation id");
    }
    decision->kernel = requested;
    return rr::ok_status();
  }
  if (requested.family == RR_FAMILY_NAIVE) {
    decision->kernel = {RR_FAMILY_NAIVE, 0};
    return rr::ok_status();
  }
  if (requested.family != RR_FAMILY_AUTO) {
    return rr::make_status(RR_STATUS_UNSUPPORTED_KERNEL_VARIANT,
                           "select_kernel: the kernel family is not one of auto / naive / optimized");
  }
  decision->kernel = {RR_FAMILY_OPTIMIZED, RR_IMPL_GFX950_NATIVE};
  return rr::ok_status();
}

}  // extern "C"
