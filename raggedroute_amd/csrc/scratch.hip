// Allocation-free chain entry: rr_chain_from_tokens with its workspace (the
// permute cursors and the sorted_route scratch) taken from a fixed device
// array instead of the caller's RuntimeContext, for callers that cannot call
// hipMalloc (code under graph capture, tight serving loops, harnesses that
// forbid allocation).
//
// `scratch` exists once per GPU the library runs on and lives until the
// process ends. In host code its name is only a host-side stand-in: the
// device address is resolved with hipGetSymbolAddress, once per device with
// that device current, and only that address is ever handed to a kernel or a
// memset. Every call on one GPU shares that GPU's copy and leaves its
// contents behind; no call relies on them (each writes the cursors and route
// scratch it reads), so nothing needs clearing between calls, but calls that
// overlap on one GPU (concurrent streams, threads) race on it. The address
// lookup of a device's first call is no stream operation: that call may sit
// inside a thread-local stream capture (the graph then replays the chain
// with the resolved address).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>

#include "common.h"

namespace rr {
namespace {

constexpr std::size_t kScratchBytes = RR_CHAIN_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch is a whole number of 256-byte blocks");

__device__ __align__(256) int32_t scratch[kScratchBytes / sizeof(int32_t)];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices] = {};
std::mutex g_scratch_init;

// Device address of `scratch` on the current device, resolved on the first
// call for that device.
rr_status scratch_address(void** out) noexcept {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return device_status(err, "no current HIP device for the chain scratch");
  if (device < 0 || device >= kMaxDevices) {
    return invalid_argument("device index beyond the chain scratch table (64 devices)");
  }
  void* ptr = g_scratch[device].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_init);
    ptr = g_scratch[device].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (err != hipSuccess) return device_status(err, "chain scratch address lookup failed");
      if (ptr == nullptr) {
        return make_status(RR_STATUS_DEVICE_ERROR, "chain scratch address lookup returned null",
                           hipErrorInvalidSymbol);
      }
      g_scratch[device].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return ok_status();
}

}  // namespace
}  // namespace rr

extern "C" rr_status rr_chain_from_tokens_noalloc(const rr_chain_args* args,
                                                  const rr_runtime_context* context) {
  if (args == nullptr) return rr::invalid_argument("rr_chain_from_tokens_noalloc: no argument struct was given");
  if (context == nullptr) return rr::invalid_argument("no runtime context was given");
  // (checked before any device call)
  if (rr_chain_workspace_size(args) > rr::kScratchBytes) {
    return rr::invalid_argument(
        "chain shape exceeds the 1 MiB static scratch of rr_chain_from_tokens_noalloc "
        "(experts + 2 * tokens must be <= 262144)");
  }
  void* ptr = nullptr;
  const rr_status status = rr::scratch_address(&ptr);
  if (status.code != RR_STATUS_SUCCESS) return status;
  rr_runtime_context ctx = *context;
  ctx.workspace = ptr;
  ctx.workspace_bytes = rr::kScratchBytes;
  return rr_chain_from_tokens(args, &ctx);
}
