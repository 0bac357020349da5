// Benchmark support kernels: cache scrub and counter-based synthetic inputs.
//
// The scrub rewrites a buffer larger than the 256 MB Infinity Cache so the next
// timed sample starts cold (role of reference src/benchmark/cache_scrub.cu:17-50).
// The fills implement the generator declared in raggedroute_capi.h so that the
// benchmark can build multi-GB inputs in HBM without a host round trip.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "launchers.h"
#include "raggedroute_capi.h"

namespace rr::kern {
namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kStreamMul = 0xD1B54A32D192ED03ull;

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + kGolden;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void rr_cache_scrub_kernel(uint32_t* buffer, std::size_t elements) {
  const std::size_t stride = static_cast<std::size_t>(blockDim.x) * gridDim.x;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < elements; i += stride) {
    buffer[i] = buffer[i] * 1664525u + 1013904223u + static_cast<uint32_t>(i);
  }
}

__global__ void rr_fill_uniform_kernel(float* out, std::size_t count, uint64_t base, float low,
                                       float span) {
  const std::size_t stride = static_cast<std::size_t>(blockDim.x) * gridDim.x;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += stride) {
    const uint64_t z = splitmix64(base + i);
    const float u = static_cast<float>(z >> 40) * 5.9604644775390625e-08F;  // 2^-24
    out[i] = __fadd_rn(low, __fmul_rn(span, u));
  }
}

__global__ void rr_fill_normal_kernel(float* out, std::size_t count, uint64_t base, double mean,
                                      double stddev) {
  const std::size_t stride = static_cast<std::size_t>(blockDim.x) * gridDim.x;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += stride) {
    const uint64_t z = splitmix64(base + i);
    const double u1 = static_cast<double>((z >> 40) + 1) * 5.9604644775390625e-08;  // (0, 1]
    const double u2 = static_cast<double>((z >> 16) & 0xFFFFFFull) * 5.9604644775390625e-08;
    const double n = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    out[i] = static_cast<float>(mean + stddev * n);
  }
}

unsigned grid_for(std::size_t elements) {
  const std::size_t blocks = (elements + 255) / 256;
  return static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
}

uint64_t base_counter(uint64_t seed, uint64_t stream_id) {
  return seed * kGolden + stream_id * kStreamMul;
}

}  // namespace

hipError_t cache_scrub(uint32_t* buffer, std::size_t elements, hipStream_t stream) {
  if (elements == 0) return hipSuccess;
  if (buffer == nullptr) return hipErrorInvalidValue;
  rr_cache_scrub_kernel<<<grid_for(elements), 256, 0, stream>>>(buffer, elements);
  return hipGetLastError();
}

hipError_t fill_uniform(float* out, std::size_t count, uint64_t seed, uint64_t stream_id,
                        float low, float high, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  if (out == nullptr) return hipErrorInvalidValue;
  rr_fill_uniform_kernel<<<grid_for(count), 256, 0, stream>>>(
      out, count, base_counter(seed, stream_id), low, high - low);
  return hipGetLastError();
}

hipError_t fill_normal(float* out, std::size_t count, uint64_t seed, uint64_t stream_id,
                       float mean, float stddev, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  if (out == nullptr) return hipErrorInvalidValue;
  rr_fill_normal_kernel<<<grid_for(count), 256, 0, stream>>>(
      out, count, base_counter(seed, stream_id), mean, stddev);
  return hipGetLastError();
}

}  // namespace rr::kern

extern "C" {

hipError_t rr_launch_cache_scrub(uint32_t* buffer, size_t elements, hipStream_t stream) {
  return rr::kern::cache_scrub(buffer, elements, stream);
}

hipError_t rr_fill_uniform(float* out, size_t count, uint64_t seed, uint64_t stream_id, float low,
                           float high, hipStream_t stream) {
  return rr::kern::fill_uniform(out, count, seed, stream_id, low, high, stream);
}

hipError_t rr_fill_normal(float* out, size_t count, uint64_t seed, uint64_t stream_id, float mean,
                          float stddev, hipStream_t stream) {
  return rr::kern::fill_normal(out, count, seed, stream_id, mean, stddev, stream);
}

const char* rr_build_target(void) { return "gfx950"; }

}  // extern "C"
