// raggedroute/types.h - v0.2 contract vocabulary (reference include/raggedroute/types.h:8-95).
// Enum ordinals are identical to the reference; DeviceArchitecture gains kGfx950
// after the reference values.
#pragma once

#include <array>
#include <cstdint>

namespace raggedroute {

enum class OperatorKind {
  kDenseGemm = 0,
  kTopKGate,
  kHistogram,
  kExclusiveScan,
  kTokenPermute,
  kGroupedGemm,
  kUnpermute,
  kHistogramExclusiveScan,
};

// Only kGfx950 executes in this build; kSm86/kSm90/kOther are classified but
// rejected with kUnsupportedArchitecture.
enum class DeviceArchitecture {
  kAuto = 0,
  kSm86,
  kSm90,
  kOther,
  kGfx950,
};

// Ordinals 0/1/2 as in the reference (kAuto, kCudaNaive, kCudaOptimized).
enum class KernelFamily {
  kAuto = 0,
  kNaive,
  kOptimized,
};

struct KernelSelection {
  KernelFamily family = KernelFamily::kAuto;
  // Zero selects the family default. 950 names the native gfx950 kernel of an
  // operator; the reference's public optimized ids are accepted as aliases.
  std::uint32_t implementation_id = 0;
};

enum class ScalarType {
  kFp32 = 0,
  kFp16,
  kBf16,
  kFp8E4M3,
  kFp8E5M2,
  kFp6E2M3,
  kFp6E3M2,
  kFp4E2M1,
};

enum class TensorLayout {
  kRowMajorContiguous = 0,
  kColumnMajorContiguous,
  kStrided,
};

// All-zero strides mean canonical contiguous strides. v0.2 executes only
// all-zero, row-major-contiguous specs.
struct TensorSpec {
  ScalarType dtype = ScalarType::kFp32;
  TensorLayout layout = TensorLayout::kRowMajorContiguous;
  std::array<std::int64_t, 3> strides = {0, 0, 0};
};

struct ConstTensorView {
  const void* data = nullptr;
  TensorSpec spec{};
};

struct MutableTensorView {
  void* data = nullptr;
  TensorSpec spec{};
};

enum class TopKNormalization {
  kSelectedSoftmax = 0,
};

enum class TopKTieBreak {
  kLowerExpertId = 0,
};

enum class TopKNaNPolicy {
  // NaN is ordered as -Inf. An all-NaN row returns ids {0, 1} and weights {0.5, 0.5}.
  kNegativeInfinityAllNaNFallback01 = 0,
};

}  // namespace raggedroute
