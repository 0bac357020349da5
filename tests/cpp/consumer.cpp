// Out-of-tree consumer of the C++ v0.2 surface (role of reference
// tests/packaging/consumer.cpp): compiles against include/raggedroute/*.h,
// links libraggedroute_amd.so and exercises host-only paths (no device).
#include <cstdio>

#include "raggedroute/raggedroute.h"

int main() {
  using namespace raggedroute;
  int failures = 0;
  auto expect = [&](bool condition, const char* what) {
    if (!condition) {
      std::printf("FAIL %s\n", what);
      ++failures;
    }
  };
  expect(classify_compute_capability(8, 6) == DeviceArchitecture::kSm86, "classify 8.6");

  DispatchRequest request;
  request.operator_kind = OperatorKind::kDenseGemm;
  request.architecture = DeviceArchitecture::kGfx950;
  request.signature.input = TensorSpec{};
  request.signature.weight = TensorSpec{};
  request.signature.accumulator = ScalarType::kFp32;
  request.signature.output = TensorSpec{};
  DispatchDecision decision;
  expect(select_kernel(request, &decision).ok(), "gfx950 auto dispatch");
  expect(decision.kernel.family == KernelFamily::kOptimized &&
             decision.kernel.implementation_id == 950,
         "auto selects the native kernel");
  request.architecture = DeviceArchitecture::kSm86;
  expect(select_kernel(request, &decision).code == StatusCode::kUnsupportedArchitecture,
         "SM86 is rejected");

  RuntimeContext context;
  context.architecture = DeviceArchitecture::kGfx950;
  DenseGemmArgs dense;
  dense.m = -1;
  expect(dense_gemm(dense, context).code == StatusCode::kInvalidArgument, "negative M");

  TokenPermuteArgs permute;
  permute.tokens = 1;
  permute.experts = 2;
  permute.top_k = 1;
  std::int32_t placeholder = 0;
  permute.expert_ids = &placeholder;
  permute.offsets = &placeholder;
  permute.route_pos = &placeholder;
  expect(get_token_permute_workspace_size(permute) == 2 * sizeof(std::int32_t), "workspace query");
  expect(token_permute(permute, context).code == StatusCode::kInsufficientWorkspace,
         "missing workspace");

  ChainArgs chain;
  chain.tokens = 4;
  chain.experts = 8;
  chain.top_k = 3;
  expect(chain_from_tokens(chain, context).code == StatusCode::kInvalidArgument, "chain top_k");

  RouteChainArgs route;
  route.tokens = 4;
  route.experts = 8;
  route.top_k = 4;
  route.hidden = 16;
  route.output = 16;
  expect(get_route_chain_workspace_size(route) == (8 + 4 * 4) * sizeof(std::int32_t),
         "route chain workspace query");
  route.top_k = 9;
  expect(chain_from_route_ids(route, context).code == StatusCode::kInvalidArgument,
         "route chain top_k > E");
  expect(ops::launch_dense_gemm_naive(nullptr, nullptr, nullptr, 0, 5, 3, nullptr) == hipSuccess,
         "empty naive dense GEMM is a no-op");

  if (failures == 0) std::printf("consumer OK\n");
  return failures == 0 ? 0 : 1;
}
