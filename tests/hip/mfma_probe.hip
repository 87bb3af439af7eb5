// Test-only probe of v_mfma_i32_16x16x64_i8 operand and result layouts.
// a, b: int8 [64 lanes][16] operand registers; c: int32 [64 lanes][4] result.
// One wave, in-bounds by construction (exactly 64 threads, fixed sizes).
#include <hip/hip_runtime.h>
#include <cstdint>

typedef int i32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(64) void probe(const i32x4* a, const i32x4* b, i32x4* c) {
  const unsigned lane = threadIdx.x;
  i32x4 acc = {0, 0, 0, 0};
  c[lane] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[lane], b[lane], acc, 0, 0, 0);
}

extern "C" int32_t mfma_probe(const void* a, const void* b, void* c) {
  hipLaunchKernelGGL(probe, dim3(1), dim3(64), 0, nullptr, static_cast<const i32x4*>(a),
                     static_cast<const i32x4*>(b), static_cast<i32x4*>(c));
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
