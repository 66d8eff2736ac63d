// Matrix-core peak probe: the fp32 MFMA rate this device sustains, measured
// beside the copy rate so every fp32 GEMM, attention and conv figure has a
// measured ceiling next to the published 157.3 TFLOP/s.
//
// Each wave issues `iters` rounds of four independent v_mfma_f32_32x32x2f32
// (4096 flops each) on register operands only: no memory traffic inside the
// loop, and four accumulator sets so no MFMA waits on the previous one's result.
#include "common.hpp"

typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(512) void k_mfma_peak(int64_t iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  // operands that differ per lane (random-looking data, not zeros: the matrix
  // cores draw less power, and clock higher, on zero operands)
  float a = 1.0f + (float)(lane * 7 + threadIdx.x % 13) * 1e-3f;
  float b = 0.5f - (float)(lane * 3 + blockIdx.x % 11) * 1e-3f;
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int64_t i = 0; i < iters; ++i) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(b, a, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, a, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x2f32(b, b, c3, 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

extern "C" int cv3_mfma_peak_f32(int64_t iters, int64_t workgroups, float* out, double* flops,
                                 cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(iters > 0 && workgroups > 0 && workgroups <= (1 << 20) && out, CV3_EINVAL,
              "bad MFMA probe arguments iters=%lld workgroups=%lld", (long long)iters, (long long)workgroups);
  hipLaunchKernelGGL(k_mfma_peak, dim3((unsigned)workgroups), dim3(512), 0, cv3::stream_of(s), iters, out);
  CV3_LAUNCHED();
  // 8 waves per workgroup, 4 MFMAs of 2 * 32 * 32 * 2 flops per iteration
  if (flops) *flops = (double)workgroups * 8.0 * (double)iters * 4.0 * 4096.0;
  return CV3_OK;
}
