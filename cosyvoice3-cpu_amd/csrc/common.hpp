// Shared helpers for the cv3hip kernels: status codes, thread-local error text,
// the calling thread's stream, and wavefront (64-lane) reductions for gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/cv3hip.h"

namespace cv3 {

// Sets the calling thread's error message; returns `code`.
int fail(int code, const char* fmt, ...);
// The stream a call runs on: `s` if non-null, else the calling thread's own
// non-blocking stream (created on first use).
hipStream_t stream_of(cv3_stream_t s);
// True once cv3_shutdown has run: every block is freed and every stream destroyed, so
// no entry point may enqueue work any more.
bool shut_down();

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Block-wide sum for blockDim.x a multiple of 64 and <= 1024.  `red` must hold
// blockDim.x/64 floats of shared memory.  Every thread receives the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = red[0];
  for (int i = 1; i < nw; ++i) t = fmaxf(t, red[i]);
  return t;
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace cv3

#define CV3_HIP(expr)                                                              \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess)                                                          \
      return cv3::fail(CV3_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));  \
  } while (0)

#define CV3_LAUNCHED()                                                             \
  do {                                                                             \
    hipError_t e_ = hipGetLastError();                                             \
    if (e_ != hipSuccess)                                                          \
      return cv3::fail(CV3_EHIP, "kernel launch failed: %s", hipGetErrorString(e_)); \
  } while (0)

#define CV3_REQUIRE(cond, code, ...)                                               \
  do {                                                                             \
    if (!(cond)) return cv3::fail((code), __VA_ARGS__);                            \
  } while (0)

// First statement of every entry point that enqueues device work.
#define CV3_ALIVE() CV3_REQUIRE(!cv3::shut_down(), CV3_EINVAL, "the library has been shut down")
