// Block quantisation (q8 / q4), row dequantisation and embedding row gather.
//
// quantize_q8 must be bit-exact with the reference (cv3cpu/quant.py:56-67):
//   amax = max|w| over the block (exact), scale = amax / 127.0f with IEEE
//   division (hipcc keeps fp32 division correctly rounded; no fast-math), 0 -> 1,
//   code = clip(rint(w / scale), -127, 127) with round-half-even, and the stored
//   scale is the fp32 scale converted to fp16 with round-to-nearest-even (or kept
//   fp32 for the per-output-channel layout).
// quantize_q4 follows cv3cpu/quant.py:70-86 (signed extreme / -8, +8 bias, nibble
// packing j | (j + block/2) << 4).
#include "common.hpp"

using namespace cv3;

namespace {

// One wavefront per (row, block).  Lanes stride over the block's elements.
template <bool F16>
__global__ __launch_bounds__(256) void k_quantize_q8(const float* __restrict__ w, int64_t n, int64_t k,
                                                     int64_t kp, int64_t block, int8_t* __restrict__ q,
                                                     void* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int64_t nb = kp / block;
  const int64_t task = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (task >= n * nb) return;
  const int64_t row = task / nb, b = task % nb;
  const float* wr = w + row * k;
  const int64_t c0 = b * block;
  float amax = 0.f;
  for (int64_t j = lane; j < block; j += 64) {
    const int64_t c = c0 + j;
    const float v = c < k ? wr[c] : 0.f;
    amax = fmaxf(amax, fabsf(v));
  }
  amax = wave_max(amax);
  float scale = amax / 127.0f;
  if (scale == 0.f) scale = 1.0f;
  int8_t* qr = q + row * kp;
  for (int64_t j = lane; j < block; j += 64) {
    const int64_t c = c0 + j;
    const float v = c < k ? wr[c] : 0.f;
    float r = rintf(v / scale);
    r = fminf(fmaxf(r, -127.f), 127.f);
    qr[c] = (int8_t)(int)r;
  }
  if (lane == 0) {
    if (F16)
      reinterpret_cast<__half*>(scales)[row * nb + b] = __float2half_rn(scale);
    else
      reinterpret_cast<float*>(scales)[row * nb + b] = scale;
  }
}

// One wavefront per (row, block); block <= 64 (q4 blocks are 32 wide).
__global__ __launch_bounds__(256) void k_quantize_q4(const float* __restrict__ w, int64_t n, int64_t k,
                                                     int64_t kp, int block, uint8_t* __restrict__ q,
                                                     __half* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int64_t nb = kp / block;
  const int64_t task = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (task >= n * nb) return;
  const int64_t row = task / nb, b = task % nb;
  const int64_t c = b * block + lane;
  const float v = (lane < block && c < k) ? w[row * k + c] : 0.f;
  // argmax of |v|, first index on ties
  float best = lane < block ? fabsf(v) : -1.f;
  int idx = lane;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (ob > best || (ob == best && oi < idx)) {
      best = ob;
      idx = oi;
    }
  }
  const float ext = __shfl(v, idx, 64);
  float scale = ext / -8.0f;
  if (scale == 0.f) scale = 1.0f;
  float r = rintf(v / scale + 8.0f);
  r = fminf(fmaxf(r, 0.f), 15.f);
  const uint32_t code = (uint32_t)(int)r;
  const int h = block >> 1;
  const uint32_t hi = __shfl(code, (lane + h) & 63, 64);
  if (lane < h) q[row * (kp >> 1) + b * h + lane] = (uint8_t)(code | (hi << 4));
  if (lane == 0) scales[row * nb + b] = __float2half_rn(scale);
}

__device__ __forceinline__ float load_scale(const void* s, int sf16, int64_t i) {
  return sf16 ? __half2float(reinterpret_cast<const __half*>(s)[i]) : reinterpret_cast<const float*>(s)[i];
}

// out[r - r0, c] for c < k: code * float(scale); q4 codes are nibble-unpacked minus 8.
__global__ void k_dequant_rows(int kind, const void* __restrict__ q, const void* __restrict__ scales, int sf16,
                               int64_t kp, int64_t block, int64_t k, int64_t r0, int64_t rows,
                               const int64_t* __restrict__ ids, float* __restrict__ out, int64_t ldo) {
  const int64_t nb = kp / block;
  for (int64_t i = blockIdx.y; i < rows; i += gridDim.y) {
  const int64_t row = ids ? ids[i] : r0 + i;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < k; c += (int64_t)gridDim.x * blockDim.x) {
    float code;
    if (kind == CV3_KIND_Q8) {
      code = (float)reinterpret_cast<const int8_t*>(q)[row * kp + c];
    } else {
      const int64_t b = c / block, j = c % block, h = block / 2;
      const uint8_t byte = reinterpret_cast<const uint8_t*>(q)[row * (kp / 2) + b * h + (j % h)];
      code = (float)(j < h ? (byte & 0xF) : (byte >> 4)) - 8.0f;
    }
    out[i * ldo + c] = code * load_scale(scales, sf16, row * nb + c / block);
  }
  }
}

template <typename T>
__global__ void k_gather_rows(const T* __restrict__ table, int64_t cols, const int64_t* __restrict__ ids,
                              int64_t n, float* __restrict__ out) {
  for (int64_t i = blockIdx.y; i < n; i += gridDim.y) {
    const T* src = table + ids[i] * cols;
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += (int64_t)gridDim.x * blockDim.x)
      out[i * cols + c] = (float)src[c];
  }
}

__global__ void k_check_ids(const int64_t* __restrict__ ids, int64_t n, int64_t rows, int* __restrict__ bad) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    if (ids[i] < 0 || ids[i] >= rows) atomicOr(bad, 1);
}

}  // namespace

extern "C" {

int cv3_quantize_q8(const float* w, int64_t n, int64_t k, int64_t block, int scale_dtype, int8_t* q,
                    void* scales, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(n >= 0 && k > 0 && block > 0, CV3_EINVAL, "bad quantize_q8 shape n=%lld k=%lld block=%lld",
              (long long)n, (long long)k, (long long)block);
  CV3_REQUIRE(scale_dtype == CV3_F16 || scale_dtype == CV3_F32, CV3_EINVAL, "scale dtype must be f16 or f32");
  if (n == 0) return CV3_OK;
  const int64_t kp = ceil_div(k, block) * block;
  const int64_t tasks = n * (kp / block);
  const dim3 grid((unsigned)ceil_div(tasks, 4)), blk(256);
  if (scale_dtype == CV3_F16)
    hipLaunchKernelGGL(k_quantize_q8<true>, grid, blk, 0, stream_of(s), w, n, k, kp, block, q, scales);
  else
    hipLaunchKernelGGL(k_quantize_q8<false>, grid, blk, 0, stream_of(s), w, n, k, kp, block, q, scales);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_quantize_q4(const float* w, int64_t n, int64_t k, int64_t block, uint8_t* q, void* scales_f16,
                    cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(n >= 0 && k > 0 && block > 0 && block <= 64 && block % 2 == 0, CV3_EINVAL,
              "q4 block must be even and <= 64 (got %lld)", (long long)block);
  if (n == 0) return CV3_OK;
  const int64_t kp = ceil_div(k, block) * block;
  const int64_t tasks = n * (kp / block);
  hipLaunchKernelGGL(k_quantize_q4, dim3((unsigned)ceil_div(tasks, 4)), dim3(256), 0, stream_of(s), w, n, k, kp,
                     (int)block, q, reinterpret_cast<__half*>(scales_f16));
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_dequant_rows(int kind, const void* q, const void* scales, int scale_dtype, int64_t kp, int64_t block,
                     int64_t k, int64_t r0, int64_t r1, float* out, int64_t ld_out, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(kind == CV3_KIND_Q8 || kind == CV3_KIND_Q4, CV3_EINVAL, "unknown quant kind %d", kind);
  CV3_REQUIRE(r1 >= r0 && k <= kp && kp % block == 0, CV3_EINVAL, "bad dequant_rows range/shape");
  const int64_t rows = r1 - r0;
  if (!rows || !k) return CV3_OK;
  const dim3 grid((unsigned)std::min<int64_t>(ceil_div(k, 256), 64), (unsigned)std::min<int64_t>(rows, 65535));
  hipLaunchKernelGGL(k_dequant_rows, grid, dim3(256), 0, stream_of(s), kind, q, scales, scale_dtype == CV3_F16,
                     kp, block, k, r0, rows, (const int64_t*)nullptr, out, ld_out);
  CV3_LAUNCHED();
  return CV3_OK;
}

// Embedding row gather (cv3cpu/ops.py:126-144).  `ids` are device int64; the
// bounds check runs on the device and is reported as CV3_EINDEX.
int cv3_embedding(int kind, const void* table, const void* scales, int scale_dtype, int64_t rows, int64_t cols,
                  int64_t kp, int64_t block, const int64_t* ids, int64_t n, float* out, cv3_stream_t s) {
  CV3_ALIVE();
  if (n == 0) return CV3_OK;
  hipStream_t st = stream_of(s);
  int* bad = nullptr;
  CV3_HIP(hipMallocAsync((void**)&bad, sizeof(int), st));
  CV3_HIP(hipMemsetAsync(bad, 0, sizeof(int), st));
  hipLaunchKernelGGL(k_check_ids, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 64)), dim3(256), 0, st, ids, n,
                     rows, bad);
  int hbad = 0;
  CV3_HIP(hipMemcpyAsync(&hbad, bad, sizeof(int), hipMemcpyDeviceToHost, st));
  CV3_HIP(hipFreeAsync(bad, st));
  CV3_HIP(hipStreamSynchronize(st));
  CV3_REQUIRE(!hbad, CV3_EINDEX, "token id is outside the %lld-row embedding table", (long long)rows);
  const dim3 grid((unsigned)std::min<int64_t>(ceil_div(cols, 256), 16), (unsigned)std::min<int64_t>(n, 65535));
  switch (kind) {
    case CV3_KIND_F32:
      hipLaunchKernelGGL(k_gather_rows<float>, grid, dim3(256), 0, st, (const float*)table, cols, ids, n, out);
      break;
    case CV3_KIND_F16:
      hipLaunchKernelGGL(k_gather_rows<__half>, grid, dim3(256), 0, st, (const __half*)table, cols, ids, n, out);
      break;
    case CV3_KIND_Q8:
    case CV3_KIND_Q4:
      hipLaunchKernelGGL(k_dequant_rows, grid, dim3(256), 0, st, kind, table, scales, scale_dtype == CV3_F16, kp,
                         block, cols, (int64_t)0, n, ids, out, cols);
      break;
    default:
      return fail(CV3_EINVAL, "unknown table kind %d", kind);
  }
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // extern "C"
