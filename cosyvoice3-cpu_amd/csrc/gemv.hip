// Small-M linear (GEMV): y[m, n] = epi(sum_k x[m, k] * W[n, k]) for m <= 4.
//
// This is the decode hot path (cv3cpu/quant.py:172-204 with m = 1): every byte
// of an int8 weight is streamed from HBM exactly once, with 16-byte loads per
// lane, dequantised in registers (code * scale, exact for fp16 scales) and
// reduced across the 64-lane wavefront.  The activation rows are staged once
// per workgroup in LDS, optionally RMS-normalised on the way in (the Qwen2
// input/post-attention norms, cv3cpu/ops.py:101-104, fused as a prologue).
//
// Weight kinds and the "chunk" a lane loads per step (always 16 bytes):
//   F32 : 4 elements          Q8 : 16 int8 codes (one scale per `block` codes)
//   Q4  : one 32-code block   (byte j: code j low nibble, code j+16 high, +8 bias)
#include "common.hpp"
#include "epilogue.hpp"

using namespace cv3;

namespace {

enum { W_F32 = 0, W_Q8 = 1, W_Q4 = 2 };
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct GemvParams {
  const float* x;
  int64_t ldx;
  int m;
  int64_t k;       // logical reduction length
  int64_t kx;      // staged x length (multiple of the chunk width, zero padded)
  const void* w;
  int64_t ldw;     // bytes between weight rows
  const void* scales;
  int64_t nb;      // scales per row
  int64_t block;   // codes per scale
  int64_t n;       // output columns (for SwiGLU: gate rows [0,n), up rows [n,2n))
  const float* bias;
  float* y;
  int64_t ldy;
  cv3_epilogue epi;
  const float* rms_w;  // optional RMSNorm prologue weight [k]
  float rms_eps;
};

template <int WK>
struct Chunk;
template <>
struct Chunk<W_F32> {
  static constexpr int E = 4;
};
template <>
struct Chunk<W_Q8> {
  static constexpr int E = 16;
};
template <>
struct Chunk<W_Q4> {
  static constexpr int E = 32;
};

__device__ __forceinline__ float i8(uint32_t w, int b) { return (float)((int32_t)(w << (24 - 8 * b)) >> 24); }

// Partial dot product of one 16-byte weight chunk with the staged activations.
template <int WK>
__device__ __forceinline__ float chunk_dot(const u32x4 wv, const float* __restrict__ xs) {
  float acc = 0.f;
  if constexpr (WK == W_F32) {
    const float4 xv = *reinterpret_cast<const float4*>(xs);
    acc = __uint_as_float(wv.x) * xv.x;
    acc = fmaf(__uint_as_float(wv.y), xv.y, acc);
    acc = fmaf(__uint_as_float(wv.z), xv.z, acc);
    acc = fmaf(__uint_as_float(wv.w), xv.w, acc);
  } else if constexpr (WK == W_Q8) {
    const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float4 xv = *reinterpret_cast<const float4*>(xs + 4 * d);
      acc = fmaf(i8(ws[d], 0), xv.x, acc);
      acc = fmaf(i8(ws[d], 1), xv.y, acc);
      acc = fmaf(i8(ws[d], 2), xv.z, acc);
      acc = fmaf(i8(ws[d], 3), xv.w, acc);
    }
  } else {
    const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float4 lo = *reinterpret_cast<const float4*>(xs + 4 * d);
      const float4 hi = *reinterpret_cast<const float4*>(xs + 16 + 4 * d);
      const uint32_t v = ws[d];
      acc = fmaf((float)((v >> 0) & 15u) - 8.f, lo.x, acc);
      acc = fmaf((float)((v >> 8) & 15u) - 8.f, lo.y, acc);
      acc = fmaf((float)((v >> 16) & 15u) - 8.f, lo.z, acc);
      acc = fmaf((float)((v >> 24) & 15u) - 8.f, lo.w, acc);
      acc = fmaf((float)((v >> 4) & 15u) - 8.f, hi.x, acc);
      acc = fmaf((float)((v >> 12) & 15u) - 8.f, hi.y, acc);
      acc = fmaf((float)((v >> 20) & 15u) - 8.f, hi.z, acc);
      acc = fmaf((float)((v >> 28) & 15u) - 8.f, hi.w, acc);
    }
  }
  return acc;
}

template <bool SF16>
__device__ __forceinline__ float scale_at(const void* s, int64_t i) {
  if constexpr (SF16)
    return __half2float(reinterpret_cast<const __half*>(s)[i]);
  else
    return reinterpret_cast<const float*>(s)[i];
}

// Stage x (m rows, zero padded to kx) into LDS, optionally RMS-normalised.
template <int M>
__device__ void stage_x(const GemvParams& p, float* xs, float* red) {
  for (int mi = 0; mi < M; ++mi) {
    const float* xr = p.x + (int64_t)mi * p.ldx;
    float* dst = xs + (int64_t)mi * p.kx;
    if (p.rms_w) {
      float ss = 0.f;
      for (int64_t c = threadIdx.x; c < p.k; c += blockDim.x) {
        const float v = xr[c];
        ss = fmaf(v, v, ss);
      }
      ss = block_sum(ss, red);
      const float inv = 1.0f / sqrtf(ss / (float)p.k + p.rms_eps);
      for (int64_t c = threadIdx.x; c < p.kx; c += blockDim.x)
        dst[c] = c < p.k ? (xr[c] * inv) * p.rms_w[c] : 0.f;
    } else {
      for (int64_t c = threadIdx.x; c < p.kx; c += blockDim.x) dst[c] = c < p.k ? xr[c] : 0.f;
    }
  }
  __syncthreads();
}

// Each wave owns RPW output columns; SWIGLU pairs gate row j with up row j + n.
template <int M, int RPW, int WK, bool SF16, bool SWIGLU>
__global__ __launch_bounds__(256) void k_gemv(GemvParams p) {
  extern __shared__ float xs[];
  __shared__ float red[4];
  stage_x<M>(p, xs, red);

  constexpr int E = Chunk<WK>::E;
  constexpr int NW = SWIGLU ? 2 * RPW : RPW;  // weight rows per wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t col0 = ((int64_t)blockIdx.x * 4 + wave) * RPW;
  if (col0 >= p.n) return;

  int64_t wrow[NW];
  bool live[NW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t c = col0 + r;
    live[r] = c < p.n;
    wrow[r] = live[r] ? c : col0;
    if constexpr (SWIGLU) {
      live[RPW + r] = live[r];
      wrow[RPW + r] = wrow[r] + p.n;
    }
  }

  float acc[NW][M];
#pragma unroll
  for (int r = 0; r < NW; ++r)
#pragma unroll
    for (int mi = 0; mi < M; ++mi) acc[r][mi] = 0.f;

  const int64_t nch = p.kx / E;
  const char* wbase = reinterpret_cast<const char*>(p.w);
  for (int64_t c = lane; c < nch; c += 64) {
    u32x4 wv[NW];
#pragma unroll
    for (int r = 0; r < NW; ++r)
      wv[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wbase + wrow[r] * p.ldw) + c);
#pragma unroll
    for (int r = 0; r < NW; ++r) {
      float sc = 1.f;
      if constexpr (WK != W_F32) sc = scale_at<SF16>(p.scales, wrow[r] * p.nb + (c * E) / p.block);
#pragma unroll
      for (int mi = 0; mi < M; ++mi) {
        const float d = chunk_dot<WK>(wv[r], xs + (int64_t)mi * p.kx + c * E);
        acc[r][mi] = (WK == W_F32) ? acc[r][mi] + d : fmaf(d, sc, acc[r][mi]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NW; ++r)
#pragma unroll
    for (int mi = 0; mi < M; ++mi) acc[r][mi] = wave_sum(acc[r][mi]);

  if (lane < RPW * M) {
    const int r = lane / M, mi = lane % M;
    // select acc[r][mi] with a static loop (registers cannot be indexed dynamically)
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
      for (int mm = 0; mm < M; ++mm)
        if (rr == r && mm == mi) {
          g = acc[rr][mm];
          if constexpr (SWIGLU) u = acc[RPW + rr][mm];
        }
    const int64_t col = col0 + r;
    if (col < p.n) {
      float v;
      if constexpr (SWIGLU) {
        v = (g / (1.0f + expf(-g))) * u;  // silu(g) * u  (cv3cpu/models/qwen2.py:177)
        v = apply_epilogue(p.epi, v, mi, col, true);
      } else {
        v = g + (p.bias ? p.bias[col] : 0.f);
        v = apply_epilogue(p.epi, v, mi, col, false);
      }
      p.y[(int64_t)mi * p.ldy + col] = v;
    }
  }
}

// Scalar fallback for shapes the 16-byte path cannot take (ragged K, unaligned rows).
__global__ __launch_bounds__(256) void k_gemv_scalar(GemvParams p, int wk, int sf16, int swiglu) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 4 + wave;
  if (col >= p.n) return;
  __shared__ float red[4];
  (void)red;
  for (int mi = 0; mi < p.m; ++mi) {
    const float* xr = p.x + (int64_t)mi * p.ldx;
    float inv = 1.f;
    if (p.rms_w) {
      float ss = 0.f;
      for (int64_t c = lane; c < p.k; c += 64) ss = fmaf(xr[c], xr[c], ss);
      ss = wave_sum(ss);
      inv = 1.0f / sqrtf(ss / (float)p.k + p.rms_eps);
    }
    float accs[2] = {0.f, 0.f};
    for (int part = 0; part < (swiglu ? 2 : 1); ++part) {
      const int64_t row = col + part * p.n;
      const char* wr = reinterpret_cast<const char*>(p.w) + row * p.ldw;
      float a = 0.f;
      for (int64_t c = lane; c < p.k; c += 64) {
        float wvv;
        if (wk == W_F32) {
          wvv = reinterpret_cast<const float*>(wr)[c];
        } else {
          float code;
          if (wk == W_Q8) {
            code = (float)reinterpret_cast<const int8_t*>(wr)[c];
          } else {
            const int64_t b = c / p.block, j = c % p.block, h = p.block / 2;
            const uint8_t byte = reinterpret_cast<const uint8_t*>(wr)[b * h + (j % h)];
            code = (float)(j < h ? (byte & 15) : (byte >> 4)) - 8.f;
          }
          const int64_t si = row * p.nb + c / p.block;
          const float sc = sf16 ? __half2float(reinterpret_cast<const __half*>(p.scales)[si])
                                : reinterpret_cast<const float*>(p.scales)[si];
          wvv = code * sc;
        }
        const float xv = p.rms_w ? (xr[c] * inv) * p.rms_w[c] : xr[c];
        a = fmaf(wvv, xv, a);
      }
      accs[part] = wave_sum(a);
    }
    if (lane == 0) {
      float v;
      float* yp = p.y + (int64_t)mi * p.ldy + col;
      if (swiglu) {
        v = (accs[0] / (1.0f + expf(-accs[0]))) * accs[1];
        v = apply_epilogue(p.epi, v, mi, col, true);
      } else {
        v = accs[0] + (p.bias ? p.bias[col] : 0.f);
        v = apply_epilogue(p.epi, v, mi, col, false);
      }
      *yp = v;
    }
  }
}

template <int M, int RPW, int WK, bool SF16, bool SW>
void launch_gemv(const GemvParams& p, hipStream_t st) {
  const int64_t cols_per_block = 4 * RPW;
  const size_t lds = (size_t)M * p.kx * sizeof(float);
  hipLaunchKernelGGL((k_gemv<M, RPW, WK, SF16, SW>), dim3((unsigned)ceil_div(p.n, cols_per_block)), dim3(256), lds,
                     st, p);
}

template <int M, int WK, bool SF16, bool SW>
void pick_rpw(const GemvParams& p, hipStream_t st) {
  // Enough workgroups to cover 256 CUs first; more rows per wave only for wide outputs.
  if (p.n >= 8192)
    launch_gemv<M, 2, WK, SF16, SW>(p, st);
  else
    launch_gemv<M, 1, WK, SF16, SW>(p, st);
}

template <int WK, bool SF16, bool SW>
void dispatch_m(const GemvParams& p, hipStream_t st) {
  switch (p.m) {
    case 1: pick_rpw<1, WK, SF16, SW>(p, st); break;
    case 2: pick_rpw<2, WK, SF16, SW>(p, st); break;
    case 3: pick_rpw<3, WK, SF16, SW>(p, st); break;
    default: pick_rpw<4, WK, SF16, SW>(p, st); break;
  }
}

}  // namespace

namespace cv3 {

// Runs y = epi(x . W^T) for m <= 4 rows (larger m is split by the caller).
int gemv(int wk, bool sf16, bool swiglu, const float* x, int64_t m, int64_t k, int64_t ldx, const void* w,
         int64_t ldw_bytes, const void* scales, int64_t nb, int64_t block, int64_t n, const float* bias, float* y,
         int64_t ldy, const cv3_epilogue* epi, const float* rms_w, float rms_eps, hipStream_t st) {
  CV3_REQUIRE(m >= 1 && m <= 4, CV3_EINVAL, "gemv takes 1..4 rows (got %lld)", (long long)m);
  GemvParams p{};
  p.x = x;
  p.ldx = ldx;
  p.m = (int)m;
  p.k = k;
  p.w = w;
  p.ldw = ldw_bytes;
  p.scales = scales;
  p.nb = nb;
  p.block = block;
  p.n = n;
  p.bias = bias;
  p.y = y;
  p.ldy = ldy;
  p.epi = epi ? *epi : cv3_epilogue{};
  p.rms_w = rms_w;
  p.rms_eps = rms_eps;
  const int E = wk == W_F32 ? 4 : (wk == W_Q8 ? 16 : 32);
  const int64_t kx = ceil_div(k, E) * E;
  p.kx = kx;
  // the 16-byte path needs every chunk of every row readable and 16-byte aligned
  const int64_t row_bytes_needed = wk == W_F32 ? kx * 4 : (wk == W_Q8 ? kx : kx / 2);
  const bool aligned = ((uintptr_t)w % 16 == 0) && (ldw_bytes % 16 == 0) && row_bytes_needed <= ldw_bytes &&
                       (wk == W_F32 || block % E == 0 || (wk == W_Q4 && block == 32));
  const bool fits = (size_t)m * kx * 4 <= 64 * 1024;
  if (aligned && fits && (wk != W_Q4 || block == 32)) {
#define CV3_GEMV_CASE(WKV, SFV, SWV) dispatch_m<WKV, SFV, SWV>(p, st)
    if (wk == W_F32) {
      if (swiglu) CV3_GEMV_CASE(W_F32, false, true); else CV3_GEMV_CASE(W_F32, false, false);
    } else if (wk == W_Q8) {
      if (sf16) {
        if (swiglu) CV3_GEMV_CASE(W_Q8, true, true); else CV3_GEMV_CASE(W_Q8, true, false);
      } else {
        if (swiglu) CV3_GEMV_CASE(W_Q8, false, true); else CV3_GEMV_CASE(W_Q8, false, false);
      }
    } else {
      if (swiglu) CV3_GEMV_CASE(W_Q4, true, true); else CV3_GEMV_CASE(W_Q4, true, false);
    }
#undef CV3_GEMV_CASE
  } else {
    hipLaunchKernelGGL(k_gemv_scalar, dim3((unsigned)ceil_div(n, 4)), dim3(256), 0, st, p, wk, (int)sf16,
                       (int)swiglu);
  }
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // namespace cv3
