// Elementwise, row-reduction and table kernels around the GEMMs:
// activations (cv3cpu/ops.py:30-81), Snake (ops.py:77-81), row softmax /
// log_softmax (ops.py:84-93), RMSNorm (ops.py:101-104), LayerNorm with optional
// affine or AdaLN modulation (ops.py:107-118, cv3cpu/models/dit.py:168-178),
// rotary tables and rotation (dit.py:21-54, cv3cpu/models/qwen2.py:35-71), the
// CFG combine + Euler update (cv3cpu/models/flow.py:86-87), resampling
// (ops.py:318-336), Hann window (ops.py:339-343) and 2-D transposes.
//
// All of these are HBM-bound: one read and one write per element, fused where a
// caller would otherwise make several passes.
#include "common.hpp"
#include "epilogue.hpp"
#include "decode_common.hpp"   // wave_sum_swap: DPP and permlane wave sums

using namespace cv3;

namespace {

inline unsigned grid_for(int64_t n, int per_block = 256, int64_t cap = 65536) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, per_block), cap));
}

__global__ void k_act(int act, float param, const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = apply_act(act, x[i], param);
}

__global__ void k_binary(int op, const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ y,
                         int64_t n, float alpha, float beta) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float u = a[i], v = b[i];
    float r;
    switch (op) {
      case 0: r = u + v; break;                    // add
      case 1: r = u * v; break;                    // mul
      case 2: r = act_silu(u) * v; break;          // silu(a) * b  (qwen2.py:177)
      case 4: r = (u + v) / alpha; break;          // (a + b) / alpha: the resblock mean (hift.py:165)
      default: r = alpha * u + beta * v; break;    // axpby
    }
    y[i] = r;
  }
}

// Snake over (C, T): x + (1 / (alpha + eps)) * sin(alpha x)^2   (ops.py:77-81)
__global__ void k_snake(const float* __restrict__ x, const float* __restrict__ alpha, float* __restrict__ y,
                        int64_t c, int64_t t, float eps) {
  const int64_t n = c * t;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float a = alpha[i / t];
    const float v = x[i];
    const float s = sinf(a * v);
    y[i] = v + (1.0f / (a + eps)) * (s * s);
  }
}

// Snake on channels-last (t, c) data: the alpha of element i is alpha[i % c].
__global__ void k_snake_cl(const float* __restrict__ x, const float* __restrict__ alpha, float* __restrict__ y,
                           uint32_t n, uint32_t c, float eps) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const float a = alpha[i % c];
    const float v = x[i];
    const float s = sinf(a * v);
    y[i] = v + (1.0f / (a + eps)) * (s * s);
  }
}

// One workgroup per row.  softmax: e = exp(x - max), e / sum;  log: z - log(sum exp z).
__global__ __launch_bounds__(256) void k_softmax_rows(const float* __restrict__ x, float* __restrict__ y, int64_t cols,
                                                      int logmode) {
  __shared__ float red[4];
  const float* xr = x + (int64_t)blockIdx.x * cols;
  float* yr = y + (int64_t)blockIdx.x * cols;
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) m = fmaxf(m, xr[c]);
  m = block_max(m, red);
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) s += expf(xr[c] - m);
  s = block_sum(s, red);
  if (logmode) {
    const float ls = logf(s);
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) yr[c] = (xr[c] - m) - ls;
  } else {
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) yr[c] = expf(xr[c] - m) / s;
  }
}

// RMSNorm: (x * (1/sqrt(mean(x^2) + eps))) * w   (ops.py:101-104)
__global__ __launch_bounds__(256) void k_rms_norm(const float* __restrict__ x, const float* __restrict__ w,
                                                  float* __restrict__ y, int64_t cols, float eps) {
  __shared__ float red[4];
  const float* xr = x + (int64_t)blockIdx.x * cols;
  float* yr = y + (int64_t)blockIdx.x * cols;
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) ss = fmaf(xr[c], xr[c], ss);
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) yr[c] = (xr[c] * inv) * w[c];
}

// LayerNorm, two-pass centred variance (ops.py:107-118), then either an affine
// (w, b) or the AdaLN modulation norm * (1 + scale[g]) + shift[g] with
// g = row / rows_per_group (cv3cpu/models/dit.py:168-169,178).
__global__ __launch_bounds__(256) void k_layer_norm(const float* __restrict__ x, float* __restrict__ y, int64_t cols,
                                                    float eps, const float* __restrict__ w,
                                                    const float* __restrict__ b, const float* __restrict__ shift,
                                                    const float* __restrict__ scale, int64_t mod_stride,
                                                    int64_t rows_per_group) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * cols;
  float* yr = y + row * cols;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) s += xr[c];
  const float mu = block_sum(s, red) / (float)cols;
  float v = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float d = xr[c] - mu;
    v = fmaf(d, d, v);
  }
  const float var = block_sum(v, red) / (float)cols;
  const float den = sqrtf(var + eps);
  const int64_t g = rows_per_group > 0 ? row / rows_per_group : 0;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    float o = (xr[c] - mu) / den;
    if (w) o = o * w[c];
    if (b) o = o + b[c];
    if (scale) o = o * (1.0f + scale[g * mod_stride + c]);
    if (shift) o = o + shift[g * mod_stride + c];
    yr[c] = o;
  }
}

// The same LayerNorm (+ affine / AdaLN) with the row held in registers: each of the
// 256 threads loads NV float4 of the row (and of w / b / shift / scale) up front, so
// a row costs one memory latency instead of one per loop trip.  cols % 4 == 0,
// cols <= 1024 * NV, 16-byte aligned operands.
template <int NV>
__global__ __launch_bounds__(256) void k_layer_norm4(const float* __restrict__ x, float* __restrict__ y, int64_t cols,
                                                     float eps, const float* __restrict__ w,
                                                     const float* __restrict__ b, const float* __restrict__ shift,
                                                     const float* __restrict__ scale, int64_t mod_stride,
                                                     int64_t rows_per_group) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t c4 = cols / 4;
  const float4* xr = reinterpret_cast<const float4*>(x + row * cols);
  const int64_t g = rows_per_group > 0 ? row / rows_per_group : 0;
  const float4* sh = shift ? reinterpret_cast<const float4*>(shift + g * mod_stride) : nullptr;
  const float4* sc = scale ? reinterpret_cast<const float4*>(scale + g * mod_stride) : nullptr;
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 v[NV], wv[NV], bv[NV], shv[NV], scv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t j = threadIdx.x + 256 * i;
    const bool ok = j < c4;
    v[i] = ok ? xr[j] : z;
    wv[i] = (ok && w) ? reinterpret_cast<const float4*>(w)[j] : z;
    bv[i] = (ok && b) ? reinterpret_cast<const float4*>(b)[j] : z;
    shv[i] = (ok && sh) ? sh[j] : z;
    scv[i] = (ok && sc) ? sc[j] : z;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  const float mu = block_sum(s, red) / (float)cols;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t j = threadIdx.x + 256 * i;
    if (j < c4) {
      const float d0 = v[i].x - mu, d1 = v[i].y - mu, d2 = v[i].z - mu, d3 = v[i].w - mu;
      q = fmaf(d0, d0, q);
      q = fmaf(d1, d1, q);
      q = fmaf(d2, d2, q);
      q = fmaf(d3, d3, q);
    }
  }
  const float den = sqrtf(block_sum(q, red) / (float)cols + eps);
  float4* yr = reinterpret_cast<float4*>(y + row * cols);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t j = threadIdx.x + 256 * i;
    if (j < c4) {
      float o[4] = {(v[i].x - mu) / den, (v[i].y - mu) / den, (v[i].z - mu) / den, (v[i].w - mu) / den};
      const float ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
      const float bb[4] = {bv[i].x, bv[i].y, bv[i].z, bv[i].w};
      const float ss[4] = {shv[i].x, shv[i].y, shv[i].z, shv[i].w};
      const float cc[4] = {scv[i].x, scv[i].y, scv[i].z, scv[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (w) o[e] = o[e] * ww[e];
        if (b) o[e] = o[e] + bb[e];
        if (scale) o[e] = o[e] * (1.0f + cc[e]);
        if (shift) o[e] = o[e] + ss[e];
      }
      yr[j] = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
}

// One wave per row for rows of at most 256 * 4 columns: each lane holds NV float4 of the
// row (and of w / b / shift / scale), loaded up front with clamped indices and zeroed
// past the row after the loads; mean and centred variance are wave reductions, so a
// row needs no barrier.  Four rows per 256-thread workgroup.
template <int NV>
__global__ __launch_bounds__(256) void k_layer_norm_wave(const float* __restrict__ x, float* __restrict__ y,
                                                         int64_t rows, int64_t cols, float eps,
                                                         const float* __restrict__ w, const float* __restrict__ b,
                                                         const float* __restrict__ shift,
                                                         const float* __restrict__ scale, int64_t mod_stride,
                                                         int64_t rows_per_group, int* __restrict__ rexp) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t c4 = cols / 4;
  const float4* xr = reinterpret_cast<const float4*>(x + row * cols);
  const int64_t g = rows_per_group > 0 ? row / rows_per_group : 0;
  const float4* sh = reinterpret_cast<const float4*>(shift ? shift + g * mod_stride : x);
  const float4* sc = reinterpret_cast<const float4*>(scale ? scale + g * mod_stride : x);
  const float4* w4 = reinterpret_cast<const float4*>(w ? w : x);
  const float4* b4 = reinterpret_cast<const float4*>(b ? b : x);
  // the optional vectors are loaded only when given (uniform branches): the DiT's AdaLN has
  // shift and scale but no affine weight or bias
  float4 v[NV], wv[NV], bv[NV], shv[NV], scv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t j = min((int64_t)lane + 64 * i, c4 - 1);
    v[i] = xr[j];
    if (w) wv[i] = w4[j];
    if (b) bv[i] = b4[j];
    if (shift) shv[i] = sh[j];
    if (scale) scv[i] = sc[j];
  }
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i >= c4) v[i] = z;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  const float mu = wave_sum_swap(s) / (float)cols;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (lane + 64 * i < c4) {
      const float d0 = v[i].x - mu, d1 = v[i].y - mu, d2 = v[i].z - mu, d3 = v[i].w - mu;
      q = fmaf(d0, d0, q);
      q = fmaf(d1, d1, q);
      q = fmaf(d2, d2, q);
      q = fmaf(d3, d3, q);
    }
  }
  const float den = sqrtf(wave_sum_swap(q) / (float)cols + eps);
  float4* yr = reinterpret_cast<float4*>(y + row * cols);
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t j = lane + 64 * i;
    if (j < c4) {
      float o[4] = {(v[i].x - mu) / den, (v[i].y - mu) / den, (v[i].z - mu) / den, (v[i].w - mu) / den};
      const float ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
      const float bb[4] = {bv[i].x, bv[i].y, bv[i].z, bv[i].w};
      const float ss[4] = {shv[i].x, shv[i].y, shv[i].z, shv[i].w};
      const float cc[4] = {scv[i].x, scv[i].y, scv[i].z, scv[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (w) o[e] = o[e] * ww[e];
        if (b) o[e] = o[e] + bb[e];
        if (scale) o[e] = o[e] * (1.0f + cc[e]);
        if (shift) o[e] = o[e] + ss[e];
      }
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
      yr[j] = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
  // optionally the binary exponent of the row's largest |y| (frexp, at least -96): the scale
  // the digit-plane q8 GEMM rounds this row to, so that GEMM needs no pass of its own
  if (rexp) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    int ex = 0;
    if (mx > 0.f) (void)frexpf(mx, &ex);
    if (lane == 0) rexp[row] = max(ex, -96);
  }
}

// Rotary tables.  kind 0 (DiT, dit.py:21-29,51-52): angle_f32 = f32(t * inv_f64),
// interleaved duplicate, cos/sin in fp32.  kind 1 (Qwen2, qwen2.py:46-56):
// angle in fp64, half-split duplicate, cos/sin in fp64 then rounded to fp32.
__global__ void k_rope_table(int kind, double theta, int dim, int64_t n, int64_t pos0, float* __restrict__ cosv,
                             float* __restrict__ sinv) {
  const int64_t total = n * dim;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / dim + pos0;
    const int c = (int)(i % dim);
    const int fi = kind == 0 ? c / 2 : c % (dim / 2);
    const double inv = 1.0 / pow(theta, (double)(2 * fi) / (double)dim);
    const double ang = (double)t * inv;
    if (kind == 0) {
      const float a = (float)ang;
      cosv[i] = cosf(a);
      sinv[i] = sinf(a);
    } else {
      cosv[i] = (float)cos(ang);
      sinv[i] = (float)sin(ang);
    }
  }
}

// DiT partial rotary on the first `rot` channels of rows of width `ld`
// (before the head split, dit.py:40-54): pairs (2i, 2i+1) -> (x0 c0 - x1 s0, x1 c1 + x0 s1).
// Row r is time step r % rows_per_batch.  Works in place.
__global__ void k_rope_pairs(float* __restrict__ x, int64_t ld, int64_t rows, int64_t rows_per_batch, int rot,
                             const float* __restrict__ cosv, const float* __restrict__ sinv) {
  const int half = rot / 2;
  const int64_t total = rows * half;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / half;
    const int p = (int)(i % half);
    const int64_t t = r % rows_per_batch;
    float* xr = x + r * ld;
    const float x0 = xr[2 * p], x1 = xr[2 * p + 1];
    const float* c = cosv + t * rot;
    const float* s = sinv + t * rot;
    xr[2 * p] = x0 * c[2 * p] + (-x1) * s[2 * p];
    xr[2 * p + 1] = x1 * c[2 * p + 1] + x0 * s[2 * p + 1];
  }
}

// Qwen2 half-split rotary over vectors of length d: x cos + rotate_half(x) sin
// (qwen2.py:64-71).  Vector v lives at x + (v / per_pos) * ld_pos + (v % per_pos) * d
// and uses table row pos0 + v / per_pos.  Works in place.
__global__ void k_rope_half(float* __restrict__ x, int64_t nvec, int64_t per_pos, int64_t ld_pos, int d,
                            const float* __restrict__ cosv, const float* __restrict__ sinv, int64_t pos0) {
  const int half = d / 2;
  const int64_t total = nvec * half;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = i / half;
    const int j = (int)(i % half);
    const int64_t t = v / per_pos;
    float* xv = x + t * ld_pos + (v % per_pos) * d;
    const float a = xv[j], b = xv[j + half];
    const float* c = cosv + (pos0 + t) * d;
    const float* s = sinv + (pos0 + t) * d;
    xv[j] = a * c[j] + (-b) * s[j];
    xv[j + half] = b * c[j + half] + a * s[j + half];
  }
}

// CFG combine + Euler step: x += dt * ((1 + w) d_cond - w d_uncond)   (flow.py:86-87)
__global__ void k_cfg_euler(float* __restrict__ x, const float* __restrict__ dc, const float* __restrict__ du,
                            int64_t n, float dt, float w) {
  const float a = 1.0f + w;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float dphi = a * dc[i] - w * du[i];
    x[i] = x[i] + dt * dphi;
  }
}

__global__ void k_interp_nearest(const float* __restrict__ x, float* __restrict__ y, int64_t c, int64_t t, int r) {
  const int64_t n = c * t * r;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / (t * r), j = i % (t * r);
    y[i] = x[row * t + j / r];
  }
}

// F.interpolate(mode='linear') over the last axis (ops.py:318-332); positions in fp64.
__global__ void k_interp_linear(const float* __restrict__ x, float* __restrict__ y, int64_t c, int64_t t,
                                int64_t size, int align) {
  const int64_t n = c * size;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / size, j = i % size;
    double pos;
    if (align) {
      pos = size > 1 ? (double)j * ((double)(t - 1) / (double)(size - 1)) : 0.0;
    } else {
      pos = ((double)j + 0.5) * ((double)t / (double)size) - 0.5;
      pos = fmin(fmax(pos, 0.0), (double)(t - 1));
    }
    const int64_t i0 = (int64_t)floor(pos);
    const int64_t i1 = i0 + 1 < t ? i0 + 1 : t - 1;
    const float f = (float)(pos - (double)i0);
    y[i] = x[row * t + i0] * (1.0f - f) + x[row * t + i1] * f;
  }
}

__global__ void k_hann(int n, int periodic, float* __restrict__ w) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const double den = periodic ? (double)n : (double)(n - 1);
    w[i] = (float)(0.5 - 0.5 * cos(2.0 * M_PI * (double)i / den));
  }
}

// batch of (rows, cols) -> (cols, rows) transposes through a padded LDS tile
__global__ void k_transpose(const float* __restrict__ x, float* __restrict__ y, int64_t rows, int64_t cols) {
  __shared__ float tile[32][33];
  const int64_t b = blockIdx.z;
  const float* xb = x + b * rows * cols;
  float* yb = y + b * rows * cols;
  const int64_t c0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
  for (int j = threadIdx.y; j < 32; j += blockDim.y) {
    const int64_t r = r0 + j, c = c0 + threadIdx.x;
    if (r < rows && c < cols) tile[j][threadIdx.x] = xb[r * cols + c];
  }
  __syncthreads();
  for (int j = threadIdx.y; j < 32; j += blockDim.y) {
    const int64_t c = c0 + j, r = r0 + threadIdx.x;
    if (r < rows && c < cols) yb[c * rows + r] = tile[threadIdx.x][j];
  }
}

// Strided 3-D copy y[i, j, l] = x[i, j, l], each side addressed by its own
// element strides: the batch transposes and channel packs around the DiT
// (cv3cpu/models/dit.py:151-153,96, cv3cpu/models/flow.py:83) without host copies.
__global__ void k_copy3(const float* __restrict__ x, float* __restrict__ y, int64_t d0, int64_t d1, int64_t d2,
                        int64_t xs0, int64_t xs1, int64_t xs2, int64_t ys0, int64_t ys1, int64_t ys2) {
  const int64_t n = d0 * d1 * d2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t l = i % d2, r = i / d2, j = r % d1, b = r / d1;
    y[b * ys0 + j * ys1 + l * ys2] = x[b * xs0 + j * xs1 + l * xs2];
  }
}

}  // namespace

extern "C" {

int cv3_act(int act, float param, const float* x, float* y, int64_t n, cv3_stream_t s) {
  CV3_ALIVE();
  if (n <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_act, dim3(grid_for(n)), dim3(256), 0, stream_of(s), act, param, x, y, n);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_binary(int op, const float* a, const float* b, float* y, int64_t n, float alpha, float beta, cv3_stream_t s) {
  CV3_ALIVE();
  if (n <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_binary, dim3(grid_for(n)), dim3(256), 0, stream_of(s), op, a, b, y, n, alpha, beta);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_snake(const float* x, const float* alpha, float* y, int64_t c, int64_t t, float eps, cv3_stream_t s) {
  CV3_ALIVE();
  if (c * t <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_snake, dim3(grid_for(c * t)), dim3(256), 0, stream_of(s), x, alpha, y, c, t, eps);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_snake_cl(const float* x, const float* alpha, float* y, int64_t t, int64_t c, float eps, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(t >= 0 && c > 0 && t * c < (1ll << 32), CV3_EINVAL, "snake: bad shape");
  if (t == 0) return CV3_OK;
  hipLaunchKernelGGL(k_snake_cl, dim3(grid_for(t * c)), dim3(256), 0, stream_of(s), x, alpha, y, (uint32_t)(t * c),
                     (uint32_t)c, eps);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_softmax_rows(const float* x, float* y, int64_t rows, int64_t cols, int log_softmax, cv3_stream_t s) {
  CV3_ALIVE();
  if (rows <= 0 || cols <= 0) return CV3_OK;
  CV3_REQUIRE(rows < (1ll << 31), CV3_EINVAL, "too many rows");
  hipLaunchKernelGGL(k_softmax_rows, dim3((unsigned)rows), dim3(256), 0, stream_of(s), x, y, cols, log_softmax);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_rms_norm(const float* x, const float* w, float* y, int64_t rows, int64_t cols, float eps, cv3_stream_t s) {
  CV3_ALIVE();
  if (rows <= 0 || cols <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)rows), dim3(256), 0, stream_of(s), x, w, y, cols, eps);
  CV3_LAUNCHED();
  return CV3_OK;
}

namespace {
int layer_norm(const float* x, float* y, int64_t rows, int64_t cols, float eps, const float* w, const float* b,
               const float* shift, const float* scale, int64_t mod_stride, int64_t rows_per_group, int* rexp,
               cv3_stream_t s) {
  auto a16 = [](const void* q) { return ((uintptr_t)q % 16) == 0; };
  const bool vec = cols % 4 == 0 && cols <= 4096 && a16(x) && a16(y) && a16(w) && a16(b) && a16(shift) &&
                   a16(scale) && mod_stride % 4 == 0;
  CV3_REQUIRE(!rexp || (vec && cols <= 1024), CV3_EUNSUPPORTED,
              "row exponents need 16-byte aligned rows of at most 1024 columns (cols = %lld)", (long long)cols);
  if (vec && cols <= 1024) {
    const dim3 grid((unsigned)ceil_div(rows, 4));
#define CV3_LNW(NV)                                                                                    \
  hipLaunchKernelGGL(k_layer_norm_wave<NV>, grid, dim3(256), 0, stream_of(s), x, y, rows, cols, eps, w, b, \
                     shift, scale, mod_stride, rows_per_group, rexp);
    if (cols <= 256) {
      CV3_LNW(1)
    } else if (cols <= 512) {
      CV3_LNW(2)
    } else {
      CV3_LNW(4)
    }
#undef CV3_LNW
  }
  else if (vec)
    hipLaunchKernelGGL(k_layer_norm4<4>, dim3((unsigned)rows), dim3(256), 0, stream_of(s), x, y, cols, eps, w, b,
                       shift, scale, mod_stride, rows_per_group);
  else
    hipLaunchKernelGGL(k_layer_norm, dim3((unsigned)rows), dim3(256), 0, stream_of(s), x, y, cols, eps, w, b, shift,
                       scale, mod_stride, rows_per_group);
  CV3_LAUNCHED();
  return CV3_OK;
}
}  // namespace

int cv3_layer_norm(const float* x, float* y, int64_t rows, int64_t cols, float eps, const float* w, const float* b,
                   const float* shift, const float* scale, int64_t mod_stride, int64_t rows_per_group,
                   cv3_stream_t s) {
  CV3_ALIVE();
  if (rows <= 0 || cols <= 0) return CV3_OK;
  return layer_norm(x, y, rows, cols, eps, w, b, shift, scale, mod_stride, rows_per_group, nullptr, s);
}

int cv3_layer_norm_rexp(const float* x, float* y, int64_t rows, int64_t cols, float eps, const float* w,
                        const float* b, const float* shift, const float* scale, int64_t mod_stride,
                        int64_t rows_per_group, int32_t* row_exp, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(row_exp, CV3_EINVAL, "layer_norm_rexp needs a row-exponent output");
  if (rows <= 0 || cols <= 0) return CV3_OK;
  return layer_norm(x, y, rows, cols, eps, w, b, shift, scale, mod_stride, rows_per_group, row_exp, s);
}

int cv3_rope_table(int kind, double theta, int dim, int64_t n, int64_t pos0, float* cos_out, float* sin_out,
                   cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(kind == 0 || kind == 1, CV3_EINVAL, "rope table kind must be 0 (dit) or 1 (qwen)");
  CV3_REQUIRE(dim > 0 && dim % 2 == 0, CV3_EINVAL, "rope dim must be even");
  if (n <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_rope_table, dim3(grid_for(n * dim)), dim3(256), 0, stream_of(s), kind, theta, dim, n, pos0,
                     cos_out, sin_out);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_rope_pairs(float* x, int64_t ld, int64_t rows, int64_t rows_per_batch, int rot, const float* cos_tab,
                   const float* sin_tab, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(rot % 2 == 0 && rot <= ld, CV3_EINVAL, "rotary width must be even and <= row width");
  if (rows <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_rope_pairs, dim3(grid_for(rows * rot / 2)), dim3(256), 0, stream_of(s), x, ld, rows,
                     rows_per_batch, rot, cos_tab, sin_tab);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_rope_half(float* x, int64_t nvec, int64_t per_pos, int64_t ld_pos, int d, const float* cos_tab,
                  const float* sin_tab, int64_t pos0, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(d % 2 == 0, CV3_EINVAL, "head dim must be even");
  if (nvec <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_rope_half, dim3(grid_for(nvec * d / 2)), dim3(256), 0, stream_of(s), x, nvec, per_pos, ld_pos,
                     d, cos_tab, sin_tab, pos0);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_cfg_euler(float* x, const float* d_cond, const float* d_uncond, int64_t n, float dt, float w,
                  cv3_stream_t s) {
  CV3_ALIVE();
  if (n <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_cfg_euler, dim3(grid_for(n)), dim3(256), 0, stream_of(s), x, d_cond, d_uncond, n, dt, w);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_interp_nearest(const float* x, float* y, int64_t c, int64_t t, int r, cv3_stream_t s) {
  CV3_ALIVE();
  if (c * t * r <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_interp_nearest, dim3(grid_for(c * t * r)), dim3(256), 0, stream_of(s), x, y, c, t, r);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_interp_linear(const float* x, float* y, int64_t c, int64_t t, int64_t size, int align_corners,
                      cv3_stream_t s) {
  CV3_ALIVE();
  if (c * size <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_interp_linear, dim3(grid_for(c * size)), dim3(256), 0, stream_of(s), x, y, c, t, size,
                     align_corners);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_hann_window(int n, int periodic, float* out, cv3_stream_t s) {
  CV3_ALIVE();
  if (n <= 0) return CV3_OK;
  hipLaunchKernelGGL(k_hann, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream_of(s), n, periodic, out);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_transpose(const float* x, float* y, int64_t batch, int64_t rows, int64_t cols, cv3_stream_t s) {
  CV3_ALIVE();
  if (batch * rows * cols <= 0) return CV3_OK;
  const dim3 grid((unsigned)ceil_div(cols, 32), (unsigned)ceil_div(rows, 32), (unsigned)batch);
  hipLaunchKernelGGL(k_transpose, grid, dim3(32, 8), 0, stream_of(s), x, y, rows, cols);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_copy_strided(const float* x, float* y, int64_t d0, int64_t d1, int64_t d2, const int64_t* x_strides,
                     const int64_t* y_strides, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(d0 >= 0 && d1 >= 0 && d2 >= 0, CV3_EINVAL, "negative copy extent");
  if (d0 * d1 * d2 == 0) return CV3_OK;
  hipLaunchKernelGGL(k_copy3, dim3(grid_for(d0 * d1 * d2)), dim3(256), 0, stream_of(s), x, y, d0, d1, d2,
                     x_strides[0], x_strides[1], x_strides[2], y_strides[0], y_strides[1], y_strides[2]);
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // extern "C"
