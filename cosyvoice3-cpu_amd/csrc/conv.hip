// 1-D convolution as an implicit GEMM on the matrix cores (cv3cpu/ops.py:165-219).
//
//   y[co, t] = epi( sum_{c < Cin/g, j < k} W[co, c, j] * xin[g*Cin/g + c, t*stride + j*dil - pad_l] )
//
// where xin is the input after an optional nearest-neighbour upsample by `up`
// (cv3cpu/ops.py:335-336 followed by a causal conv, cv3cpu/models/hift.py:139-142):
// xin[c, u] = x[c, u / up] for 0 <= u < T_in * up, zero outside (the zero padding).
// The upsampled signal is never materialised.  x and y are addressed through
// (channel, time) strides, so channels-first (C, T) and channels-last (T, C)
// buffers both work.
//
// GEMM view per group: M = Cout/g (rows of W), N = T_out, K = (Cin/g) * k with
// the weight's natural (c, j) order.  Tiles, MFMA and K permutation are those of
// the linear GEMM: a 64 x 64 tile per workgroup, 32 x 32 per wave,
// v_mfma_f32_32x32x2_f32, BK = 16.
//
// Epilogue: y = residual + act(acc + bias), or y = snake(acc + bias) with a
// per-output-channel alpha (the resblock's second Snake, hift.py:124).
#include "bf16x3.hpp"
#include "common.hpp"
#include "epilogue.hpp"

using namespace cv3;

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
constexpr int BM = 64, BN = 64, BK = 16, LDS_STRIDE = BK + 4;

struct ConvParams {
  const float* x;
  int64_t x_cs, x_ts, t_in;
  const float* w;  // [cout, cin_g, k] contiguous
  int64_t cout, cin_g, k;
  const float* bias;
  int64_t groups, stride, dil, pad_l, up;
  int64_t t_out;
  float* y;
  int64_t y_cs, y_ts;
  int act;
  float act_param;
  const float* snake_alpha;
  float snake_eps;
  const float* res;
  int64_t r_cs, r_ts;
};

__device__ __forceinline__ float xin(const ConvParams& p, int64_t c, int64_t u) {
  if (u < 0 || u >= p.t_in * p.up) return 0.f;
  return p.x[c * p.x_cs + (u / p.up) * p.x_ts];
}

__global__ __launch_bounds__(256) void k_conv_mfma(ConvParams p) {
  __shared__ float As[2][BM * LDS_STRIDE];
  __shared__ float Bs[2][BN * LDS_STRIDE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t g = blockIdx.z;
  const int64_t cout_g = p.cout / p.groups;
  const int64_t m0 = (int64_t)blockIdx.y * BM;  // output channel within group
  const int64_t n0 = (int64_t)blockIdx.x * BN;  // output time
  const int64_t K = p.cin_g * p.k;
  const float* wg = p.w + g * cout_g * K;
  const int64_t cbase = g * p.cin_g;

  // A (weights): thread -> row tid/4, 4 consecutive k at (tid%4)*4
  const int arow = tid >> 2, ak = (tid & 3) * 4;
  // B (im2col): thread -> k index tid/16, 4 consecutive times at (tid%16)*4
  const int bk = tid >> 4, bt = (tid & 15) * 4;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int r32 = lane & 31, h = lane >> 5;

  auto load_a = [&](int64_t kk, float* out4) {
    const int64_t row = m0 + arow;
#pragma unroll
    for (int i = 0; i < 4; ++i) out4[i] = (row < cout_g && kk + i < K) ? wg[row * K + kk + i] : 0.f;
  };
  auto load_b = [&](int64_t kk, float* out4) {
    const int64_t kidx = kk + bk;
    if (kidx >= K) {
#pragma unroll
      for (int i = 0; i < 4; ++i) out4[i] = 0.f;
      return;
    }
    const int64_t c = kidx / p.k, j = kidx % p.k;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t t = n0 + bt + i;
      out4[i] = t < p.t_out ? xin(p, cbase + c, t * p.stride + j * p.dil - p.pad_l) : 0.f;
    }
  };

  float ra[4], rb[4];
  load_a(ak, ra);
  load_b(0, rb);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    As[0][arow * LDS_STRIDE + ak + i] = ra[i];
    Bs[0][(bt + i) * LDS_STRIDE + bk] = rb[i];
  }
  __syncthreads();

  f32x16 acc = {0.f};
  const int64_t ksteps = ceil_div(K, BK);
  for (int64_t s = 0; s < ksteps; ++s) {
    const int buf = s & 1;
    const bool more = s + 1 < ksteps;
    if (more) {
      load_a((s + 1) * BK + ak, ra);
      load_b((s + 1) * BK, rb);
    }
    const float* as = &As[buf][(wm + r32) * LDS_STRIDE + h * 4];
    const float* bs = &Bs[buf][(wn + r32) * LDS_STRIDE + h * 4];
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
      const float4 av = *reinterpret_cast<const float4*>(as + gq * 8);
      const float4 bv = *reinterpret_cast<const float4*>(bs + gq * 8);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        As[buf ^ 1][arow * LDS_STRIDE + ak + i] = ra[i];
        Bs[buf ^ 1][(bt + i) * LDS_STRIDE + bk] = rb[i];
      }
    }
    __syncthreads();
  }

  // acc reg i -> (row = output channel, col = time): row (i/4)*8 + h*4 + i%4, col lane%32.
  // The epilogue's operands are loaded for all 16 registers before the first store:
  // y may alias the residual, and a load after a store to y would wait for it.
  const int64_t t = n0 + wn + r32;
  if (t >= p.t_out) return;
  float bias[16], alpha[16], res[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t co_g = min(m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3), cout_g - 1);
    const int64_t co = g * cout_g + co_g;
    bias[i] = p.bias ? p.bias[co] : 0.f;
    alpha[i] = p.snake_alpha ? p.snake_alpha[co] : 0.f;
    res[i] = p.res ? p.res[co * p.r_cs + t * p.r_ts] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t co_g = m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3);
    if (co_g < cout_g) {
      const int64_t co = g * cout_g + co_g;
      float v = acc[i] + bias[i];
      if (p.snake_alpha) {
        const float a = alpha[i];
        const float sn = sinf(a * v);
        v = v + (1.0f / (a + p.snake_eps)) * (sn * sn);
      } else {
        v = apply_act(p.act, v, p.act_param);
      }
      if (p.res) v = res[i] + v;
      p.y[co * p.y_cs + t * p.y_ts] = v;
    }
  }
}

// Fast path for stride 1 and groups 1 (every HiFT conv but the strided source_downs):
// the weight is repacked (cout, k, cin), so with cin % 64 == 0 a BK = 32 stage is 32
// channels of one tap and its im2col rows are plain shifted rows of x, with 32-bit
// index math done once per stage.  A thread owns one time column and 8 channels of
// the B tile, so its 8 loads per stage are coalesced over the wave along time (x
// time-contiguous).  Global loads run two stages ahead in ping-pong register sets, as
// in the linear GEMM; taps and channels of the K loop follow from the stage index.
struct ConvFast {
  const float* x;
  int64_t x_cs;
  int t_in, up;
  const float* w;  // [cout, k, cin]
  int cout, cin, k, dil, pad_l, t_out;
  const float* bias;
  float* y;
  int64_t y_cs, y_ts;
  int act;
  float act_param;
  const float* snake_alpha;
  float snake_eps;
  const float* res;
  int64_t r_cs, r_ts;
  float* part;  // split-K partials [ksplit, cout, t_out] (ksplit > 1), epilogue in k_conv_reduce
  int ksplit;
};
constexpr int FBK = 32, FLS = FBK + 4;

__device__ __forceinline__ void fast_mma(const float* As, const float* Bs, int wm, int wn, int r32, int h,
                                         f32x16& acc) {
  const float* as = &As[(wm + r32) * FLS + h * 4];
  const float* bs = &Bs[(wn + r32) * FLS + h * 4];
#pragma unroll
  for (int g = 0; g < FBK / 8; ++g) {
    const float4 av = *reinterpret_cast<const float4*>(as + g * 8);
    const float4 bv = *reinterpret_cast<const float4*>(bs + g * 8);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
  }
}

__global__ __launch_bounds__(256) void k_conv_fast(ConvFast p) {
  __shared__ float As[2][64 * FLS];  // [co][k]
  __shared__ float Bs[2][64 * FLS];  // [t][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int lrow = tid >> 3, lk = (tid & 7) * 4;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int r32 = lane & 31, h = lane >> 5;
  const int K = p.k * p.cin;
  const float* wa0 = p.w + (int64_t)min(m0 + lrow, p.cout - 1) * K + lk;
  const float* wa1 = p.w + (int64_t)min(m0 + lrow + 32, p.cout - 1) * K + lk;
  const int tt = tid & 63, cg = tid >> 6;  // B: time column, group of 8 channels
  const int t = n0 + tt;
  const int tin_up = p.t_in * p.up;
  const float* xb = p.x + (int64_t)(cg * 8) * p.x_cs;
  // this workgroup's stages: all of them, or slice blockIdx.z of ksplit (an even count)
  const int S = K / FBK / p.ksplit;
  const int sb = blockIdx.z * S;
  const int cpt = p.cin / FBK;  // stages per tap
  f32x16 acc = {0.f};
  float4 xa0, xa1, ya0, ya1;
  float xv[8], yv[8];
  // stage s: tap j = s / cpt, channels [c0, c0 + 32), c0 = (s % cpt) * 32; the padded and
  // out-of-range time positions load a valid element and are replaced by zero after the load
#define CV3_CLOAD(A0, A1, V, S_)                                                                  \
  {                                                                                               \
    const int s_ = sb + (S_);                                                                     \
    const int j_ = s_ / cpt, c0_ = (s_ - j_ * cpt) * FBK;                                         \
    A0 = *reinterpret_cast<const float4*>(wa0 + s_ * FBK);                                        \
    A1 = *reinterpret_cast<const float4*>(wa1 + s_ * FBK);                                        \
    const int u_ = t + j_ * p.dil - p.pad_l;                                                      \
    const bool ok_ = u_ >= 0 && u_ < tin_up && t < p.t_out;                                       \
    const int src_ = ok_ ? (p.up == 1 ? u_ : (int)((unsigned)u_ / (unsigned)p.up)) : 0;           \
    const float* xp_ = xb + (int64_t)c0_ * p.x_cs + src_;                                         \
    _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_) V[i_] = xp_[(int64_t)i_ * p.x_cs];           \
    _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_) V[i_] = ok_ ? V[i_] : 0.f;                   \
  }
#define CV3_CSTORE(BUF, A0, A1, V)                                                                       \
  *reinterpret_cast<float4*>(&As[BUF][lrow * FLS + lk]) = A0;                                            \
  *reinterpret_cast<float4*>(&As[BUF][(lrow + 32) * FLS + lk]) = A1;                                     \
  *reinterpret_cast<float4*>(&Bs[BUF][tt * FLS + cg * 8]) = make_float4(V[0], V[1], V[2], V[3]);         \
  *reinterpret_cast<float4*>(&Bs[BUF][tt * FLS + cg * 8 + 4]) = make_float4(V[4], V[5], V[6], V[7]);
  CV3_CLOAD(xa0, xa1, xv, 0)
  CV3_CLOAD(ya0, ya1, yv, 1)
  CV3_CSTORE(0, xa0, xa1, xv)
  __syncthreads();
  for (int s = 0; s + 2 < S; s += 2) {
    // LDS[0] = stage s, y = stage s + 1 in flight
    CV3_CLOAD(xa0, xa1, xv, s + 2)
    __builtin_amdgcn_sched_barrier(0);  // issue the loads before the MFMAs
    fast_mma(As[0], Bs[0], wm, wn, r32, h, acc);
    CV3_CSTORE(1, ya0, ya1, yv)
    __syncthreads();
    CV3_CLOAD(ya0, ya1, yv, s + 3)
    __builtin_amdgcn_sched_barrier(0);
    fast_mma(As[1], Bs[1], wm, wn, r32, h, acc);
    CV3_CSTORE(0, xa0, xa1, xv)
    __syncthreads();
  }
  fast_mma(As[0], Bs[0], wm, wn, r32, h, acc);
  CV3_CSTORE(1, ya0, ya1, yv)
  __syncthreads();
  fast_mma(As[1], Bs[1], wm, wn, r32, h, acc);
#undef CV3_CLOAD
#undef CV3_CSTORE
  const int tc = n0 + wn + r32;
  if (tc >= p.t_out) return;
  if (p.ksplit > 1) {  // raw partial sums; k_conv_reduce adds the slices in order
    float* dst = p.part + (int64_t)blockIdx.z * p.cout * p.t_out + tc;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int co = m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3);
      if (co < p.cout) dst[(int64_t)co * p.t_out] = acc[i];
    }
    return;
  }
  // epilogue (same operand-first order as k_conv_mfma)
  float bias[16], alpha[16], res[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int co = min(m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3), p.cout - 1);
    bias[i] = p.bias ? p.bias[co] : 0.f;
    alpha[i] = p.snake_alpha ? p.snake_alpha[co] : 0.f;
    res[i] = p.res ? p.res[co * p.r_cs + tc * p.r_ts] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int co = m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3);
    if (co < p.cout) {
      float v = acc[i] + bias[i];
      if (p.snake_alpha) {
        const float sn = sinf(alpha[i] * v);
        v = v + (1.0f / (alpha[i] + p.snake_eps)) * (sn * sn);
      } else {
        v = apply_act(p.act, v, p.act_param);
      }
      if (p.res) v = res[i] + v;
      p.y[co * p.y_cs + tc * p.y_ts] = v;
    }
  }
}

// Split-K epilogue: y[co, t] = epi(sum_z part[z, co, t] + bias[co]), slices added in
// order z = 0, 1, ... so the result does not depend on scheduling.
__global__ void k_conv_reduce(ConvFast p) {
  const int64_t n = (int64_t)p.cout * p.t_out;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int co = (int)(e / p.t_out), t = (int)(e - (int64_t)co * p.t_out);
    const float r = p.res ? p.res[co * p.r_cs + t * p.r_ts] : 0.f;
    float acc = p.part[e];
    for (int z = 1; z < p.ksplit; ++z) acc += p.part[(int64_t)z * n + e];
    float v = acc + (p.bias ? p.bias[co] : 0.f);
    if (p.snake_alpha) {
      const float a = p.snake_alpha[co];
      const float sn = sinf(a * v);
      v = v + (1.0f / (a + p.snake_eps)) * (sn * sn);
    } else {
      v = apply_act(p.act, v, p.act_param);
    }
    if (p.res) v = r + v;
    p.y[co * p.y_cs + t * p.y_ts] = v;
  }
}

// Channels-last stride-1 conv (groups 1) as an implicit GEMM fed by global -> LDS DMA,
// the structure of the linear GEMM's k_gemm_dma: C[t, co] over M = t_out time rows,
// N = cout, K = k * cin in (tap, channel) order, weight repacked (cout, k, cin).  A BK =
// 32 stage is 32 channels of one tap, so each A row is a 128-byte piece of one input
// row x[(t + tap*dil - pad_l) / up] (nearest upsample fused); rows outside the padded
// input read a static zero row instead, so the DMA needs no predicates.  Rows are
// XOR-swizzled in LDS and the ring holds three stages (see k_gemm_dma in gemm.hip).
__device__ float g_conv_zero_row[32];  // zero-initialised, only ever read

struct ConvCL {
  const float* x;
  int64_t ldx;
  int t_in, up, cin;
  const float* w;  // [cout, k, cin]
  int cout, k, dil, pad_l, t_out;
  const float* bias;
  float* y;
  int64_t y_ts, y_cs;
  int act;
  float act_param;
  const float* snake_alpha;
  float snake_eps;
  const float* res;
  int64_t r_ts, r_cs;
  float* part;  // split-K partials [ksplit, t_out, cout]
  int ksplit;
};
#define CV3_VMCNT(n) (((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

struct ClSrc {
  int r0, r1;              // this lane's two A rows (time)
  const float* b0;         // this lane's two B rows (weight), at its chunk
  const float* b1;
  int lc, lc8;             // chunk offsets of rows r0 and r1 (the swizzle of k_gemm_dma)
};

__device__ __forceinline__ void cl_stage(const ConvCL& p, const ClSrc& s, int sg, float* as, float* bs, int w) {
  const int cpt = p.cin / 32;
  const int j = sg / cpt, c0 = (sg - j * cpt) * 32;
  const int tin_up = p.t_in * p.up;
  const int u0 = s.r0 + j * p.dil - p.pad_l, u1 = s.r1 + j * p.dil - p.pad_l;
  const bool ok0 = s.r0 < p.t_out && u0 >= 0 && u0 < tin_up;
  const bool ok1 = s.r1 < p.t_out && u1 >= 0 && u1 < tin_up;
  const int q0 = ok0 ? (p.up == 1 ? u0 : (int)((unsigned)u0 / (unsigned)p.up)) : 0;
  const int q1 = ok1 ? (p.up == 1 ? u1 : (int)((unsigned)u1 / (unsigned)p.up)) : 0;
  const float* a0 = ok0 ? p.x + (int64_t)q0 * p.ldx + c0 + s.lc : g_conv_zero_row + s.lc;
  const float* a1 = ok1 ? p.x + (int64_t)q1 * p.ldx + c0 + s.lc8 : g_conv_zero_row + s.lc8;
  __builtin_amdgcn_global_load_lds(a0, as + (w * 16) * 32, 16, 0, 0);
  __builtin_amdgcn_global_load_lds(a1, as + (w * 16 + 8) * 32, 16, 0, 0);
  __builtin_amdgcn_global_load_lds(s.b0 + sg * 32, bs + (w * 16) * 32, 16, 0, 0);
  __builtin_amdgcn_global_load_lds(s.b1 + sg * 32, bs + (w * 16 + 8) * 32, 16, 0, 0);
}

__device__ __forceinline__ void cl_mma(const float* as, const float* bs, int arow, int brow, int sw, int h,
                                       f32x16& acc) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int c = ((2 * g + h) ^ sw) * 4;
    const float4 av = *reinterpret_cast<const float4*>(as + arow + c);
    const float4 bv = *reinterpret_cast<const float4*>(bs + brow + c);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
  }
}

// Epilogue of the channels-last conv's 32 x 32 accumulator (reg i -> time row
// m0 + wm + (i/4)*8 + h*4 + i%4, output channel n0 + wn + lane%32): split-K partials, or
// bias, Snake / activation and residual.
__device__ __forceinline__ void cl_epilogue(const ConvCL& p, const f32x16& acc, int m0, int n0, int wm, int wn,
                                            int r32, int h) {
  const int co = n0 + wn + r32;
  if (co >= p.cout) return;
  if (p.ksplit > 1) {
    float* dst = p.part + (int64_t)blockIdx.z * p.t_out * p.cout + co;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tr = m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3);
      if (tr < p.t_out) dst[(int64_t)tr * p.cout] = acc[i];
    }
    return;
  }
  const float bias = p.bias ? p.bias[co] : 0.f;
  const float alpha = p.snake_alpha ? p.snake_alpha[co] : 0.f;
  float res[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tr = min(m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3), p.t_out - 1);
    res[i] = p.res ? p.res[(int64_t)tr * p.r_ts + co * p.r_cs] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tr = m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3);
    if (tr < p.t_out) {
      float v = acc[i] + bias;
      if (p.snake_alpha) {
        const float sn = sinf(alpha * v);
        v = v + (1.0f / (alpha + p.snake_eps)) * (sn * sn);
      } else {
        v = apply_act(p.act, v, p.act_param);
      }
      if (p.res) v = res[i] + v;
      p.y[(int64_t)tr * p.y_ts + co * p.y_cs] = v;
    }
  }
}

__global__ __launch_bounds__(256) void k_conv_cl_dma(ConvCL p, int tiles_m) {
  __shared__ float A0[2048], A1[2048], A2[2048];
  __shared__ float B0[2048], B1[2048], B2[2048];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int T = gridDim.x, L = blockIdx.x;
  const int t = (T % 8 == 0) ? (L % 8) * (T / 8) + L / 8 : L;
  const int m0 = (t % tiles_m) * 64, n0 = (t / tiles_m) * 64;
  const int lr = lane >> 3;
  const int K = p.k * p.cin;
  ClSrc src;
  src.lc = ((lane & 7) ^ (lr >> 1)) * 4;
  src.lc8 = src.lc ^ 16;
  src.r0 = m0 + w * 16 + lr;
  src.r1 = src.r0 + 8;
  src.b0 = p.w + (int64_t)min(n0 + w * 16 + lr, p.cout - 1) * K + src.lc;
  src.b1 = p.w + (int64_t)min(n0 + w * 16 + 8 + lr, p.cout - 1) * K + src.lc8;
  const int wm = (w >> 1) * 32, wn = (w & 1) * 32;
  const int r32 = lane & 31, h = lane >> 5, sw = (r32 >> 1) & 7;
  const int arow = (wm + r32) * 32, brow = (wn + r32) * 32;
  const int S = K / 32 / p.ksplit;  // this workgroup's stages
  const int sb = blockIdx.z * S;
  f32x16 acc = {0.f};
  cl_stage(p, src, sb, A0, B0, w);
  cl_stage(p, src, sb + min(1, S - 1), A1, B1, w);
#define CV3_CL_STEP(AN, BN_, AC, BC, ST)                            \
  __builtin_amdgcn_sched_barrier(0);                                \
  __builtin_amdgcn_s_waitcnt(CV3_VMCNT(4));                         \
  __builtin_amdgcn_s_barrier();                                     \
  __builtin_amdgcn_sched_barrier(0);                                \
  cl_stage(p, src, sb + min((ST) + 2, S - 1), AN, BN_, w);          \
  __builtin_amdgcn_sched_barrier(0);                                \
  cl_mma(AC, BC, arow, brow, sw, h, acc);
  int st = 0;
  for (; st + 3 <= S; st += 3) {
    CV3_CL_STEP(A2, B2, A0, B0, st)
    CV3_CL_STEP(A0, B0, A1, B1, st + 1)
    CV3_CL_STEP(A1, B1, A2, B2, st + 2)
  }
  if (st < S) {
    CV3_CL_STEP(A2, B2, A0, B0, st)
    if (st + 1 < S) { CV3_CL_STEP(A0, B0, A1, B1, st + 1) }
  }
#undef CV3_CL_STEP
  // no DMA may still be writing this workgroup's LDS when it ends
  __builtin_amdgcn_s_waitcnt(CV3_VMCNT(0));
  cl_epilogue(p, acc, m0, n0, wm, wn, r32, h);
}

// The channels-last conv of k_conv_cl_dma on the bfloat16 matrix cores: x split into its
// three bfloat16 planes on its way into LDS (bf16x3.hpp), the packed weight held as planes
// [3][cout][k * cin], six 32x32x16 bf16 products per product (hh into one accumulator, the rest
// into a second).  A stage is 32 channels of one tap, as there; the rows of 64 bytes per plane
// sit at slot r * 4 + (c ^ (r / 4) % 4) (16-byte chunk c), conflict-free for a 16-lane read.
// Loads run two stages ahead in ping-pong registers; a slice's stage count must be even.
struct ClStageX {
  float4 a0, a1;     // x: this thread's time row, channels 8 lc .. + 7 of the stage
  uint4 b0, b1, b2;  // weight planes: this thread's output channel, the same 8 k
};

__device__ __forceinline__ int cl_xslot(int row, int chunk) { return row * 4 + (chunk ^ ((row >> 2) & 3)); }

__global__ __launch_bounds__(256) void k_conv_cl_x3(ConvCL p, const uint16_t* wp, int64_t wps, int tiles_m) {
  __shared__ uint4 sA[2][3][64 * 4];
  __shared__ uint4 sB[2][3][64 * 4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int T = gridDim.x, L = blockIdx.x;
  const int t = (T % 8 == 0) ? (L % 8) * (T / 8) + L / 8 : L;
  const int m0 = (t % tiles_m) * 64, n0 = (t / tiles_m) * 64;
  const int K = p.k * p.cin, cpt = p.cin / 32, tin_up = p.t_in * p.up;
  const int lr = tid >> 2, lc = tid & 3, tr = m0 + lr;
  const int wslot = cl_xslot(lr, lc);
  const uint16_t* pbr = wp + (int64_t)min(n0 + lr, p.cout - 1) * K + lc * 8;
  const int wm = (w >> 1) * 32, wn = (w & 1) * 32, r32 = lane & 31, h = lane >> 5;
  const int ar = wm + r32, br = wn + r32, asw = (ar >> 2) & 3, bsw = (br >> 2) & 3;
  const int S = K / 32 / p.ksplit, sb = blockIdx.z * S;
  f32x16 big = {0.f}, small = {0.f};

  auto load = [&](ClStageX& x, int sg) {
    const int j = sg / cpt, c0 = (sg - j * cpt) * 32;
    const int u = tr + j * p.dil - p.pad_l;
    const bool ok = tr < p.t_out && u >= 0 && u < tin_up;
    const int q = ok ? (p.up == 1 ? u : (int)((unsigned)u / (unsigned)p.up)) : 0;
    const float* a = ok ? p.x + (int64_t)q * p.ldx + c0 + lc * 8 : g_conv_zero_row + lc * 8;
    x.a0 = *reinterpret_cast<const float4*>(a);
    x.a1 = *reinterpret_cast<const float4*>(a + 4);
    const uint16_t* b = pbr + (int64_t)sg * 32;
    x.b0 = *reinterpret_cast<const uint4*>(b);
    x.b1 = *reinterpret_cast<const uint4*>(b + wps);
    x.b2 = *reinterpret_cast<const uint4*>(b + 2 * wps);
  };
  auto store = [&](int buf, const ClStageX& x) {
    uint4 hi, mid, lo;
    split_x3(x.a0, x.a1, hi, mid, lo);
    sA[buf][0][wslot] = hi;
    sA[buf][1][wslot] = mid;
    sA[buf][2][wslot] = lo;
    sB[buf][0][wslot] = x.b0;
    sB[buf][1][wslot] = x.b1;
    sB[buf][2][wslot] = x.b2;
  };
  auto mma = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 2 + h;
      const int sa = ar * 4 + (c ^ asw), sbb = br * 4 + (c ^ bsw);
      const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, sA[buf][0][sa]);
      const bf16x8_t am = __builtin_bit_cast(bf16x8_t, sA[buf][1][sa]);
      const bf16x8_t al = __builtin_bit_cast(bf16x8_t, sA[buf][2][sa]);
      const bf16x8_t bh = __builtin_bit_cast(bf16x8_t, sB[buf][0][sbb]);
      const bf16x8_t bm = __builtin_bit_cast(bf16x8_t, sB[buf][1][sbb]);
      const bf16x8_t bl = __builtin_bit_cast(bf16x8_t, sB[buf][2][sbb]);
      big = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, big, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bm, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bh, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bm, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, small, 0, 0, 0);
    }
  };

  // S even and >= 2
  ClStageX x, y;
  load(x, sb);
  load(y, sb + 1);
  store(0, x);
  __syncthreads();
  for (int s = 0; s + 2 < S; s += 2) {
    load(x, sb + s + 2);
    __builtin_amdgcn_sched_barrier(0);
    mma(0);
    store(1, y);
    __syncthreads();
    load(y, sb + s + 3);
    __builtin_amdgcn_sched_barrier(0);
    mma(1);
    store(0, x);
    __syncthreads();
  }
  mma(0);
  store(1, y);
  __syncthreads();
  mma(1);
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = big[i] + small[i];
  cl_epilogue(p, acc, m0, n0, wm, wn, r32, h);
}

// k_conv_cl_x3 with the weight planes packed once in MFMA fragment order (cv3_split_x3_frag over
// the packed (cout, k * cin) rows): frag[p][nb][t][l] is plane p of w[32 nb + l % 32][16 t + 8 (l / 32)
// .. + 7], the B operand of lane l for 16-k step t of output-channel block nb, so each wave loads
// its B fragments straight into registers two stages ahead and only x goes through LDS.  Every
// MFMA sees the operands k_conv_cl_x3 gives it, in the same order: the results are the same bits.
__global__ __launch_bounds__(256) void k_conv_cl_x3f(ConvCL p, const uint4* frag, int64_t per_plane, int tiles_m) {
  __shared__ uint4 sA[2][3][64 * 4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int T = gridDim.x, L = blockIdx.x;
  const int t = (T % 8 == 0) ? (L % 8) * (T / 8) + L / 8 : L;
  const int m0 = (t % tiles_m) * 64, n0 = (t / tiles_m) * 64;
  const int K = p.k * p.cin, cpt = p.cin / 32, tin_up = p.t_in * p.up;
  const int lr = tid >> 2, lc = tid & 3, tr = m0 + lr;
  const int wslot = cl_xslot(lr, lc);
  const int wm = (w >> 1) * 32, wn = (w & 1) * 32, r32 = lane & 31, h = lane >> 5;
  const int ar = wm + r32, asw = (ar >> 2) & 3;
  const int S = K / 32 / p.ksplit, sb = blockIdx.z * S;
  // this wave's 32-channel block; one past the last (cout % 64 in 1 .. 32) reads the last one
  // instead, its channels are dropped by cl_epilogue
  const int nblk = min((n0 + wn) >> 5, (p.cout - 1) >> 5);
  const uint4* fb = frag + (int64_t)nblk * (K / 16) * 64 + lane;
  f32x16 big = {0.f}, small = {0.f};
  struct XA {
    float4 a0, a1;  // this thread's time row, channels 8 lc .. + 7 of the stage
  };
  struct BF {
    uint4 v[2][3];  // [16-k step of the stage][plane]
  };

  auto load = [&](XA& x, int sg) {
    const int j = sg / cpt, c0 = (sg - j * cpt) * 32;
    const int u = tr + j * p.dil - p.pad_l;
    const bool ok = tr < p.t_out && u >= 0 && u < tin_up;
    const int q = ok ? (p.up == 1 ? u : (int)((unsigned)u / (unsigned)p.up)) : 0;
    const float* a = ok ? p.x + (int64_t)q * p.ldx + c0 + lc * 8 : g_conv_zero_row + lc * 8;
    x.a0 = *reinterpret_cast<const float4*>(a);
    x.a1 = *reinterpret_cast<const float4*>(a + 4);
  };
  auto loadb = [&](BF& b, int sg) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int pl = 0; pl < 3; ++pl) b.v[ks][pl] = fb[pl * per_plane + (int64_t)(2 * sg + ks) * 64];
  };
  auto store = [&](int buf, const XA& x) {
    uint4 hi, mid, lo;
    split_x3(x.a0, x.a1, hi, mid, lo);
    sA[buf][0][wslot] = hi;
    sA[buf][1][wslot] = mid;
    sA[buf][2][wslot] = lo;
  };
  auto mma = [&](int buf, const BF& b) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 2 + h;
      const int sa = ar * 4 + (c ^ asw);
      const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, sA[buf][0][sa]);
      const bf16x8_t am = __builtin_bit_cast(bf16x8_t, sA[buf][1][sa]);
      const bf16x8_t al = __builtin_bit_cast(bf16x8_t, sA[buf][2][sa]);
      const bf16x8_t bh = __builtin_bit_cast(bf16x8_t, b.v[ks][0]);
      const bf16x8_t bm = __builtin_bit_cast(bf16x8_t, b.v[ks][1]);
      const bf16x8_t bl = __builtin_bit_cast(bf16x8_t, b.v[ks][2]);
      big = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, big, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bm, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bh, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bm, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, small, 0, 0, 0);
    }
  };

  // S even and >= 2: x ping-pongs through registers x / y and LDS buffers 0 / 1, the B fragments
  // of the even and odd stages through b0 / b1, each refilled right after its use
  XA x, y;
  BF b0, b1;
  load(x, sb);
  load(y, sb + 1);
  loadb(b0, sb);
  loadb(b1, sb + 1);
  store(0, x);
  __syncthreads();
  for (int s = 0; s + 2 < S; s += 2) {
    load(x, sb + s + 2);
    __builtin_amdgcn_sched_barrier(0);
    mma(0, b0);
    loadb(b0, sb + s + 2);
    store(1, y);
    __syncthreads();
    load(y, sb + s + 3);
    __builtin_amdgcn_sched_barrier(0);
    mma(1, b1);
    loadb(b1, sb + s + 3);
    store(0, x);
    __syncthreads();
  }
  mma(0, b0);
  store(1, y);
  __syncthreads();
  mma(1, b1);
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = big[i] + small[i];
  cl_epilogue(p, acc, m0, n0, wm, wn, r32, h);
}

// Split-K epilogue of k_conv_cl_dma: slices added in order z = 0, 1, ...
__global__ void k_conv_cl_reduce(ConvCL p) {
  const int64_t n = (int64_t)p.t_out * p.cout;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int tr = (int)(e / p.cout), co = (int)(e - (int64_t)tr * p.cout);
    const float r = p.res ? p.res[(int64_t)tr * p.r_ts + co * p.r_cs] : 0.f;
    float acc = p.part[e];
    for (int z = 1; z < p.ksplit; ++z) acc += p.part[(int64_t)z * n + e];
    float v = acc + (p.bias ? p.bias[co] : 0.f);
    if (p.snake_alpha) {
      const float a = p.snake_alpha[co];
      const float sn = sinf(a * v);
      v = v + (1.0f / (a + p.snake_eps)) * (sn * sn);
    } else {
      v = apply_act(p.act, v, p.act_param);
    }
    if (p.res) v = r + v;
    p.y[(int64_t)tr * p.y_ts + co * p.y_cs] = v;
  }
}

// groups == C convolution as k shifted multiply-accumulates (ops.py:222-237)
__global__ void k_depthwise(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
                            float* __restrict__ y, int64_t c, int64_t t_in, int64_t k, int64_t dil, int64_t pad_l,
                            int64_t t_out) {
  const int64_t n = c * t_out;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ch = i / t_out, t = i % t_out;
    float acc = 0.f;
    for (int64_t j = 0; j < k; ++j) {
      const int64_t u = t + j * dil - pad_l;
      const float xv = (u >= 0 && u < t_in) ? x[ch * t_in + u] : 0.f;
      acc = acc + w[ch * k + j] * xv;
    }
    if (bias) acc += bias[ch];
    y[i] = acc;
  }
}

}  // namespace

namespace cv3 {
int conv_cl(const float* x, int64_t batch, int64_t t, int64_t ldx, const float* w, int64_t cout, int64_t k,
            int64_t cin_g, int64_t pad_l, const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi,
            hipStream_t st);
int64_t x3_frag_plane(int64_t n, int64_t k);  // gemm.hip: one plane of a fragment-ordered weight
int conv_cl_x3f(const float* x, int64_t batch, int64_t t, int64_t ldx, const uint16_t* frag, int64_t cout, int64_t k,
                int64_t cin_g, int64_t pad_l, const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi,
                hipStream_t st);
}

extern "C" {

int cv3_conv1d_cl(const float* x, int64_t batch, int64_t t, int64_t cin, int64_t ldx, const float* w_packed,
                  int64_t cout, int64_t k, int64_t groups, int64_t pad_l, const float* bias, float* y, int64_t ldy,
                  const cv3_epilogue* epi, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(groups >= 1 && cin % groups == 0 && cout % groups == 0, CV3_EASSERT,
              "channels %lld/%lld not divisible by groups %lld", (long long)cin, (long long)cout, (long long)groups);
  CV3_REQUIRE(cout / groups == 64, CV3_EUNSUPPORTED, "channels-last conv takes 64 output channels per group");
  CV3_REQUIRE(ldx >= cin && ldy >= cout && k >= 1, CV3_EINVAL, "bad channels-last conv strides");
  if (batch <= 0 || t <= 0) return CV3_OK;
  return conv_cl(x, batch, t, ldx, w_packed, cout, k, cin / groups, pad_l, bias, y, ldy, epi, stream_of(s));
}


int cv3_conv1d_cl_x3f(const float* x, int64_t batch, int64_t t, int64_t cin, int64_t ldx, const uint16_t* w_frag,
                      int64_t cout, int64_t k, int64_t groups, int64_t pad_l, const float* bias, float* y, int64_t ldy,
                      const cv3_epilogue* epi, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(w_frag, CV3_EINVAL, "null weight fragments");
  CV3_REQUIRE(groups >= 1 && cin % groups == 0 && cout % groups == 0, CV3_EASSERT,
              "channels %lld/%lld not divisible by groups %lld", (long long)cin, (long long)cout, (long long)groups);
  CV3_REQUIRE(cout / groups == 64, CV3_EUNSUPPORTED, "channels-last conv takes 64 output channels per group");
  CV3_REQUIRE(ldx >= cin && ldy >= cout && k >= 1, CV3_EINVAL, "bad channels-last conv strides");
  if (batch <= 0 || t <= 0) return CV3_OK;
  return conv_cl_x3f(x, batch, t, ldx, w_frag, cout, k, cin / groups, pad_l, bias, y, ldy, epi, stream_of(s));
}

int cv3_conv1d(const float* x, int64_t cin, int64_t t_in, int64_t x_cs, int64_t x_ts, const float* w, int64_t cout,
               int64_t k, const float* bias, int64_t stride, int64_t dilation, int64_t groups, int64_t pad_l,
               int64_t pad_r, int64_t up, float* y, int64_t y_cs, int64_t y_ts, int64_t* t_out_ptr, int act,
               float act_param, const float* snake_alpha, float snake_eps, const float* residual, int64_t r_cs,
               int64_t r_ts, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(groups >= 1 && cin % groups == 0 && cout % groups == 0, CV3_EASSERT,
              "channels %lld/%lld not divisible by groups %lld", (long long)cin, (long long)cout, (long long)groups);
  CV3_REQUIRE(stride >= 1 && dilation >= 1 && up >= 1 && k >= 1 && pad_l >= 0 && pad_r >= 0, CV3_EINVAL,
              "bad conv geometry");
  const int64_t tp = t_in * up + pad_l + pad_r;
  const int64_t span = dilation * (k - 1) + 1;
  const int64_t t_out = tp >= span ? (tp - span) / stride + 1 : 0;
  if (t_out_ptr) *t_out_ptr = t_out;
  if (t_out <= 0 || !y) return CV3_OK;
  ConvParams p{};
  p.x = x;
  p.x_cs = x_cs;
  p.x_ts = x_ts;
  p.t_in = t_in;
  p.w = w;
  p.cout = cout;
  p.cin_g = cin / groups;
  p.k = k;
  p.bias = bias;
  p.groups = groups;
  p.stride = stride;
  p.dil = dilation;
  p.pad_l = pad_l;
  p.up = up;
  p.t_out = t_out;
  p.y = y;
  p.y_cs = y_cs;
  p.y_ts = y_ts;
  p.act = act;
  p.act_param = act_param;
  p.snake_alpha = snake_alpha;
  p.snake_eps = snake_eps;
  p.res = residual;
  p.r_cs = r_cs;
  p.r_ts = r_ts;
  const dim3 grid((unsigned)ceil_div(t_out, BN), (unsigned)ceil_div(cout / groups, BM), (unsigned)groups);
  hipLaunchKernelGGL(k_conv_mfma, grid, dim3(256), 0, stream_of(s), p);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_conv1d_packed(const float* x, int64_t cin, int64_t t_in, int64_t x_cs, const float* w_packed, int64_t cout,
                      int64_t k, const float* bias, int64_t dilation, int64_t pad_l, int64_t pad_r, int64_t up,
                      float* y, int64_t y_cs, int64_t y_ts, int act, float act_param, const float* snake_alpha,
                      float snake_eps, const float* residual, int64_t r_cs, int64_t r_ts, int64_t ksplit,
                      float* workspace, int64_t workspace_floats, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(dilation >= 1 && up >= 1 && k >= 1 && pad_l >= 0 && pad_r >= 0 && cin > 0 && cout > 0, CV3_EINVAL,
              "bad conv geometry");
  CV3_REQUIRE(ksplit >= 1 && ksplit <= 16 && (k * cin / FBK) % (2 * ksplit) == 0, CV3_EINVAL,
              "ksplit %lld must divide the %lld K stages into even slices", (long long)ksplit,
              (long long)(k * cin / FBK));
  CV3_REQUIRE(cin % 64 == 0, CV3_EUNSUPPORTED, "packed conv needs cin %% 64 == 0 (cin %lld)", (long long)cin);
  CV3_REQUIRE(((uintptr_t)w_packed % 16) == 0, CV3_EINVAL, "packed conv weight must be 16-byte aligned");
  const int64_t tp = t_in * up + pad_l + pad_r;
  const int64_t span = dilation * (k - 1) + 1;
  const int64_t t_out = tp >= span ? tp - span + 1 : 0;
  CV3_REQUIRE(t_in * up < (1ll << 31) && tp < (1ll << 31) && cin * k < (1ll << 31) && cout < (1ll << 31) &&
                  dilation * k < (1ll << 31),
              CV3_EINVAL, "packed conv sizes exceed 32-bit indexing");
  if (t_out <= 0) return CV3_OK;
  CV3_REQUIRE(ksplit == 1 || (workspace && workspace_floats >= ksplit * cout * t_out), CV3_EINVAL,
              "split-K conv needs a workspace of ksplit * cout * t_out floats");
  ConvFast p{};
  p.x = x;
  p.x_cs = x_cs;
  p.t_in = (int)t_in;
  p.up = (int)up;
  p.w = w_packed;
  p.cout = (int)cout;
  p.cin = (int)cin;
  p.k = (int)k;
  p.dil = (int)dilation;
  p.pad_l = (int)pad_l;
  p.t_out = (int)t_out;
  p.bias = bias;
  p.y = y;
  p.y_cs = y_cs;
  p.y_ts = y_ts;
  p.act = act;
  p.act_param = act_param;
  p.snake_alpha = snake_alpha;
  p.snake_eps = snake_eps;
  p.res = residual;
  p.r_cs = r_cs;
  p.r_ts = r_ts;
  p.part = workspace;
  p.ksplit = (int)ksplit;
  const dim3 grid((unsigned)ceil_div(t_out, 64), (unsigned)ceil_div(cout, 64), (unsigned)ksplit);
  hipLaunchKernelGGL(k_conv_fast, grid, dim3(256), 0, stream_of(s), p);
  CV3_LAUNCHED();
  if (ksplit > 1) {
    const int64_t n = cout * t_out;
    hipLaunchKernelGGL(k_conv_reduce, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 4096)), dim3(256), 0,
                       stream_of(s), p);
    CV3_LAUNCHED();
  }
  return CV3_OK;
}

// The channels-last packed conv: float32 weights (k_conv_cl_dma) or, with `planes`, their three
// bfloat16 planes [3][cout][k * cin] (k_conv_cl_x3).
static int conv_cl_packed(const float* x, int64_t t_in, int64_t cin, int64_t ldx, const float* w_packed,
                          const uint16_t* planes, bool frag, int64_t cout, int64_t k, const float* bias,
                          int64_t dilation,
                          int64_t pad_l, int64_t pad_r, int64_t up, float* y, int64_t y_ts, int64_t y_cs, int act,
                          float act_param, const float* snake_alpha, float snake_eps, const float* residual,
                          int64_t r_ts, int64_t r_cs, int64_t ksplit, float* workspace, int64_t workspace_floats,
                          cv3_stream_t s) {
  CV3_REQUIRE(dilation >= 1 && up >= 1 && k >= 1 && pad_l >= 0 && pad_r >= 0 && cin > 0 && cout > 0, CV3_EINVAL,
              "bad conv geometry");
  CV3_REQUIRE(cin % 32 == 0, CV3_EUNSUPPORTED, "channels-last packed conv needs cin %% 32 == 0 (cin %lld)",
              (long long)cin);
  const uintptr_t wa = planes ? (uintptr_t)planes : (uintptr_t)w_packed;
  CV3_REQUIRE(((uintptr_t)x % 16) == 0 && ldx % 4 == 0 && ldx >= cin && wa % 16 == 0, CV3_EINVAL,
              "channels-last packed conv needs 16-byte aligned rows");
  const int64_t stages = k * cin / 32;
  CV3_REQUIRE(ksplit >= 1 && ksplit <= 16 && stages % ksplit == 0, CV3_EINVAL,
              "ksplit %lld must divide the %lld K stages", (long long)ksplit, (long long)stages);
  CV3_REQUIRE(!planes || (stages / ksplit) % 2 == 0, CV3_EUNSUPPORTED,
              "the bfloat16-plane conv needs an even number of 32-channel stages per K slice (%lld / %lld)",
              (long long)stages, (long long)ksplit);
  const int64_t tp = t_in * up + pad_l + pad_r;
  const int64_t span = dilation * (k - 1) + 1;
  const int64_t t_out = tp >= span ? tp - span + 1 : 0;
  CV3_REQUIRE(tp < (1ll << 31) && k * cin < (1ll << 31) && dilation * k < (1ll << 31), CV3_EINVAL,
              "channels-last packed conv sizes exceed 32-bit indexing");
  if (t_out <= 0) return CV3_OK;
  CV3_REQUIRE(ksplit == 1 || (workspace && workspace_floats >= ksplit * cout * t_out), CV3_EINVAL,
              "split-K conv needs a workspace of ksplit * cout * t_out floats");
  ConvCL p{};
  p.x = x;
  p.ldx = ldx;
  p.t_in = (int)t_in;
  p.up = (int)up;
  p.cin = (int)cin;
  p.w = w_packed;
  p.cout = (int)cout;
  p.k = (int)k;
  p.dil = (int)dilation;
  p.pad_l = (int)pad_l;
  p.t_out = (int)t_out;
  p.bias = bias;
  p.y = y;
  p.y_ts = y_ts;
  p.y_cs = y_cs;
  p.act = act;
  p.act_param = act_param;
  p.snake_alpha = snake_alpha;
  p.snake_eps = snake_eps;
  p.res = residual;
  p.r_ts = r_ts;
  p.r_cs = r_cs;
  p.part = workspace;
  p.ksplit = (int)ksplit;
  const int64_t tiles_m = ceil_div(t_out, 64), tiles_n = ceil_div(cout, 64);
  CV3_REQUIRE(tiles_m * tiles_n < (1ll << 31), CV3_EINVAL, "conv too large");
  if (planes && frag)
    hipLaunchKernelGGL(k_conv_cl_x3f, dim3((unsigned)(tiles_m * tiles_n), 1, (unsigned)ksplit), dim3(256), 0,
                       stream_of(s), p, reinterpret_cast<const uint4*>(planes), x3_frag_plane(cout, k * cin) / 8,
                       (int)tiles_m);
  else if (planes)
    hipLaunchKernelGGL(k_conv_cl_x3, dim3((unsigned)(tiles_m * tiles_n), 1, (unsigned)ksplit), dim3(256), 0,
                       stream_of(s), p, planes, cout * k * cin, (int)tiles_m);
  else
    hipLaunchKernelGGL(k_conv_cl_dma, dim3((unsigned)(tiles_m * tiles_n), 1, (unsigned)ksplit), dim3(256), 0,
                       stream_of(s), p, (int)tiles_m);
  CV3_LAUNCHED();
  if (ksplit > 1) {
    const int64_t n = cout * t_out;
    hipLaunchKernelGGL(k_conv_cl_reduce, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 4096)), dim3(256), 0,
                       stream_of(s), p);
    CV3_LAUNCHED();
  }
  return CV3_OK;
}

int cv3_conv1d_cl_packed(const float* x, int64_t t_in, int64_t cin, int64_t ldx, const float* w_packed,
                         int64_t cout, int64_t k, const float* bias, int64_t dilation, int64_t pad_l, int64_t pad_r,
                         int64_t up, float* y, int64_t y_ts, int64_t y_cs, int act, float act_param,
                         const float* snake_alpha, float snake_eps, const float* residual, int64_t r_ts, int64_t r_cs,
                         int64_t ksplit, float* workspace, int64_t workspace_floats, cv3_stream_t s) {
  CV3_ALIVE();
  return conv_cl_packed(x, t_in, cin, ldx, w_packed, nullptr, false, cout, k, bias, dilation, pad_l, pad_r, up, y,
                        y_ts, y_cs,
                        act, act_param, snake_alpha, snake_eps, residual, r_ts, r_cs, ksplit, workspace,
                        workspace_floats, s);
}

int cv3_conv1d_cl_packed_x3(const float* x, int64_t t_in, int64_t cin, int64_t ldx, const uint16_t* w_planes,
                            int64_t cout, int64_t k, const float* bias, int64_t dilation, int64_t pad_l,
                            int64_t pad_r, int64_t up, float* y, int64_t y_ts, int64_t y_cs, int act, float act_param,
                            const float* snake_alpha, float snake_eps, const float* residual, int64_t r_ts,
                            int64_t r_cs, int64_t ksplit, float* workspace, int64_t workspace_floats,
                            cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(w_planes, CV3_EINVAL, "null weight planes");
  return conv_cl_packed(x, t_in, cin, ldx, nullptr, w_planes, false, cout, k, bias, dilation, pad_l, pad_r, up, y, y_ts,
                        y_cs, act, act_param, snake_alpha, snake_eps, residual, r_ts, r_cs, ksplit, workspace,
                        workspace_floats, s);
}

int cv3_conv1d_cl_packed_x3f(const float* x, int64_t t_in, int64_t cin, int64_t ldx, const uint16_t* w_frag,
                             int64_t cout, int64_t k, const float* bias, int64_t dilation, int64_t pad_l,
                             int64_t pad_r, int64_t up, float* y, int64_t y_ts, int64_t y_cs, int act,
                             float act_param, const float* snake_alpha, float snake_eps, const float* residual,
                             int64_t r_ts, int64_t r_cs, int64_t ksplit, float* workspace, int64_t workspace_floats,
                             cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(w_frag, CV3_EINVAL, "null weight fragments");
  return conv_cl_packed(x, t_in, cin, ldx, nullptr, w_frag, true, cout, k, bias, dilation, pad_l, pad_r, up, y, y_ts,
                        y_cs, act, act_param, snake_alpha, snake_eps, residual, r_ts, r_cs, ksplit, workspace,
                        workspace_floats, s);
}

int cv3_depthwise_conv1d(const float* x, int64_t c, int64_t t_in, const float* w, int64_t k, const float* bias,
                         int64_t dilation, int64_t pad_l, int64_t pad_r, float* y, int64_t* t_out_ptr,
                         cv3_stream_t s) {
  CV3_ALIVE();
  const int64_t t_out = t_in + pad_l + pad_r - dilation * (k - 1);
  if (t_out_ptr) *t_out_ptr = t_out;
  if (t_out <= 0 || !y) return CV3_OK;
  const int64_t n = c * t_out;
  hipLaunchKernelGGL(k_depthwise, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 65536)), dim3(256), 0,
                     stream_of(s), x, w, bias, y, c, t_in, k, dilation, pad_l, t_out);
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // extern "C"
