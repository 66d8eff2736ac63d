// fp32 GEMM on the CDNA4 matrix cores: C[m, n] = epi(A[m, :k] . W[n, :k]),
// both operands K-contiguous (the reference's (out, in) weight layout,
// cv3cpu/ops.py:121-123).  Used for every multi-row linear (the DiT's
// projections, cv3cpu/quant.py:165-170) and, with an int8 B operand dequantised
// on its way into LDS, for q8 weights (cv3cpu/quant.py:176-190).
//
// Tiling: a 256-thread workgroup owns a BM x BN = 64 x 64 output tile; each of
// its four waves owns a 32 x 32 quadrant computed with v_mfma_f32_32x32x2_f32
// (fp32 in, fp32 accumulate).  K advances in steps of BK = 16, staged through
// LDS with the next step's global loads held in registers meanwhile.
//
// K permutation: an MFMA step j consumes two k values per lane half (h = lane/32).
// Mapping step j, half h -> k = (j/4)*8 + h*4 + j%4 lets every lane read four
// consecutive k with one 16-byte LDS load for four consecutive MFMAs.  The
// same map is used for A and B, so the products pair correctly.
#include "common.hpp"
#include "epilogue.hpp"

using namespace cv3;

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 64, BN = 64, BK = 16, LDS_STRIDE = BK + 4;

enum { B_F32 = 0, B_Q8 = 1 };

struct GemmParams {
  const float* a;
  int64_t lda;
  const void* b;      // fp32 [n, ldb] or int8 codes [n, ldb]
  int64_t ldb;        // elements between B rows
  const void* scales; // q8 only
  int sf16;
  int64_t nb, block;
  int64_t m, n, k;
  const float* bias;
  float* c;
  int64_t ldc;
  cv3_epilogue epi;
};

template <int BK_KIND>
__device__ __forceinline__ float4 load_b(const GemmParams& p, int64_t row, int64_t kk, bool fast) {
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (row >= p.n) return v;
  if constexpr (BK_KIND == B_F32) {
    const float* src = reinterpret_cast<const float*>(p.b) + row * p.ldb + kk;
    if (fast) return *reinterpret_cast<const float4*>(src);
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = (kk + i < p.k) ? src[i] : 0.f;
    return make_float4(t[0], t[1], t[2], t[3]);
  } else {
    const int8_t* src = reinterpret_cast<const int8_t*>(p.b) + row * p.ldb + kk;
    float t[4];
    if (fast) {
      // four codes in one word share a scale because block % 4 == 0 on this path
      const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
      const int64_t si = row * p.nb + kk / p.block;
      const float s = p.sf16 ? __half2float(reinterpret_cast<const __half*>(p.scales)[si])
                             : reinterpret_cast<const float*>(p.scales)[si];
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = (float)((int32_t)(w << (24 - 8 * i)) >> 24) * s;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        t[i] = 0.f;
        if (kk + i < p.k) {
          const int64_t si = row * p.nb + (kk + i) / p.block;
          const float s = p.sf16 ? __half2float(reinterpret_cast<const __half*>(p.scales)[si])
                                 : reinterpret_cast<const float*>(p.scales)[si];
          t[i] = (float)src[i] * s;
        }
      }
    }
    return make_float4(t[0], t[1], t[2], t[3]);
  }
}

__device__ __forceinline__ float4 load_a(const GemmParams& p, int64_t row, int64_t kk, bool fast) {
  if (row >= p.m) return make_float4(0.f, 0.f, 0.f, 0.f);
  const float* src = p.a + row * p.lda + kk;
  if (fast) return *reinterpret_cast<const float4*>(src);
  float t[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) t[i] = (kk + i < p.k) ? src[i] : 0.f;
  return make_float4(t[0], t[1], t[2], t[3]);
}

template <int BK_KIND>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p, int fast_a, int fast_b) {
  __shared__ float As[2][BM * LDS_STRIDE];
  __shared__ float Bs[2][BN * LDS_STRIDE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  // global -> LDS assignment: each thread moves one float4 of A and of B per K step
  const int lrow = tid >> 2, lk = (tid & 3) * 4;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int r32 = lane & 31, h = lane >> 5;

  const int64_t ksteps = ceil_div(p.k, BK);
  const bool fa = fast_a, fb = fast_b;

  float4 ra = load_a(p, m0 + lrow, lk, fa && lk + 4 <= p.k);
  float4 rb = load_b<BK_KIND>(p, n0 + lrow, lk, fb && lk + 4 <= p.k);
  *reinterpret_cast<float4*>(&As[0][lrow * LDS_STRIDE + lk]) = ra;
  *reinterpret_cast<float4*>(&Bs[0][lrow * LDS_STRIDE + lk]) = rb;
  __syncthreads();

  f32x16 acc = {0.f};
  for (int64_t s = 0; s < ksteps; ++s) {
    const int buf = s & 1;
    const bool more = s + 1 < ksteps;
    if (more) {
      const int64_t kk = (s + 1) * BK + lk;
      ra = load_a(p, m0 + lrow, kk, fa && kk + 4 <= p.k);
      rb = load_b<BK_KIND>(p, n0 + lrow, kk, fb && kk + 4 <= p.k);
    }
    const float* as = &As[buf][(wm + r32) * LDS_STRIDE + h * 4];
    const float* bs = &Bs[buf][(wn + r32) * LDS_STRIDE + h * 4];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const float4 av = *reinterpret_cast<const float4*>(as + g * 8);
      const float4 bv = *reinterpret_cast<const float4*>(bs + g * 8);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
    }
    if (more) {
      *reinterpret_cast<float4*>(&As[buf ^ 1][lrow * LDS_STRIDE + lk]) = ra;
      *reinterpret_cast<float4*>(&Bs[buf ^ 1][lrow * LDS_STRIDE + lk]) = rb;
    }
    __syncthreads();
  }

  // accumulator layout (32x32x2 f32): reg i -> row (i/4)*8 + h*4 + i%4, col = lane%32
  const int64_t col = n0 + wn + r32;
  if (col >= p.n) return;
  const float bv = p.bias ? p.bias[col] : 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3);
    if (row < p.m) {
      float v = acc[i] + bv;
      v = apply_epilogue(p.epi, v, row, col, false);
      p.c[row * p.ldc + col] = v;
    }
  }
}

}  // namespace

namespace cv3 {

int gemm(bool q8, const float* a, int64_t m, int64_t k, int64_t lda, const void* b, int64_t ldb, const void* scales,
         bool sf16, int64_t nb, int64_t block, int64_t n, const float* bias, float* c, int64_t ldc,
         const cv3_epilogue* epi, hipStream_t st) {
  GemmParams p{};
  p.a = a;
  p.lda = lda;
  p.b = b;
  p.ldb = ldb;
  p.scales = scales;
  p.sf16 = sf16;
  p.nb = nb;
  p.block = block;
  p.m = m;
  p.n = n;
  p.k = k;
  p.bias = bias;
  p.c = c;
  p.ldc = ldc;
  p.epi = epi ? *epi : cv3_epilogue{};
  const int fast_a = ((uintptr_t)a % 16 == 0) && (lda % 4 == 0);
  const int fast_b = q8 ? (((uintptr_t)b % 4 == 0) && (ldb % 4 == 0) && (block % 4 == 0))
                        : (((uintptr_t)b % 16 == 0) && (ldb % 4 == 0));
  const dim3 grid((unsigned)ceil_div(n, BN), (unsigned)ceil_div(m, BM));
  if (q8)
    hipLaunchKernelGGL(k_gemm<B_Q8>, grid, dim3(256), 0, st, p, fast_a, fast_b);
  else
    hipLaunchKernelGGL(k_gemm<B_F32>, grid, dim3(256), 0, st, p, fast_a, fast_b);
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // namespace cv3
