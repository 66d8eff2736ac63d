// fp32 GEMM on the CDNA4 matrix cores: C[m, n] = epi(A[m, :k] . W[n, :k]),
// both operands K-contiguous (the reference's (out, in) weight layout,
// cv3cpu/ops.py:121-123).  Used for every multi-row linear (the DiT's
// projections, cv3cpu/quant.py:165-170) and, with a quantised B operand
// dequantised on its way into LDS, for q8 and q4 weights (cv3cpu/quant.py:176-204):
// each code becomes the float32 (code * scale) the reference's dequantisation
// forms (quant.py:70-86), so only the summation order differs from it.
//
// Tiling: a 256-thread workgroup owns a BM x BN = 64 x 64 output tile; each of
// its four waves owns a 32 x 32 quadrant computed with v_mfma_f32_32x32x2_f32
// (fp32 in, fp32 accumulate).  K advances in stages of BK = 32 through a
// double-buffered LDS tile, and the global loads run two stages ahead in
// registers (ping-pong sets r0 / r1), so each load has two stages of MFMA work
// (32 MFMAs per wave) to hide behind.
//
// K permutation: within a stage, group g (8 k values) and lane half h = lane/32
// give MFMA j the k value g*8 + h*4 + j, so every lane reads four consecutive k
// with one 16-byte LDS load for four consecutive MFMAs.  A and B use the same
// map, so the products pair correctly.
//
// Workgroup -> tile mapping is XCD-aware: workgroups are dispatched round-robin
// over the 8 XCDs, so linear id L runs on XCD L % 8; tile t = (L % 8) * (T / 8) +
// L / 8 with M-tiles fastest gives each XCD whole columns of N-tiles, and each
// weight tile is fetched into one XCD's L2 only.  When the activation A is larger
// than an XCD's 4 MB L2 (the 30 s utterance: 3000 x 1024 floats), walking a column
// would stream all of A again for every column; the register-staged kernel then
// walks groups of 8 M-tiles across all N-tiles instead (group_m = 8), so the tiles
// in flight share A rows and W columns (5-6 % on those GEMMs).
#include "bf16x3.hpp"
#include "common.hpp"
#include "epilogue.hpp"

using namespace cv3;

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 64, BN = 64, BK = 32, LDS_STRIDE = BK + 4;

struct Stage {
  float4 a0, a1, b0, b1;
};

enum { B_F32 = 0, B_Q8 = 1, B_Q4 = 2 };

// q4 (cv3cpu/quant.py:70-86): blocks of 32 codes in 16 bytes, byte j holding code j in its
// low nibble and code j + 16 in its high nibble, +8 biased, one float16 scale per block.
// A GEMM stage (BK = 32, k0 % 32 == 0) is one block, so a thread's four consecutive k
// (lk % 4 == 0) are four nibbles of one aligned 32-bit word, all low (lk < 16) or all high.
__device__ __forceinline__ float4 q4_word(uint32_t w, int lk, float s) {
  const uint32_t v = lk >= 16 ? (w >> 4) : w;
  return make_float4((float)((int)(v & 0xF) - 8) * s, (float)((int)((v >> 8) & 0xF) - 8) * s,
                     (float)((int)((v >> 16) & 0xF) - 8) * s, (float)((int)((v >> 24) & 0xF) - 8) * s);
}

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
  // channels-last grouped temporal conv as an implicit GEMM (A_CONV): rows are
  // (batch, time) with conv_t rows per batch, K = (tap, channel-in-group)
  int conv_t, conv_cg, conv_pad;
};

enum { A_ROWS = 0, A_CONV = 1 };

// A operand of the FAST kernel.  A_ROWS: base = a + row * lda + lk.
// A_CONV: base = x + batch * conv_t * lda + group channel base + lk, t_row = the
// row's time index; k = tap * conv_cg + channel, so x[t_row + tap - pad, channel]
// with zeros outside [0, conv_t) (loaded from the row itself and replaced by a select).
template <int AMODE>
__device__ __forceinline__ float4 load_a_fast(const GemmParams& p, const float* base, int t_row, int64_t koff) {
  if constexpr (AMODE == A_ROWS) {
    return *reinterpret_cast<const float4*>(base + koff);
  } else {
    const int kk = (int)koff;
    const int tap = kk / p.conv_cg, c = kk - tap * p.conv_cg;
    const int tt = t_row + tap - p.conv_pad;
    const bool ok = (unsigned)tt < (unsigned)p.conv_t;
    const float4 v = *reinterpret_cast<const float4*>(base + (int64_t)(ok ? tt : t_row) * p.lda + c);
    return ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

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
  } else if constexpr (BK_KIND == B_Q4) {
    // kk = k0 + lk: block kk / 32, byte (kk % 16) of it, nibble half by kk % 32 >= 16
    const uint8_t* blk = reinterpret_cast<const uint8_t*>(p.b) + row * p.ldb + (kk >> 5) * 16;
    const int lk = (int)(kk & 31);
    const float s = __half2float(reinterpret_cast<const __half*>(p.scales)[row * p.nb + (kk >> 5)]);
    if (fast) return q4_word(*reinterpret_cast<const uint32_t*>(blk + (lk & 15)), lk, s);
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lk + i;  // within the block (lk % 4 == 0, so c < 32)
      const uint8_t byte = blk[c & 15];
      t[i] = (kk + i < p.k) ? (float)((int)((c >= 16 ? byte >> 4 : byte) & 0xF) - 8) * s : 0.f;
    }
    return make_float4(t[0], t[1], t[2], t[3]);
  } else {
    const int8_t* src = reinterpret_cast<const int8_t*>(p.b) + row * p.ldb + kk;
    float t[4];
    if (fast) {
      // four codes in one word share a scale because block % 4 == 0 on this path
      const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
      const int64_t si = row * p.nb + (int64_t)((uint32_t)kk / (uint32_t)p.block);
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

// Branch-free loads for the FAST kernel: K % BK == 0, 16-byte aligned rows; rows past
// M / N are clamped to the last row (their results are never stored), so the
// loads carry no predicates and the compiler can count them (vmcnt) across the
// two-stage pipeline.
// B row pointer of the FAST kernels: thread's row `row`, k offset lk folded in.
struct BRow {
  const void* codes;   // float* or int8_t* at (row, lk)
  const void* scales;  // q8: the row's scales
  int lk;
};

template <int BK_KIND>
__device__ __forceinline__ BRow b_row(const GemmParams& p, int64_t row, int lk) {
  BRow r;
  if constexpr (BK_KIND == B_F32) {
    r.codes = reinterpret_cast<const float*>(p.b) + row * p.ldb + lk;
    r.scales = nullptr;
  } else if constexpr (BK_KIND == B_Q4) {
    r.codes = reinterpret_cast<const uint8_t*>(p.b) + row * p.ldb + (lk & 15);
    r.scales = reinterpret_cast<const __half*>(p.scales) + row * p.nb;
  } else {
    r.codes = reinterpret_cast<const int8_t*>(p.b) + row * p.ldb + lk;
    r.scales = p.sf16 ? (const void*)(reinterpret_cast<const __half*>(p.scales) + row * p.nb)
                      : (const void*)(reinterpret_cast<const float*>(p.scales) + row * p.nb);
  }
  r.lk = lk;
  return r;
}

template <int BK_KIND>
__device__ __forceinline__ float4 load_b_fast(const GemmParams& p, const BRow& r, int64_t koff) {
  if constexpr (BK_KIND == B_F32) {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(r.codes) + koff);
  } else if constexpr (BK_KIND == B_Q4) {
    // koff % 32 == 0: block koff / 32 starts at byte koff / 2
    const uint32_t w = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(r.codes) + (koff >> 1));
    return q4_word(w, r.lk, __half2float(reinterpret_cast<const __half*>(r.scales)[koff >> 5]));
  } else {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const int8_t*>(r.codes) + koff);
    const uint32_t si = ((uint32_t)koff + (uint32_t)r.lk) / (uint32_t)p.block;
    const float s = p.sf16 ? __half2float(reinterpret_cast<const __half*>(r.scales)[si])
                           : reinterpret_cast<const float*>(r.scales)[si];
    return make_float4((float)((int32_t)(w << 24) >> 24) * s, (float)((int32_t)(w << 16) >> 24) * s,
                       (float)((int32_t)(w << 8) >> 24) * s, (float)((int32_t)w >> 24) * s);
  }
}

// General-kernel loads: thread -> rows lrow and lrow + 32 of the A and B tiles,
// 4 consecutive k at lk, every element guarded.
template <int BK_KIND>
__device__ __forceinline__ void load_stage(const GemmParams& p, int64_t m0, int64_t n0, int64_t k0, int lrow, int lk,
                                           bool fa, bool fb, Stage& st) {
  const int64_t kk = k0 + lk;
  const bool kfull = kk + 4 <= p.k;
  st.a0 = load_a(p, m0 + lrow, kk, fa && kfull);
  st.a1 = load_a(p, m0 + lrow + 32, kk, fa && kfull);
  st.b0 = load_b<BK_KIND>(p, n0 + lrow, kk, fb && kfull);
  st.b1 = load_b<BK_KIND>(p, n0 + lrow + 32, kk, fb && kfull);
}

__device__ __forceinline__ void store_stage(float* As, float* Bs, int lrow, int lk, const Stage& st) {
  *reinterpret_cast<float4*>(&As[lrow * LDS_STRIDE + lk]) = st.a0;
  *reinterpret_cast<float4*>(&As[(lrow + 32) * LDS_STRIDE + lk]) = st.a1;
  *reinterpret_cast<float4*>(&Bs[lrow * LDS_STRIDE + lk]) = st.b0;
  *reinterpret_cast<float4*>(&Bs[(lrow + 32) * LDS_STRIDE + lk]) = st.b1;
}

__device__ __forceinline__ void mma_stage(const float* As, const float* Bs, int wm, int wn, int r32, int h, f32x16& acc) {
  const float* as = &As[(wm + r32) * LDS_STRIDE + h * 4];
  const float* bs = &Bs[(wn + r32) * LDS_STRIDE + h * 4];
#pragma unroll
  for (int g = 0; g < BK / 8; ++g) {
    const float4 av = *reinterpret_cast<const float4*>(as + g * 8);
    const float4 bv = *reinterpret_cast<const float4*>(bs + g * 8);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
  }
}

// Epilogue of one wave's 32 x 32 accumulator tile (32x32x2 f32 layout: reg i -> row
// r0 + (i/4)*8 + h*4 + i%4, column col = lane's column).  Every operand the epilogue
// reads (rotary table, gate, residual) is loaded for all 16 registers before the first
// store: C may be the residual itself (in-place residual adds), so a load issued after
// a store to C would have to wait for it, one memory round trip per register.  Each
// element is read and written by the same lane, so the early loads are exact.
//
// DiT partial rotary (dit.py:40-54): columns c < rope_limit with c % rope_period <
// rope_width are interleaved pairs (2i, 2i+1) -> (a cos - b sin, b cos + a sin), table
// row = row % rope_rows; the pair partner of column c is held by lane ^ 1.
__device__ __forceinline__ void store_tile(const GemmParams& p, const f32x16& acc, int64_t r0, int h, int64_t col) {
  const cv3_epilogue& e = p.epi;
  const bool cin = col < p.n;
  const int64_t cc = cin ? col : p.n - 1;
  const float bv = p.bias ? p.bias[cc] : 0.f;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = acc[i] + bv;
  if (e.rope_cos) {  // uniform branch, shuffles inside
    // 32-bit index arithmetic (the host bounds the table and the row count): one modulo for
    // the lane's first row, then row i % rope_rows = base + offset_i, less rope_rows once
    // when rope_rows exceeds the 27-row spread of the 16 registers (else a modulo each)
    const uint32_t rr = (uint32_t)e.rope_rows, rw = (uint32_t)e.rope_width;
    const uint32_t cp = (uint32_t)col % (uint32_t)e.rope_period;
    const bool rot = col < e.rope_limit && cp < rw;
    // most waves hold no rotated column (the DiT rotates 2 x 64 of 3072): skip the table
    // loads and shuffles there (a wave-uniform branch, so the shuffles stay whole-wave)
    if (__any(rot)) {
      const uint32_t first = (uint32_t)(r0 + h * 4) % rr;
      float cs[16], sn[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t off = (uint32_t)((i >> 2) * 8 + (i & 3));
        uint32_t tr = first + off;
        tr = rr > 27u ? (tr >= rr ? tr - rr : tr) : tr % rr;
        const uint32_t ti = tr * rw + (rot ? cp : 0u);
        cs[i] = e.rope_cos[ti];
        sn[i] = e.rope_sin[ti];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float other = __shfl_xor(v[i], 1, 64);
        if (rot) v[i] = (col & 1) ? v[i] * cs[i] + other * sn[i] : v[i] * cs[i] + (-other) * sn[i];
      }
    }
  }
  float g[16], res[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = min(r0 + (i >> 2) * 8 + h * 4 + (i & 3), p.m - 1);
    g[i] = e.gate ? e.gate[(e.rows_per_gate > 1 ? row / e.rows_per_gate : row) * e.gate_stride + cc] : 1.f;
    res[i] = e.residual ? e.residual[row * e.ld_res + cc] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = r0 + (i >> 2) * 8 + h * 4 + (i & 3);
    float y = apply_act(e.act, v[i], e.act_param);
    if (e.gate) y = g[i] * y;
    if (e.residual) y = res[i] + y;
    if (row < p.m && cin) p.c[row * p.ldc + col] = y;
  }
}

// The GEMM kernel: 4 waves, 64 x 64 tile.  FAST (K % 64 == 0, aligned rows):
// branch-free loads two stages ahead; otherwise one stage of guarded prefetch.
template <int BK_KIND, bool FAST, int AMODE = A_ROWS>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p, int fast_a, int fast_b, int tiles_m, int group_m) {
  __shared__ float As[2][BM * LDS_STRIDE];
  __shared__ float Bs[2][BN * LDS_STRIDE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = gridDim.x, L = blockIdx.x;
  const int t = (T % 8 == 0) ? (L % 8) * (T / 8) + L / 8 : L;
  int tm, tn;
  if (group_m > 0) {  // groups of group_m M-tiles, M fastest within a group, across all N-tiles
    const int tiles_n = T / tiles_m, per_group = group_m * tiles_n, first = (t / per_group) * group_m;
    const int rows = min(tiles_m - first, group_m), r = t % per_group;
    tm = first + r % rows;
    tn = r / rows;
  } else {
    tm = t % tiles_m;
    tn = t / tiles_m;
  }
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int lrow = tid >> 3, lk = (tid & 7) * 4;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int r32 = lane & 31, h = lane >> 5;
  const bool fa = fast_a, fb = fast_b;

  const int64_t S = ceil_div(p.k, BK);
  f32x16 acc = {0.f};
  if constexpr (FAST) {
    // S even and >= 2 (K % 64 == 0): straight-line ping-pong between two register
    // sets (x0 / x1: A rows lrow, lrow + 32 and B rows lrow, lrow + 32), no predicates
    const int64_t ra0 = min(m0 + lrow, p.m - 1), ra1 = min(m0 + lrow + 32, p.m - 1);
    const BRow rb0 = b_row<BK_KIND>(p, min(n0 + lrow, p.n - 1), lk);
    const BRow rb1 = b_row<BK_KIND>(p, min(n0 + lrow + 32, p.n - 1), lk);
    const float* pa0;
    const float* pa1;
    int t0 = 0, t1 = 0;
    if constexpr (AMODE == A_ROWS) {
      pa0 = p.a + ra0 * p.lda + lk;
      pa1 = p.a + ra1 * p.lda + lk;
    } else {
      // output channels of this N-tile form one group: channel base = group * conv_cg
      const int64_t cbase = (n0 / BN) * p.conv_cg;
      const int b0 = (int)ra0 / p.conv_t, b1 = (int)ra1 / p.conv_t;
      t0 = (int)ra0 - b0 * p.conv_t;
      t1 = (int)ra1 - b1 * p.conv_t;
      pa0 = p.a + (int64_t)b0 * p.conv_t * p.lda + cbase + lk;
      pa1 = p.a + (int64_t)b1 * p.conv_t * p.lda + cbase + lk;
    }
    float4 xa0, xa1, xb0, xb1, ya0, ya1, yb0, yb1;
#define CV3_LOAD(A0, A1, B0, B1, KOFF)                                   \
  A0 = load_a_fast<AMODE>(p, pa0, t0, (KOFF));                           \
  A1 = load_a_fast<AMODE>(p, pa1, t1, (KOFF));                           \
  B0 = load_b_fast<BK_KIND>(p, rb0, (KOFF));                             \
  B1 = load_b_fast<BK_KIND>(p, rb1, (KOFF));
#define CV3_STORE(BUF, A0, A1, B0, B1)                                               \
  *reinterpret_cast<float4*>(&As[BUF][lrow * LDS_STRIDE + lk]) = A0;                 \
  *reinterpret_cast<float4*>(&As[BUF][(lrow + 32) * LDS_STRIDE + lk]) = A1;          \
  *reinterpret_cast<float4*>(&Bs[BUF][lrow * LDS_STRIDE + lk]) = B0;                 \
  *reinterpret_cast<float4*>(&Bs[BUF][(lrow + 32) * LDS_STRIDE + lk]) = B1;
    CV3_LOAD(xa0, xa1, xb0, xb1, 0)
    CV3_LOAD(ya0, ya1, yb0, yb1, BK)
    CV3_STORE(0, xa0, xa1, xb0, xb1)
    __syncthreads();
    for (int64_t s = 0; s + 2 < S; s += 2) {
      // LDS[0] = stage s, y = stage s + 1 in flight
      CV3_LOAD(xa0, xa1, xb0, xb1, (s + 2) * BK)
      __builtin_amdgcn_sched_barrier(0);  // issue the loads before anything below
      mma_stage(As[0], Bs[0], wm, wn, r32, h, acc);
      CV3_STORE(1, ya0, ya1, yb0, yb1)
      __syncthreads();
      // LDS[1] = stage s + 1, x = stage s + 2 in flight
      CV3_LOAD(ya0, ya1, yb0, yb1, (s + 3) * BK)
      __builtin_amdgcn_sched_barrier(0);
      mma_stage(As[1], Bs[1], wm, wn, r32, h, acc);
      CV3_STORE(0, xa0, xa1, xb0, xb1)
      __syncthreads();
    }
    mma_stage(As[0], Bs[0], wm, wn, r32, h, acc);
    CV3_STORE(1, ya0, ya1, yb0, yb1)
    __syncthreads();
    mma_stage(As[1], Bs[1], wm, wn, r32, h, acc);
#undef CV3_LOAD
#undef CV3_STORE
  } else {
    // ragged K / unaligned rows: one stage of register prefetch, guarded loads
    Stage r0;
    load_stage<BK_KIND>(p, m0, n0, 0, lrow, lk, fa, fb, r0);
    store_stage(As[0], Bs[0], lrow, lk, r0);
    __syncthreads();
    for (int64_t s = 0; s < S; ++s) {
      const int buf = s & 1;
      if (s + 1 < S) load_stage<BK_KIND>(p, m0, n0, (s + 1) * BK, lrow, lk, fa, fb, r0);
      mma_stage(As[buf], Bs[buf], wm, wn, r32, h, acc);
      if (s + 1 < S) store_stage(As[buf ^ 1], Bs[buf ^ 1], lrow, lk, r0);
      __syncthreads();
    }
  }

  store_tile(p, acc, m0 + wm, h, n0 + wn + r32);
}



// Half of a stage's MFMAs: k groups 2*kh and 2*kh + 1 of the 4 in a BK = 32 stage.
__device__ __forceinline__ void mma_half(const float* As, const float* Bs, int wm, int wn, int r32, int h, int kh,
                                         f32x16& acc) {
  const float* as = &As[(wm + r32) * LDS_STRIDE + h * 4 + kh * 16];
  const float* bs = &Bs[(wn + r32) * LDS_STRIDE + h * 4 + kh * 16];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const float4 av = *reinterpret_cast<const float4*>(as + g * 8);
    const float4 bv = *reinterpret_cast<const float4*>(bs + g * 8);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
  }
}

// The FAST kernel with 8 waves, for grids of at most one workgroup per CU (e.g.
// [1000, 1024] outputs): waves q and q + 4 share output quadrant q and split each
// stage's K between them (k groups 0-1 / 2-3), so two waves per SIMD keep the
// matrix core busy while the other waits on LDS or the barrier.  The halves meet
// in LDS at the end.  One A and one B float4 per thread per stage.
template <int BK_KIND, int AMODE>
__global__ __launch_bounds__(512) void k_gemm8(GemmParams p, int tiles_m) {
  __shared__ float As[2][BM * LDS_STRIDE];
  __shared__ float Bs[2][BN * LDS_STRIDE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = gridDim.x, L = blockIdx.x;
  const int t = (T % 8 == 0) ? (L % 8) * (T / 8) + L / 8 : L;
  const int64_t m0 = (int64_t)(t % tiles_m) * BM, n0 = (int64_t)(t / tiles_m) * BN;
  const int lrow = tid >> 3, lk = (tid & 7) * 4;
  const int quad = wave & 3, kh = wave >> 2;
  const int wm = (quad >> 1) * 32, wn = (quad & 1) * 32;
  const int r32 = lane & 31, h = lane >> 5;
  const int64_t S = p.k / BK;  // even, >= 2
  const int64_t ra = min(m0 + lrow, p.m - 1);
  const BRow rb = b_row<BK_KIND>(p, min(n0 + lrow, p.n - 1), lk);
  const float* pa;
  int t0 = 0;
  if constexpr (AMODE == A_ROWS) {
    pa = p.a + ra * p.lda + lk;
  } else {
    const int64_t cbase = (n0 / BN) * p.conv_cg;
    const int b0 = (int)ra / p.conv_t;
    t0 = (int)ra - b0 * p.conv_t;
    pa = p.a + (int64_t)b0 * p.conv_t * p.lda + cbase + lk;
  }
  f32x16 acc = {0.f};
  float4 xa, xb, ya, yb;
#define CV3_LOAD8(A, B, KOFF)                  \
  A = load_a_fast<AMODE>(p, pa, t0, (KOFF));   \
  B = load_b_fast<BK_KIND>(p, rb, (KOFF));
#define CV3_STORE8(BUF, A, B)                                          \
  *reinterpret_cast<float4*>(&As[BUF][lrow * LDS_STRIDE + lk]) = A;    \
  *reinterpret_cast<float4*>(&Bs[BUF][lrow * LDS_STRIDE + lk]) = B;
  CV3_LOAD8(xa, xb, 0)
  CV3_LOAD8(ya, yb, BK)
  CV3_STORE8(0, xa, xb)
  __syncthreads();
  for (int64_t s = 0; s + 2 < S; s += 2) {
    CV3_LOAD8(xa, xb, (s + 2) * BK)
    __builtin_amdgcn_sched_barrier(0);
    mma_half(As[0], Bs[0], wm, wn, r32, h, kh, acc);
    CV3_STORE8(1, ya, yb)
    __syncthreads();
    CV3_LOAD8(ya, yb, (s + 3) * BK)
    __builtin_amdgcn_sched_barrier(0);
    mma_half(As[1], Bs[1], wm, wn, r32, h, kh, acc);
    CV3_STORE8(0, xa, xb)
    __syncthreads();
  }
  mma_half(As[0], Bs[0], wm, wn, r32, h, kh, acc);
  CV3_STORE8(1, ya, yb)
  __syncthreads();
  mma_half(As[1], Bs[1], wm, wn, r32, h, kh, acc);
#undef CV3_LOAD8
#undef CV3_STORE8
  // the K halves meet: waves 4..7 park their quadrant in LDS, waves 0..3 add it
  __syncthreads();
  float* red = &As[0][0];  // 4 quadrants x 16 regs x 64 lanes = 4096 floats
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) red[(quad * 16 + i) * 64 + lane] = acc[i];
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] += red[(quad * 16 + i) * 64 + lane];
  store_tile(p, acc, m0 + wm, h, n0 + wn + r32);
}

// fp32 GEMM fed by global -> LDS DMA (global_load_lds_dwordx4): no register
// staging, so the ring holds NST stages of BK = 32 and NST - 1 of them are in
// flight while the waves run MFMAs on the oldest.  Each stage is its own LDS
// array, so the compiler can tell a DMA into one stage from the MFMA reads of
// another and leaves the waiting to the explicit vmcnt below.
//
// A DMA writes 64 lanes x 16 B contiguously; lane l of a wave's load covers tile
// row r = base + l / 8 and slot l % 8, and fetches the row's 16-byte chunk
// (l % 8) ^ sw(r) with sw(r) = (r / 2) % 8.  Chunk c of row r therefore sits at
// r * 32 + ((c ^ sw(r)) * 4) floats.  A 16-byte read is served 16 lanes at a time from
// a 256-byte bank window, which holds two 128-byte rows: rows r and r + 1 fall in its
// two halves and (r / 2) % 8 differs across the 8 row pairs of 16 consecutive rows, so
// the 16 rows a read touches hit 16 distinct 16-byte slots.  (Swizzling by r % 8 gave
// rows r and r + 8 the same slot: half the LDS cycles were bank-conflict stalls.)
//
// Per step: wait until this wave's DMA of the current stage has landed (vmcnt:
// loads complete in order), barrier (every wave's DMA has landed and every wave
// is done with the previous stage), issue the stage NST - 1 ahead into the
// buffer the previous stage used, run the MFMAs.  sched_barrier pins that
// order against the scheduler; the barrier carries no fence, which would wait
// for every outstanding DMA.
constexpr int DMA_NST = 3;
#define CV3_VMCNT(n) (((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

struct DmaSrc {
  const float* a0;
  const float* a1;
  const float* b0;
  const float* b1;
};

__device__ __forceinline__ void dma_stage(const DmaSrc& s, int64_t koff, float* as, float* bs, int w) {
  __builtin_amdgcn_global_load_lds(s.a0 + koff, as + (w * 16) * BK, 16, 0, 0);
  __builtin_amdgcn_global_load_lds(s.a1 + koff, as + (w * 16 + 8) * BK, 16, 0, 0);
  __builtin_amdgcn_global_load_lds(s.b0 + koff, bs + (w * 16) * BK, 16, 0, 0);
  __builtin_amdgcn_global_load_lds(s.b1 + koff, bs + (w * 16 + 8) * BK, 16, 0, 0);
}

__device__ __forceinline__ void mma_swz(const float* as, const float* bs, int arow, int brow, int sw, int h,
                                        f32x16& acc) {
#pragma unroll
  for (int g = 0; g < BK / 8; ++g) {
    const int c = ((2 * g + h) ^ sw) * 4;
    const float4 av = *reinterpret_cast<const float4*>(as + arow + c);
    const float4 bv = *reinterpret_cast<const float4*>(bs + brow + c);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
  }
}

// fp32 A rows and fp32 B rows, 16-byte aligned, K % 32 == 0.
__global__ __launch_bounds__(256) void k_gemm_dma(GemmParams p, int tiles_m) {
  static_assert(DMA_NST == 3, "the step sequence below is written for a ring of three stages");
  __shared__ float A0[BM * BK], A1[BM * BK], A2[BM * BK];
  __shared__ float B0[BN * BK], B1[BN * BK], B2[BN * BK];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int T = gridDim.x, L = blockIdx.x;
  const int t = (T % 8 == 0) ? (L % 8) * (T / 8) + L / 8 : L;
  const int64_t m0 = (int64_t)(t % tiles_m) * BM, n0 = (int64_t)(t / tiles_m) * BN;
  // rows w*16 + lr (sw = lr / 2) and w*16 + 8 + lr (sw = 4 + lr / 2: the chunk index ^ 4)
  const int lr = lane >> 3, lc = ((lane & 7) ^ (lr >> 1)) * 4, lc8 = lc ^ 16;
  const float* b = reinterpret_cast<const float*>(p.b);
  DmaSrc src;
  src.a0 = p.a + min(m0 + w * 16 + lr, p.m - 1) * p.lda + lc;
  src.a1 = p.a + min(m0 + w * 16 + 8 + lr, p.m - 1) * p.lda + lc8;
  src.b0 = b + min(n0 + w * 16 + lr, p.n - 1) * p.ldb + lc;
  src.b1 = b + min(n0 + w * 16 + 8 + lr, p.n - 1) * p.ldb + lc8;
  const int wm = (w >> 1) * 32, wn = (w & 1) * 32;
  const int r32 = lane & 31, h = lane >> 5, sw = (r32 >> 1) & 7;
  const int arow = (wm + r32) * BK, brow = (wn + r32) * BK;
  const int64_t S = p.k / BK;
  f32x16 acc = {0.f};
  dma_stage(src, 0, A0, B0, w);
  dma_stage(src, min((int64_t)1, S - 1) * BK, A1, B1, w);
#define CV3_DMA_STEP(AN, BN_, AC, BC, ST)                           \
  __builtin_amdgcn_sched_barrier(0);                                \
  __builtin_amdgcn_s_waitcnt(CV3_VMCNT(4 * (DMA_NST - 2)));         \
  __builtin_amdgcn_s_barrier();                                     \
  __builtin_amdgcn_sched_barrier(0);                                \
  dma_stage(src, min((ST) + DMA_NST - 1, S - 1) * BK, AN, BN_, w);  \
  __builtin_amdgcn_sched_barrier(0);                                \
  mma_swz(AC, BC, arow, brow, sw, h, acc);
  int64_t st = 0;
  for (; st + 3 <= S; st += 3) {
    CV3_DMA_STEP(A2, B2, A0, B0, st)
    CV3_DMA_STEP(A0, B0, A1, B1, st + 1)
    CV3_DMA_STEP(A1, B1, A2, B2, st + 2)
  }
  if (st < S) {
    CV3_DMA_STEP(A2, B2, A0, B0, st)
    if (st + 1 < S) { CV3_DMA_STEP(A0, B0, A1, B1, st + 1) }
  }
#undef CV3_DMA_STEP
  // no DMA may still be writing this workgroup's LDS when it ends
  __builtin_amdgcn_s_waitcnt(CV3_VMCNT(0));
  store_tile(p, acc, m0 + wm, h, n0 + wn + r32);
}

// ---- split-bfloat16 GEMM: float32 products on the bfloat16 matrix cores ----
// C = epi(A . B^T) for float32 A and B, with B given as its three bfloat16 planes
// (hi, mid, lo: B = hi + mid + lo to all 24 bits, bf16x3.hpp) and A split into its
// planes on the way into LDS.  Each 32 x 32 x 16 k-step runs six
// v_mfma_f32_32x32x16_bf16: hi.hi into one accumulator, hi.mid, mid.hi, hi.lo,
// mid.mid and lo.hi into a second, added at the end, so the big term does not absorb
// the small ones' low bits on every step.  Per k-step that is 6 x 16K = 96K multiply-adds
// of bfloat16 at 16x the float32 rate: 2.7x the float32 MFMA's throughput, with errors
// against float64 no larger than its own (measured over K = 1024..4096).
//
// Tiling as the float32 kernel: 64 x 64 tile, four waves of 32 x 32, stages of 32 k
// double-buffered in LDS, global loads two stages ahead in registers.  LDS holds each
// plane as 64 rows x four 16-byte chunks (8 k); chunk c of row r sits in slot
// r * 4 + (c ^ (r / 4) % 4), so the 16 lanes of a 16-byte read (rows r .. r + 15, one
// chunk) cover all 16 slots of a 256-byte bank window.
constexpr int XBK = 32;

struct XStage {
  float4 a0, a1;   // A: row lr, k = 8 * lc .. + 7 of the stage
  uint4 b0, b1, b2;  // B planes hi, mid, lo: row lr, the same 8 k
};

__device__ __forceinline__ int xslot(int row, int chunk) { return row * 4 + (chunk ^ ((row >> 2) & 3)); }

// K % 64 == 0; A rows 16-byte aligned (lda % 4 == 0); plane rows 16-byte aligned.
// Tile of workgroup L: the remap hands each XCD (workgroup L runs on XCD L % 8) a contiguous
// range of tiles, walked in groups of gm row tiles across all column tiles.  gm = tiles_m walks
// column by column (B streamed once, A re-read from L2: the DiT's plane GEMMs, whose weights are
// the larger operand); a small gm keeps a few row tiles of A in L2 while the columns stream past
// (the 30 s q8 GEMMs, whose float32 activations outweigh the int8 codes).
__device__ __forceinline__ void tile_xcd(int L, int T, int tiles_m, int tiles_n, int gm, int64_t& m0, int64_t& n0) {
  const int t = (T % 8 == 0) ? (L % 8) * (T / 8) + L / 8 : L;
  const int per = gm * tiles_n, g = t / per, r = t - g * per;
  const int first = g * gm, gh = min(gm, tiles_m - first);
  m0 = (int64_t)(first + r % gh) * BM;
  n0 = (int64_t)(r / gh) * BN;
}

__global__ __launch_bounds__(256) void k_gemm_x3(GemmParams p, const uint16_t* pb, int64_t ldp, int64_t pstride,
                                                 int tiles_m, int tiles_n, int gm) {
  __shared__ uint4 sA[2][3][BM * 4];
  __shared__ uint4 sB[2][3][BN * 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int64_t m0, n0;
  tile_xcd(blockIdx.x, gridDim.x, tiles_m, tiles_n, gm, m0, n0);
  const int lr = tid >> 2, lc = tid & 3;
  const float* pa = p.a + min(m0 + lr, p.m - 1) * p.lda + lc * 8;
  const uint16_t* pbr = pb + min(n0 + lr, p.n - 1) * ldp + lc * 8;
  const int wslot = xslot(lr, lc);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32, r32 = lane & 31, h = lane >> 5;
  const int ar = wm + r32, br = wn + r32, asw = (ar >> 2) & 3, bsw = (br >> 2) & 3;
  const int64_t S = p.k / XBK;
  f32x16 big = {0.f}, small = {0.f};

  auto load = [&](XStage& x, int64_t k0) {
    x.a0 = *reinterpret_cast<const float4*>(pa + k0);
    x.a1 = *reinterpret_cast<const float4*>(pa + k0 + 4);
    x.b0 = *reinterpret_cast<const uint4*>(pbr + k0);
    x.b1 = *reinterpret_cast<const uint4*>(pbr + pstride + k0);
    x.b2 = *reinterpret_cast<const uint4*>(pbr + 2 * pstride + k0);
  };
  auto store = [&](int buf, const XStage& x) {
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
    for (int ks = 0; ks < XBK / 16; ++ks) {
      const int c = ks * 2 + h;
      const int sa = ar * 4 + (c ^ asw), sb = br * 4 + (c ^ bsw);
      const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, sA[buf][0][sa]);
      const bf16x8_t am = __builtin_bit_cast(bf16x8_t, sA[buf][1][sa]);
      const bf16x8_t al = __builtin_bit_cast(bf16x8_t, sA[buf][2][sa]);
      const bf16x8_t bh = __builtin_bit_cast(bf16x8_t, sB[buf][0][sb]);
      const bf16x8_t bm = __builtin_bit_cast(bf16x8_t, sB[buf][1][sb]);
      const bf16x8_t bl = __builtin_bit_cast(bf16x8_t, sB[buf][2][sb]);
      big = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, big, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bm, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bh, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bm, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, small, 0, 0, 0);
    }
  };

  // S even and >= 2: ping-pong between register stages x and y, as the float32 kernel
  XStage x, y;
  load(x, 0);
  load(y, XBK);
  store(0, x);
  __syncthreads();
  for (int64_t s = 0; s + 2 < S; s += 2) {
    load(x, (s + 2) * XBK);
    __builtin_amdgcn_sched_barrier(0);
    mma(0);
    store(1, y);
    __syncthreads();
    load(y, (s + 3) * XBK);
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
  store_tile(p, acc, m0 + wm, h, n0 + wn + r32);
}

// The same GEMM with B's planes packed once in MFMA fragment order (k_split_x3_frag):
// frag[p][nb][t][l] is the 16-byte B operand of lane l for the 16-k step t of the 32-row block
// nb (row 32 nb + l % 32, k = 16 t + 8 (l / 32) .. + 7), so each wave loads its B fragments
// straight into registers, one contiguous kilobyte per plane and step, a stage ahead; only A
// goes through LDS (half the LDS traffic of k_gemm_x3).  Every MFMA sees the operands
// k_gemm_x3 gives it, in the same order: the results are the same bits.
// AMODE A_CONV reads A as the channels-last grouped causal conv's implicit im2col (load_a_fast): each
// 64-column tile is one group of 64 output channels, whose rows of the fragment-ordered weight are its
// own (cout, k * cin_g) rows, so B needs no group addressing.
template <int AMODE>
__global__ __launch_bounds__(256) void k_gemm_x3f(GemmParams p, const uint4* frag, int64_t per_plane, int tiles_m,
                                                  int tiles_n, int gm) {
  __shared__ uint4 sA[2][3][BM * 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int64_t m0, n0;
  tile_xcd(blockIdx.x, gridDim.x, tiles_m, tiles_n, gm, m0, n0);
  const int lr = tid >> 2, lc = tid & 3;
  const int64_t arow = min(m0 + lr, p.m - 1);
  int t_row = 0;
  const float* pa;
  if constexpr (AMODE == A_CONV) {
    const int bi = (int)arow / p.conv_t;
    t_row = (int)arow - bi * p.conv_t;
    pa = p.a + (int64_t)bi * p.conv_t * p.lda + (n0 / BN) * p.conv_cg + lc * 8;
  } else {
    pa = p.a + arow * p.lda + lc * 8;
  }
  const int wslot = xslot(lr, lc);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32, r32 = lane & 31, h = lane >> 5;
  const int ar = wm + r32, asw = (ar >> 2) & 3;
  const int64_t S = p.k / XBK, T16 = p.k / 16;
  // this wave's 32-column block; a block past the last (n % 64 in 1 .. 32) reads the last one
  // instead, its columns are dropped by store_tile
  const int64_t nblk = min((n0 + wn) >> 5, (p.n - 1) >> 5);
  const uint4* fb = frag + nblk * T16 * 64 + lane;
  f32x16 big = {0.f}, small = {0.f};
  struct XA {
    float4 a0, a1;
  };
  struct BF {
    uint4 v[2][3];  // [16-k step of the stage][plane]
  };
  auto load = [&](XA& x, int64_t k0) {
    x.a0 = load_a_fast<AMODE>(p, pa, t_row, k0);
    x.a1 = load_a_fast<AMODE>(p, pa, t_row, k0 + 4);
  };
  auto loadb = [&](BF& b, int64_t st) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int pl = 0; pl < 3; ++pl) b.v[ks][pl] = fb[pl * per_plane + (2 * st + ks) * 64];
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
    for (int ks = 0; ks < XBK / 16; ++ks) {
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

  // S even and >= 2: A ping-pongs through registers x / y and LDS buffers 0 / 1 as in k_gemm_x3;
  // the B fragments of the even and odd stages in b0 / b1, each refilled right after its use
  XA x, y;
  BF b0, b1;
  load(x, 0);
  load(y, XBK);
  loadb(b0, 0);
  loadb(b1, 1);
  store(0, x);
  __syncthreads();
  for (int64_t s = 0; s + 2 < S; s += 2) {
    load(x, (s + 2) * XBK);
    __builtin_amdgcn_sched_barrier(0);
    mma(0, b0);
    loadb(b0, s + 2);
    store(1, y);
    __syncthreads();
    load(y, (s + 3) * XBK);
    __builtin_amdgcn_sched_barrier(0);
    mma(1, b1);
    loadb(b1, s + 3);
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
  store_tile(p, acc, m0 + wm, h, n0 + wn + r32);
}

// frag[p][nb][t][l] = plane p of w[32 nb + l % 32][16 t + 8 (l / 32) .. + 7] (rows past n zero), the
// planes k_split_x3 makes, in k_gemm_x3f's fragment order.
__global__ __launch_bounds__(256) void k_split_x3_frag(const float* w, int64_t n, int64_t k, int64_t ldw, uint4* frag,
                                                       int64_t per_plane) {
  const int64_t T = k / 16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < per_plane;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const int64_t t = (i >> 6) % T, nb = (i >> 6) / T;
    const int64_t row = nb * 32 + (l & 31), k0 = 16 * t + 8 * (l >> 5);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (row < n) {
      a = *reinterpret_cast<const float4*>(w + row * ldw + k0);
      b = *reinterpret_cast<const float4*>(w + row * ldw + k0 + 4);
    }
    uint4 hi, mid, lo;
    split_x3(a, b, hi, mid, lo);
    frag[i] = hi;
    frag[per_plane + i] = mid;
    frag[2 * per_plane + i] = lo;
  }
}

// q8 weights on the bfloat16 matrix cores.  An int8 code is exact in bfloat16, so x . q
// needs only x's three planes: xh q, xm q and xl q, each exact in the float32 accumulate
// (three MFMAs per 16-k step where a float32 weight needs six).  The scale multiplies each
// block's sum: y = sum_b s_b (sum_{k in b} x_k q_k), where the reference sums x_k (q_k s_b)
// (quant.py:70-86,165-190): the same products, the scale applied once per block sum.  Tiling,
// A's split and the LDS layout are those of k_gemm_x3; B is one bfloat16 plane in LDS.
struct XStageQ {
  float4 a0, a1;  // A: row lr, k = 8 * lc .. + 7 of the stage
  uint2 b;        // B: the same row's 8 codes
};

__device__ __forceinline__ uint4 codes_bf16(uint2 w) {
  uint4 r;
  uint32_t* o = &r.x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t word = j < 2 ? w.x : w.y;
    const int sh = (j & 1) * 16;
    const f32x2_t v = {(float)((int32_t)(word << (24 - sh)) >> 24), (float)((int32_t)(word << (16 - sh)) >> 24)};
    o[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  }
  return r;
}

// K % 64 == 0, block % 64 == 0; A rows 16-byte aligned, code rows 8-byte aligned.
__global__ __launch_bounds__(256) void k_gemm_x3q(GemmParams p, int tiles_m, int tiles_n, int gm) {
  __shared__ uint4 sA[2][3][BM * 4];
  __shared__ uint4 sB[2][BN * 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int64_t m0, n0;
  tile_xcd(blockIdx.x, gridDim.x, tiles_m, tiles_n, gm, m0, n0);
  const int lr = tid >> 2, lc = tid & 3;
  const float* pa = p.a + min(m0 + lr, p.m - 1) * p.lda + lc * 8;
  const int8_t* pbr = reinterpret_cast<const int8_t*>(p.b) + min(n0 + lr, p.n - 1) * p.ldb + lc * 8;
  const int wslot = xslot(lr, lc);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32, r32 = lane & 31, h = lane >> 5;
  const int ar = wm + r32, br = wn + r32, asw = (ar >> 2) & 3, bsw = (br >> 2) & 3;
  const int64_t S = p.k / XBK, spb = p.block / XBK;
  // the lane's output column's scales
  const int64_t srow = min(n0 + wn + r32, p.n - 1) * p.nb;
  auto scale = [&](int64_t b) {
    return p.sf16 ? __half2float(reinterpret_cast<const __half*>(p.scales)[srow + b])
                  : reinterpret_cast<const float*>(p.scales)[srow + b];
  };
  f32x16 big = {0.f}, small = {0.f}, acc = {0.f};
  float s_cur = scale(0);
  int64_t blk = 0;
  // acc += s_b * (this block's sum); the next block's scale is loaded here, a block ahead
  auto fold = [&]() {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i] = fmaf(s_cur, big[i] + small[i], acc[i]);
      big[i] = 0.f;
      small[i] = 0.f;
    }
    ++blk;
    s_cur = scale(min(blk, p.nb - 1));
  };

  auto load = [&](XStageQ& x, int64_t k0) {
    x.a0 = *reinterpret_cast<const float4*>(pa + k0);
    x.a1 = *reinterpret_cast<const float4*>(pa + k0 + 4);
    x.b = *reinterpret_cast<const uint2*>(pbr + k0);
  };
  auto store = [&](int buf, const XStageQ& x) {
    uint4 hi, mid, lo;
    split_x3(x.a0, x.a1, hi, mid, lo);
    sA[buf][0][wslot] = hi;
    sA[buf][1][wslot] = mid;
    sA[buf][2][wslot] = lo;
    sB[buf][wslot] = codes_bf16(x.b);
  };
  auto mma = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < XBK / 16; ++ks) {
      const int c = ks * 2 + h;
      const int sa = ar * 4 + (c ^ asw), sb = br * 4 + (c ^ bsw);
      const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, sA[buf][0][sa]);
      const bf16x8_t am = __builtin_bit_cast(bf16x8_t, sA[buf][1][sa]);
      const bf16x8_t al = __builtin_bit_cast(bf16x8_t, sA[buf][2][sa]);
      const bf16x8_t bq = __builtin_bit_cast(bf16x8_t, sB[buf][sb]);
      big = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bq, big, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bq, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bq, small, 0, 0, 0);
    }
  };

  // S even and >= 2; a block is an even number of stages, so blocks end between iterations
  XStageQ x, y;
  load(x, 0);
  load(y, XBK);
  store(0, x);
  __syncthreads();
  int64_t s = 0;
  for (; s + 2 < S; s += 2) {
    load(x, (s + 2) * XBK);
    __builtin_amdgcn_sched_barrier(0);
    mma(0);
    store(1, y);
    __syncthreads();
    load(y, (s + 3) * XBK);
    __builtin_amdgcn_sched_barrier(0);
    mma(1);
    store(0, x);
    __syncthreads();
    if ((s + 2) % spb == 0) fold();
  }
  mma(0);
  store(1, y);
  __syncthreads();
  mma(1);
  fold();  // the last block (or the part of it K covers)
  store_tile(p, acc, m0 + wm, h, n0 + wn + r32);
}

// The same q8 GEMM with the codes packed once in MFMA fragment order (k_pack_q8_frag):
// qfrag[nb][t][l] holds the 8 codes of lane l for the 16-k step t of the 32-row block nb (row
// 32 nb + l % 32, k = 16 t + 8 (l / 32) .. + 7), so each wave loads its B fragments (8 bytes per
// lane, 512 contiguous bytes) straight into registers a stage ahead and widens them to bfloat16
// there; only A goes through LDS.  The same products in the same order as k_gemm_x3q.
__global__ __launch_bounds__(256) void k_gemm_x3qf(GemmParams p, const uint2* qfrag, int tiles_m, int tiles_n,
                                                   int gm) {
  __shared__ uint4 sA[2][3][BM * 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int64_t m0, n0;
  tile_xcd(blockIdx.x, gridDim.x, tiles_m, tiles_n, gm, m0, n0);
  const int lr = tid >> 2, lc = tid & 3;
  const float* pa = p.a + min(m0 + lr, p.m - 1) * p.lda + lc * 8;
  const int wslot = xslot(lr, lc);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32, r32 = lane & 31, h = lane >> 5;
  const int ar = wm + r32, asw = (ar >> 2) & 3;
  const int64_t S = p.k / XBK, spb = p.block / XBK, T16 = p.k / 16;
  const int64_t nblk = min((n0 + wn) >> 5, (p.n - 1) >> 5);  // clamped as in k_gemm_x3f
  const uint2* fb = qfrag + nblk * T16 * 64 + lane;
  // the lane's output column's scales
  const int64_t srow = min(n0 + wn + r32, p.n - 1) * p.nb;
  auto scale = [&](int64_t b) {
    return p.sf16 ? __half2float(reinterpret_cast<const __half*>(p.scales)[srow + b])
                  : reinterpret_cast<const float*>(p.scales)[srow + b];
  };
  f32x16 big = {0.f}, small = {0.f}, acc = {0.f};
  float s_cur = scale(0);
  int64_t blk = 0;
  auto fold = [&]() {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i] = fmaf(s_cur, big[i] + small[i], acc[i]);
      big[i] = 0.f;
      small[i] = 0.f;
    }
    ++blk;
    s_cur = scale(min(blk, p.nb - 1));
  };
  struct XA {
    float4 a0, a1;
  };
  struct BQ {
    uint2 v[2];  // the stage's two 16-k steps
  };
  auto load = [&](XA& x, int64_t k0) {
    x.a0 = *reinterpret_cast<const float4*>(pa + k0);
    x.a1 = *reinterpret_cast<const float4*>(pa + k0 + 4);
  };
  auto loadb = [&](BQ& b, int64_t st) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) b.v[ks] = fb[(2 * st + ks) * 64];
  };
  auto store = [&](int buf, const XA& x) {
    uint4 hi, mid, lo;
    split_x3(x.a0, x.a1, hi, mid, lo);
    sA[buf][0][wslot] = hi;
    sA[buf][1][wslot] = mid;
    sA[buf][2][wslot] = lo;
  };
  auto mma = [&](int buf, const BQ& b) {
#pragma unroll
    for (int ks = 0; ks < XBK / 16; ++ks) {
      const int c = ks * 2 + h;
      const int sa = ar * 4 + (c ^ asw);
      const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, sA[buf][0][sa]);
      const bf16x8_t am = __builtin_bit_cast(bf16x8_t, sA[buf][1][sa]);
      const bf16x8_t al = __builtin_bit_cast(bf16x8_t, sA[buf][2][sa]);
      const bf16x8_t bq = __builtin_bit_cast(bf16x8_t, codes_bf16(b.v[ks]));
      big = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bq, big, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bq, small, 0, 0, 0);
      small = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bq, small, 0, 0, 0);
    }
  };

  // as k_gemm_x3f: A through registers x / y and LDS buffers 0 / 1, B fragments in b0 / b1
  XA x, y;
  BQ b0, b1;
  load(x, 0);
  load(y, XBK);
  loadb(b0, 0);
  loadb(b1, 1);
  store(0, x);
  __syncthreads();
  int64_t s = 0;
  for (; s + 2 < S; s += 2) {
    load(x, (s + 2) * XBK);
    __builtin_amdgcn_sched_barrier(0);
    mma(0, b0);
    loadb(b0, s + 2);
    store(1, y);
    __syncthreads();
    load(y, (s + 3) * XBK);
    __builtin_amdgcn_sched_barrier(0);
    mma(1, b1);
    loadb(b1, s + 3);
    store(0, x);
    __syncthreads();
    if ((s + 2) % spb == 0) fold();
  }
  mma(0, b0);
  store(1, y);
  __syncthreads();
  mma(1, b1);
  fold();  // the last block (or the part of it K covers)
  store_tile(p, acc, m0 + wm, h, n0 + wn + r32);
}

// qfrag[nb][t][l] = the 8 codes q[32 nb + l % 32][16 t + 8 (l / 32) .. + 7] (rows past n zero): the
// q8 codes in k_gemm_x3qf's fragment order.
__global__ __launch_bounds__(256) void k_pack_q8_frag(const int8_t* q, int64_t n, int64_t k, int64_t ldq, uint2* frag,
                                                      int64_t total) {
  const int64_t T = k / 16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const int64_t t = (i >> 6) % T, nb = (i >> 6) / T;
    const int64_t row = nb * 32 + (l & 31), k0 = 16 * t + 8 * (l >> 5);
    frag[i] = row < n ? *reinterpret_cast<const uint2*>(q + row * ldq + k0) : make_uint2(0u, 0u);
  }
}

// planes[p][row][0 .. k) = plane p of w[row][0 .. k); eight k per thread.
__global__ __launch_bounds__(256) void k_split_x3(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* pb,
                                                  int64_t ldp, int64_t pstride) {
  const int64_t per_row = k / 8, total = n * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / per_row, k0 = (i - row * per_row) * 8;
    const float* src = w + row * ldw + k0;
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 b = *reinterpret_cast<const float4*>(src + 4);
    uint4 hi, mid, lo;
    split_x3(a, b, hi, mid, lo);
    uint16_t* dst = pb + row * ldp + k0;
    *reinterpret_cast<uint4*>(dst) = hi;
    *reinterpret_cast<uint4*>(dst + pstride) = mid;
    *reinterpret_cast<uint4*>(dst + 2 * pstride) = lo;
  }
}


// q8 linears with the activation as four int8 digit planes (per-channel scales).  Row r of A
// is rounded once to X = rint(a 2^(30 - E_r)), E_r the exponent of the row's largest |a| (every
// |a| < 2^E_r, so |X| < 2^30), whose bytes are its base-256 digits: X = b0 + 256 b1 + 65536 b2
// + 2^24 b3 with b0..b2 unsigned (0..255) and b3 = X >> 24 signed (-64..63).  The matrix cores
// take signed bytes, so planes 0-2 carry b - 128 (the byte with its top bit flipped) and the
// epilogue adds back 128 times the column's code sum.  Each plane times the int8 codes is an
// exact int32 sum on v_mfma_i32_32x32x32_i8 (|sum| < 2^31 for K <= 2048), the four are
// combined exactly in float64, times 2^(E_r - 30) and the column's scale: the dot product of
// the codes with a rounded 30 bits below the row's largest element.  Four int8 products where
// the bfloat16 planes need three bfloat16 ones at half the rate; the digits are byte permutes
// of X, the codes go to the matrix cores as they are, and A takes 4 bytes of LDS per element
// instead of 6.

// E_r for each row: one wave per row (frexp of the row's largest |a|; at least -96, so
// 2^(27 - E) stays finite and tiny rows only lose low bits).
__global__ __launch_bounds__(256) void k_row_exp(const float* __restrict__ a, int64_t m, int64_t k, int64_t lda,
                                                 int* __restrict__ e) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m) return;
  const float* r = a + row * lda;
  float mx = 0.f;
  for (int64_t j = 4 * lane; j < k; j += 256) {
    const float4 v = *reinterpret_cast<const float4*>(r + j);
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  int ex = 0;
  if (mx > 0.f) (void)frexpf(mx, &ex);
  if (lane == 0) e[row] = max(ex, -96);
}

// frag[i], i = (nb T + t) 64 + l, T = k / 32: the 16 codes q[32 nb + l % 32][32 t + 16 (l / 32) .. + 15]
// (rows past n zero), the B operand of v_mfma_i32_32x32x32_i8 for 32-row block nb, step t;
// then (k_q8_row_sums) each row's code sum as int32.
__global__ __launch_bounds__(256) void k_pack_q8_frag32(const int8_t* q, int64_t n, int64_t k, int64_t ldq, uint4* frag,
                                                        int64_t total) {
  const int64_t T = k / 32;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const int64_t t = (i >> 6) % T, nb = (i >> 6) / T;
    const int64_t row = nb * 32 + (l & 31), k0 = 32 * t + 16 * (l >> 5);
    frag[i] = row < n ? *reinterpret_cast<const uint4*>(q + row * ldq + k0) : make_uint4(0u, 0u, 0u, 0u);
  }
}

// sums[row] = sum of the row's k codes (rows past n zero): one wave per row.
__global__ __launch_bounds__(256) void k_q8_row_sums(const int8_t* q, int64_t n, int64_t npad, int64_t k, int64_t ldq,
                                                     int* sums) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= npad) return;
  int acc = 0;
  if (row < n)
    for (int64_t j = lane; j < k; j += 64) acc += q[row * ldq + j];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (lane == 0) sums[row] = acc;
}

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x4v __attribute__((ext_vector_type(4)));

// 64 x 64 tiles, four waves of 32 x 32, 64-k stages.  A goes global -> registers -> its four
// digit planes -> LDS (16-byte chunk c of row r at slot 4 r + (c ^ (r / 4) % 4), so the 16
// rows a wave reads at one chunk land on 16 different banks); the codes go global -> registers
// in fragment order (k_pack_q8_frag32), a stage ahead.
__global__ __launch_bounds__(256) void k_gemm_q8d(GemmParams p, const uint4* qfrag, const int* qsums, const int* rexp,
                                                  int tiles_m, int tiles_n, int gm) {
  __shared__ uint4 sA[2][4][BM * 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int64_t m0, n0;
  tile_xcd(blockIdx.x, gridDim.x, tiles_m, tiles_n, gm, m0, n0);
  const int lr = tid >> 2, lc = tid & 3;  // staging: row lr, k 16 lc .. + 15 of the stage
  const int64_t arow = min(m0 + lr, p.m - 1);
  const float* pa = p.a + arow * p.lda + lc * 16;
  const float up = ldexpf(1.0f, 30 - rexp[arow]);
  const int wslot = lr * 4 + (lc ^ ((lr >> 2) & 3));
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32, r32 = lane & 31, h = lane >> 5;
  const int ar = wm + r32;
  const int64_t S = p.k / 64, T32 = p.k / 32;
  const int64_t nblk = min((n0 + wn) >> 5, (p.n - 1) >> 5);
  const uint4* fb = qfrag + nblk * T32 * 64 + lane;
  i32x16 acc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) acc[q] = i32x16{0};
  struct XA {
    float4 v[4];
  };
  struct BQ {
    uint4 v[2];  // the stage's two 32-k steps
  };
  auto load = [&](XA& x, int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x.v[i] = *reinterpret_cast<const float4*>(pa + k0 + 4 * i);
  };
  auto loadb = [&](BQ& b, int64_t st) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) b.v[ks] = fb[(2 * st + ks) * 64];
  };
  auto store = [&](int buf, const XA& x) {
    uint32_t pl[4][4];  // plane, 4 bytes of the 16 k
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      const uint32_t X0 = (uint32_t)__float2int_rn(x.v[w4].x * up), X1 = (uint32_t)__float2int_rn(x.v[w4].y * up);
      const uint32_t X2 = (uint32_t)__float2int_rn(x.v[w4].z * up), X3 = (uint32_t)__float2int_rn(x.v[w4].w * up);
      // bytes (X0.b0, X1.b0, X0.b1, X1.b1) and (X0.b2, X1.b2, X0.b3, X1.b3), the same for X2, X3
      const uint32_t lo01 = __builtin_amdgcn_perm(X1, X0, 0x05010400u), hi01 = __builtin_amdgcn_perm(X1, X0, 0x07030602u);
      const uint32_t lo23 = __builtin_amdgcn_perm(X3, X2, 0x05010400u), hi23 = __builtin_amdgcn_perm(X3, X2, 0x07030602u);
      pl[0][w4] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;
      pl[1][w4] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;
      pl[2][w4] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u) ^ 0x80808080u;
      pl[3][w4] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) sA[buf][q][wslot] = make_uint4(pl[q][0], pl[q][1], pl[q][2], pl[q][3]);
  };
  auto mma = [&](int buf, const BQ& b) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 2 + h;
      const int sa = ar * 4 + (c ^ ((ar >> 2) & 3));
      const i32x4v bq = __builtin_bit_cast(i32x4v, b.v[ks]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4v, sA[buf][q][sa]), bq, acc[q], 0, 0, 0);
    }
  };
  XA x, y;
  BQ b0, b1;
  load(x, 0);
  if (S > 1) load(y, 64);
  loadb(b0, 0);
  if (S > 1) loadb(b1, 1);
  store(0, x);
  __syncthreads();
  int64_t s = 0;
  for (; s + 2 < S; s += 2) {
    load(x, (s + 2) * 64);
    __builtin_amdgcn_sched_barrier(0);
    mma(0, b0);
    loadb(b0, s + 2);
    store(1, y);
    __syncthreads();
    load(y, (s + 3) * 64);
    __builtin_amdgcn_sched_barrier(0);
    mma(1, b1);
    loadb(b1, s + 3);
    store(0, x);
    __syncthreads();
  }
  mma(0, b0);
  if (s + 1 < S) {
    store(1, y);
    __syncthreads();
    mma(1, b1);
  }
  // T = sum_q 256^q acc_q + 128 (1 + 256 + 65536) (the column's code sum) exactly in float64,
  // times 2^(E - 30) and the column's scale
  const int64_t col = min(n0 + wn + r32, p.n - 1);
  const double sc = p.sf16 ? (double)__half2float(reinterpret_cast<const __half*>(p.scales)[col])
                           : (double)reinterpret_cast<const float*>(p.scales)[col];
  const double corr = 128.0 * 65793.0 * (double)qsums[col];
  f32x16 out;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = min(m0 + wm + (i >> 2) * 8 + h * 4 + (i & 3), p.m - 1);
    const double t = (double)acc[0][i] + 256.0 * (double)acc[1][i] + 65536.0 * (double)acc[2][i] +
                     16777216.0 * (double)acc[3][i] + corr;
    out[i] = (float)(t * ldexp(1.0, rexp[row] - 30) * sc);
  }
  store_tile(p, out, m0 + wm, h, n0 + wn + r32);
}
}  // namespace

namespace cv3 {

int gemm(int bkind, const float* a, int64_t m, int64_t k, int64_t lda, const void* b, int64_t ldb,
         const void* scales, bool sf16, int64_t nb, int64_t block, int64_t n, const float* bias, float* c,
         int64_t ldc, const cv3_epilogue* epi, hipStream_t st) {
  CV3_REQUIRE(bkind == B_F32 || bkind == B_Q8 || bkind == B_Q4, CV3_EINVAL, "unknown GEMM operand kind %d", bkind);
  CV3_REQUIRE(bkind != B_Q4 || (block == 32 && sf16), CV3_EUNSUPPORTED,
              "q4 GEMM needs 32-code blocks with float16 scales");
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
  const int fast_b = bkind == B_Q8   ? (((uintptr_t)b % 4 == 0) && (ldb % 4 == 0) && (block % 4 == 0))
                     : bkind == B_Q4 ? (((uintptr_t)b % 4 == 0) && (ldb % 4 == 0))
                                     : (((uintptr_t)b % 16 == 0) && (ldb % 4 == 0));
  const int64_t tiles_m = ceil_div(m, BM), tiles_n = ceil_div(n, BN);
  CV3_REQUIRE(tiles_m * tiles_n < (1ll << 31), CV3_EINVAL, "GEMM too large");
  const dim3 grid((unsigned)(tiles_m * tiles_n));
  p.conv_t = p.conv_cg = p.conv_pad = 0;
  // the branch-free kernel: whole K stages and aligned rows for both operands
  const bool fast = fast_a && fast_b && k % (2 * BK) == 0;
  CV3_REQUIRE(fast || !p.epi.rope_cos, CV3_EUNSUPPORTED, "rotary epilogue needs aligned rows and K %% 64 == 0");
  CV3_REQUIRE(!p.epi.rope_cos || (p.epi.rope_rows > 0 && p.epi.rope_period > 0 && p.epi.rope_width > 0 &&
                                  p.epi.rope_rows * p.epi.rope_width < (1ll << 31) && m + 64 < (1ll << 31) &&
                                  n < (1ll << 31)),
              CV3_EINVAL, "rotary epilogue: table or GEMM beyond 32-bit indexing");
  // at most one 64 x 64 tile per CU: the 8-wave kernel keeps two waves per SIMD
  const bool small = tiles_m * tiles_n <= 256;
  // A beyond one XCD's L2: walk groups of 8 M-tiles (the tile order note at the top)
  const int group_m = m * k * (int64_t)sizeof(float) > (4ll << 20) ? 8 : 0;
  if (bkind == B_Q8) {
    if (fast && small)
      hipLaunchKernelGGL((k_gemm8<B_Q8, A_ROWS>), grid, dim3(512), 0, st, p, (int)tiles_m);
    else if (fast)
      hipLaunchKernelGGL((k_gemm<B_Q8, true>), grid, dim3(256), 0, st, p, fast_a, fast_b, (int)tiles_m, group_m);
    else
      hipLaunchKernelGGL((k_gemm<B_Q8, false>), grid, dim3(256), 0, st, p, fast_a, fast_b, (int)tiles_m, group_m);
  } else if (bkind == B_Q4) {
    if (fast && small)
      hipLaunchKernelGGL((k_gemm8<B_Q4, A_ROWS>), grid, dim3(512), 0, st, p, (int)tiles_m);
    else if (fast)
      hipLaunchKernelGGL((k_gemm<B_Q4, true>), grid, dim3(256), 0, st, p, fast_a, fast_b, (int)tiles_m, group_m);
    else
      hipLaunchKernelGGL((k_gemm<B_Q4, false>), grid, dim3(256), 0, st, p, fast_a, fast_b, (int)tiles_m, group_m);
  } else {
    if (fast && tiles_m * tiles_n <= 512)
      hipLaunchKernelGGL(k_gemm_dma, grid, dim3(256), 0, st, p, (int)tiles_m);
    else if (fast)
      hipLaunchKernelGGL((k_gemm<B_F32, true>), grid, dim3(256), 0, st, p, fast_a, fast_b, (int)tiles_m, group_m);
    else
      hipLaunchKernelGGL((k_gemm<B_F32, false>), grid, dim3(256), 0, st, p, fast_a, fast_b, (int)tiles_m, group_m);
  }
  CV3_LAUNCHED();
  return CV3_OK;
}

// Group height for tile_xcd: column by column while A is the smaller operand; otherwise one
// XCD's share of the tiles covers a few row tiles across all columns, so A streams from HBM once.
static int tile_group(int64_t tiles_m, int64_t tiles_n, double a_bytes, double b_bytes) {
  if (a_bytes <= b_bytes) return (int)tiles_m;
  const int64_t per_xcd = ceil_div(tiles_m * tiles_n, 8);
  return (int)std::max<int64_t>(1, std::min<int64_t>(tiles_m, ceil_div(per_xcd, tiles_n)));
}

// C = epi(A . B^T) on the bfloat16 matrix cores, B as three bfloat16 planes
// planes[p][n][ldp] (pstride elements apart).  K % 64 == 0.
int gemm_x3(const float* a, int64_t m, int64_t k, int64_t lda, const uint16_t* planes, int64_t ldp, int64_t pstride,
            int64_t n, const float* bias, float* c, int64_t ldc, const cv3_epilogue* epi, hipStream_t st) {
  CV3_REQUIRE(k % (2 * XBK) == 0, CV3_EUNSUPPORTED, "split-bfloat16 GEMM needs K %% 64 == 0 (K = %lld)",
              (long long)k);
  CV3_REQUIRE(((uintptr_t)a % 16 == 0) && lda % 4 == 0 && ((uintptr_t)planes % 16 == 0) && ldp % 8 == 0 &&
                  pstride % 8 == 0 && ldp >= k && pstride >= n * ldp,
              CV3_EINVAL, "split-bfloat16 GEMM operands must be 16-byte aligned rows");
  GemmParams p{};
  p.a = a;
  p.lda = lda;
  p.m = m;
  p.n = n;
  p.k = k;
  p.bias = bias;
  p.c = c;
  p.ldc = ldc;
  p.epi = epi ? *epi : cv3_epilogue{};
  CV3_REQUIRE(!p.epi.rope_cos || (p.epi.rope_rows > 0 && p.epi.rope_period > 0 && p.epi.rope_width > 0 &&
                                  p.epi.rope_rows * p.epi.rope_width < (1ll << 31) && m + 64 < (1ll << 31) &&
                                  n < (1ll << 31)),
              CV3_EINVAL, "rotary epilogue: table or GEMM beyond 32-bit indexing");
  const int64_t tiles_m = ceil_div(m, BM), tiles_n = ceil_div(n, BN);
  CV3_REQUIRE(tiles_m * tiles_n < (1ll << 31), CV3_EINVAL, "GEMM too large");
  const int gm = tile_group(tiles_m, tiles_n, 4.0 * (double)m * k, 6.0 * (double)n * k);
  hipLaunchKernelGGL(k_gemm_x3, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st, p, planes, ldp, pstride,
                     (int)tiles_m, (int)tiles_n, gm);
  CV3_LAUNCHED();
  return CV3_OK;
}

int pack_q8_frag(const int8_t* q, int64_t n, int64_t k, int64_t ldq, int8_t* frag, hipStream_t st) {
  CV3_REQUIRE(k % 64 == 0 && ((uintptr_t)q % 8 == 0) && ldq % 8 == 0 && ldq >= k && ((uintptr_t)frag % 8 == 0),
              CV3_EINVAL, "fragment-ordered codes need K %% 64 == 0 and 8-byte aligned rows");
  const int64_t total = ceil_div(n, 32) * 32 * k / 8;  // 8-byte fragments
  if (total == 0) return CV3_OK;
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 65536);
  hipLaunchKernelGGL(k_pack_q8_frag, dim3((unsigned)blocks), dim3(256), 0, st, q, n, k, ldq,
                     reinterpret_cast<uint2*>(frag), total);
  CV3_LAUNCHED();
  return CV3_OK;
}

// C = epi(A . dequant(q)^T) with the codes in fragment order (pack_q8_frag), scales [n, nb].
int gemm_x3qf(const float* a, int64_t m, int64_t k, int64_t lda, const int8_t* qfrag, const void* scales, bool sf16,
              int64_t nb, int64_t block, int64_t n, const float* bias, float* c, int64_t ldc,
              const cv3_epilogue* epi, hipStream_t st) {
  CV3_REQUIRE(k % (2 * XBK) == 0 && block % (2 * XBK) == 0 && nb * block >= k, CV3_EUNSUPPORTED,
              "split-bfloat16 q8 GEMM needs K %% 64 == 0 and blocks of a multiple of 64 (K = %lld, block = %lld)",
              (long long)k, (long long)block);
  CV3_REQUIRE(((uintptr_t)a % 16 == 0) && lda % 4 == 0 && ((uintptr_t)qfrag % 8 == 0), CV3_EINVAL,
              "split-bfloat16 q8 GEMM operands must be aligned rows");
  GemmParams p{};
  p.a = a;
  p.lda = lda;
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
  CV3_REQUIRE(!p.epi.rope_cos || (p.epi.rope_rows > 0 && p.epi.rope_period > 0 && p.epi.rope_width > 0 &&
                                  p.epi.rope_rows * p.epi.rope_width < (1ll << 31) && m + 64 < (1ll << 31) &&
                                  n < (1ll << 31)),
              CV3_EINVAL, "rotary epilogue: table or GEMM beyond 32-bit indexing");
  const int64_t tiles_m = ceil_div(m, BM), tiles_n = ceil_div(n, BN);
  CV3_REQUIRE(tiles_m * tiles_n < (1ll << 31), CV3_EINVAL, "GEMM too large");
  const int gm = tile_group(tiles_m, tiles_n, 4.0 * (double)m * k, (double)n * k);
  hipLaunchKernelGGL(k_gemm_x3qf, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st, p,
                     reinterpret_cast<const uint2*>(qfrag), (int)tiles_m, (int)tiles_n, gm);
  CV3_LAUNCHED();
  return CV3_OK;
}


int pack_q8_frag32(const int8_t* q, int64_t n, int64_t k, int64_t ldq, int8_t* frag, hipStream_t st) {
  CV3_REQUIRE(k % 64 == 0 && ((uintptr_t)q % 16 == 0) && ldq % 16 == 0 && ldq >= k && ((uintptr_t)frag % 16 == 0),
              CV3_EINVAL, "digit-plane codes need K %% 64 == 0 and 16-byte aligned rows");
  const int64_t npad = ceil_div(n, 32) * 32, total = npad * k / 16;  // 16-byte fragments
  if (total == 0) return CV3_OK;
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 65536);
  hipLaunchKernelGGL(k_pack_q8_frag32, dim3((unsigned)blocks), dim3(256), 0, st, q, n, k, ldq,
                     reinterpret_cast<uint4*>(frag), total);
  hipLaunchKernelGGL(k_q8_row_sums, dim3((unsigned)ceil_div(npad, 4)), dim3(256), 0, st, q, n, npad, k, ldq,
                     reinterpret_cast<int*>(frag + npad * k));
  CV3_LAUNCHED();
  return CV3_OK;
}

// C = epi(A . dequant(q)^T) with A as four int8 digit planes per row and per-channel scales [n];
// rexp: m ints of workspace (the rows' exponents, written here first).
int gemm_q8d(const float* a, int64_t m, int64_t k, int64_t lda, const int8_t* qfrag32, const void* scales, bool sf16,
             int64_t n, const float* bias, float* c, int64_t ldc, const cv3_epilogue* epi, int* rexp, bool rexp_given, hipStream_t st) {
  CV3_REQUIRE(k % 64 == 0 && k <= 2048, CV3_EUNSUPPORTED,
              "digit-plane q8 GEMM needs K %% 64 == 0 and K <= 2048 (K = %lld)", (long long)k);
  CV3_REQUIRE(((uintptr_t)a % 16 == 0) && lda % 4 == 0 && ((uintptr_t)qfrag32 % 16 == 0) && rexp, CV3_EINVAL,
              "digit-plane q8 GEMM operands must be aligned rows, with a row-exponent workspace");
  GemmParams p{};
  p.a = a;
  p.lda = lda;
  p.scales = scales;
  p.sf16 = sf16;
  p.nb = 1;
  p.block = k;
  p.m = m;
  p.n = n;
  p.k = k;
  p.bias = bias;
  p.c = c;
  p.ldc = ldc;
  p.epi = epi ? *epi : cv3_epilogue{};
  CV3_REQUIRE(!p.epi.rope_cos || (p.epi.rope_rows > 0 && p.epi.rope_period > 0 && p.epi.rope_width > 0 &&
                                  p.epi.rope_rows * p.epi.rope_width < (1ll << 31) && m + 64 < (1ll << 31) &&
                                  n < (1ll << 31)),
              CV3_EINVAL, "rotary epilogue: table or GEMM beyond 32-bit indexing");
  const int64_t tiles_m = ceil_div(m, BM), tiles_n = ceil_div(n, BN);
  CV3_REQUIRE(tiles_m * tiles_n < (1ll << 31), CV3_EINVAL, "GEMM too large");
  if (!rexp_given)
    hipLaunchKernelGGL(k_row_exp, dim3((unsigned)ceil_div(m, 4)), dim3(256), 0, st, a, m, k, lda, rexp);
  const int gm = tile_group(tiles_m, tiles_n, 4.0 * (double)m * k, (double)n * k);
  hipLaunchKernelGGL(k_gemm_q8d, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st, p,
                     reinterpret_cast<const uint4*>(qfrag32),
                     reinterpret_cast<const int*>(qfrag32 + ceil_div(n, 32) * 32 * k), rexp, (int)tiles_m,
                     (int)tiles_n, gm);
  CV3_LAUNCHED();
  return CV3_OK;
}

// Elements of one plane of the fragment-ordered weight: 32-row blocks x K.
int64_t x3_frag_plane(int64_t n, int64_t k) { return ceil_div(n, 32) * 32 * k; }

int split_x3_frag(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* frag, hipStream_t st) {
  CV3_REQUIRE(k % 64 == 0 && ((uintptr_t)w % 16 == 0) && ldw % 4 == 0 && ldw >= k && ((uintptr_t)frag % 16 == 0),
              CV3_EINVAL, "fragment-ordered planes need K %% 64 == 0 and 16-byte aligned rows");
  const int64_t per_plane = x3_frag_plane(n, k) / 8;  // 16-byte fragments
  if (per_plane == 0) return CV3_OK;
  const int64_t blocks = std::min<int64_t>(ceil_div(per_plane, 256), 65536);
  hipLaunchKernelGGL(k_split_x3_frag, dim3((unsigned)blocks), dim3(256), 0, st, w, n, k, ldw,
                     reinterpret_cast<uint4*>(frag), per_plane);
  CV3_LAUNCHED();
  return CV3_OK;
}

// C = epi(A . B^T) with B as fragment-ordered planes (split_x3_frag).  K % 64 == 0.
int gemm_x3f(const float* a, int64_t m, int64_t k, int64_t lda, const uint16_t* frag, int64_t n, const float* bias,
             float* c, int64_t ldc, const cv3_epilogue* epi, hipStream_t st) {
  CV3_REQUIRE(k % (2 * XBK) == 0, CV3_EUNSUPPORTED, "split-bfloat16 GEMM needs K %% 64 == 0 (K = %lld)",
              (long long)k);
  CV3_REQUIRE(((uintptr_t)a % 16 == 0) && lda % 4 == 0 && ((uintptr_t)frag % 16 == 0), CV3_EINVAL,
              "split-bfloat16 GEMM operands must be 16-byte aligned rows");
  GemmParams p{};
  p.a = a;
  p.lda = lda;
  p.m = m;
  p.n = n;
  p.k = k;
  p.bias = bias;
  p.c = c;
  p.ldc = ldc;
  p.epi = epi ? *epi : cv3_epilogue{};
  CV3_REQUIRE(!p.epi.rope_cos || (p.epi.rope_rows > 0 && p.epi.rope_period > 0 && p.epi.rope_width > 0 &&
                                  p.epi.rope_rows * p.epi.rope_width < (1ll << 31) && m + 64 < (1ll << 31) &&
                                  n < (1ll << 31)),
              CV3_EINVAL, "rotary epilogue: table or GEMM beyond 32-bit indexing");
  const int64_t tiles_m = ceil_div(m, BM), tiles_n = ceil_div(n, BN);
  CV3_REQUIRE(tiles_m * tiles_n < (1ll << 31), CV3_EINVAL, "GEMM too large");
  const int gm = tile_group(tiles_m, tiles_n, 4.0 * (double)m * k, 6.0 * (double)n * k);
  hipLaunchKernelGGL(k_gemm_x3f<A_ROWS>, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st, p,
                     reinterpret_cast<const uint4*>(frag), x3_frag_plane(n, k) / 8, (int)tiles_m, (int)tiles_n, gm);
  CV3_LAUNCHED();
  return CV3_OK;
}

// C = epi(A . dequant(q)^T) on the bfloat16 matrix cores: q8 codes [n, ldq], scales [n, nb].
int gemm_x3q(const float* a, int64_t m, int64_t k, int64_t lda, const int8_t* q, int64_t ldq, const void* scales,
             bool sf16, int64_t nb, int64_t block, int64_t n, const float* bias, float* c, int64_t ldc,
             const cv3_epilogue* epi, hipStream_t st) {
  CV3_REQUIRE(k % (2 * XBK) == 0 && block % (2 * XBK) == 0 && nb * block >= k, CV3_EUNSUPPORTED,
              "split-bfloat16 q8 GEMM needs K %% 64 == 0 and blocks of a multiple of 64 (K = %lld, block = %lld)",
              (long long)k, (long long)block);
  CV3_REQUIRE(((uintptr_t)a % 16 == 0) && lda % 4 == 0 && ((uintptr_t)q % 8 == 0) && ldq % 8 == 0 && ldq >= k,
              CV3_EINVAL, "split-bfloat16 q8 GEMM operands must be aligned rows");
  GemmParams p{};
  p.a = a;
  p.lda = lda;
  p.b = q;
  p.ldb = ldq;
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
  CV3_REQUIRE(!p.epi.rope_cos || (p.epi.rope_rows > 0 && p.epi.rope_period > 0 && p.epi.rope_width > 0 &&
                                  p.epi.rope_rows * p.epi.rope_width < (1ll << 31) && m + 64 < (1ll << 31) &&
                                  n < (1ll << 31)),
              CV3_EINVAL, "rotary epilogue: table or GEMM beyond 32-bit indexing");
  const int64_t tiles_m = ceil_div(m, BM), tiles_n = ceil_div(n, BN);
  CV3_REQUIRE(tiles_m * tiles_n < (1ll << 31), CV3_EINVAL, "GEMM too large");
  const int gm = tile_group(tiles_m, tiles_n, 4.0 * (double)m * k, (double)n * k);
  hipLaunchKernelGGL(k_gemm_x3q, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st, p, (int)tiles_m,
                     (int)tiles_n, gm);
  CV3_LAUNCHED();
  return CV3_OK;
}

int split_x3(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* planes, int64_t ldp, int64_t pstride,
             hipStream_t st) {
  CV3_REQUIRE(k % 8 == 0 && ((uintptr_t)w % 16 == 0) && ldw % 4 == 0 && ((uintptr_t)planes % 16 == 0) &&
                  ldp % 8 == 0 && pstride % 8 == 0 && ldw >= k && ldp >= k && pstride >= n * ldp,
              CV3_EINVAL, "bfloat16 planes need K %% 8 == 0 and 16-byte aligned rows");
  const int64_t total = n * (k / 8);
  if (total == 0) return CV3_OK;
  const int64_t blocks = ceil_div(total, 256) < 65536 ? ceil_div(total, 256) : 65536;
  hipLaunchKernelGGL(k_split_x3, dim3((unsigned)blocks), dim3(256), 0, st, w, n, k, ldw, planes, ldp, pstride);
  CV3_LAUNCHED();
  return CV3_OK;
}

// y[b, t, co] = epi(bias[co] + sum_{tap, c} w[co, tap, c] * x[b, t + tap - pad_l, g * cin_g + c]),
// g = co / 64: the DiT's grouped conv_pos (cv3cpu/models/dit.py:99-112) on
// channels-last activations, as an implicit GEMM on the FAST kernel.  w is the
// reference's (cout, cin_g, k) weight repacked as (cout, k, cin_g).
// The same grouped conv with the packed weight as bfloat16 planes in fragment order
// (split_x3_frag of the (cout, k * cin_g) rows): k_gemm_x3f in its conv mode.
int conv_cl_x3f(const float* x, int64_t batch, int64_t t, int64_t ldx, const uint16_t* frag, int64_t cout, int64_t k,
                int64_t cin_g, int64_t pad_l, const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi,
                hipStream_t st) {
  CV3_REQUIRE(cin_g % XBK == 0 && (k * cin_g) % (2 * XBK) == 0 && cout % BN == 0, CV3_EUNSUPPORTED,
              "channels-last conv needs cin/groups %% 32 == 0, k*cin/groups %% 64 == 0, 64 outputs per group");
  CV3_REQUIRE(((uintptr_t)x % 16 == 0) && ldx % 4 == 0 && ((uintptr_t)frag % 16 == 0), CV3_EINVAL,
              "channels-last conv operands must be 16-byte aligned");
  CV3_REQUIRE(batch * t < (1ll << 31) && pad_l >= 0 && pad_l < k, CV3_EINVAL, "bad conv geometry");
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.m = batch * t;
  p.n = cout;
  p.k = k * cin_g;
  p.bias = bias;
  p.c = y;
  p.ldc = ldy;
  p.epi = epi ? *epi : cv3_epilogue{};
  CV3_REQUIRE(!p.epi.rope_cos, CV3_EINVAL, "no rotary epilogue on a conv");
  p.conv_t = (int)t;
  p.conv_cg = (int)cin_g;
  p.conv_pad = (int)pad_l;
  const int64_t tiles_m = ceil_div(p.m, BM), tiles_n = cout / BN;
  const int gm = tile_group(tiles_m, tiles_n, 4.0 * (double)p.m * p.k, 6.0 * (double)cout * p.k);
  hipLaunchKernelGGL(k_gemm_x3f<A_CONV>, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st, p,
                     reinterpret_cast<const uint4*>(frag), x3_frag_plane(cout, p.k) / 8, (int)tiles_m, (int)tiles_n,
                     gm);
  CV3_LAUNCHED();
  return CV3_OK;
}

int conv_cl(const float* x, int64_t batch, int64_t t, int64_t ldx, const float* w, int64_t cout, int64_t k,
            int64_t cin_g, int64_t pad_l, const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi,
            hipStream_t st) {
  CV3_REQUIRE(cin_g % BK == 0 && (k * cin_g) % (2 * BK) == 0 && cout % BN == 0, CV3_EUNSUPPORTED,
              "channels-last conv needs cin/groups %% 32 == 0, k*cin/groups %% 64 == 0, 64 outputs per group");
  CV3_REQUIRE(((uintptr_t)x % 16 == 0) && ldx % 4 == 0 && ((uintptr_t)w % 16 == 0), CV3_EINVAL,
              "channels-last conv operands must be 16-byte aligned");
  CV3_REQUIRE(batch * t < (1ll << 31) && pad_l >= 0 && pad_l < k, CV3_EINVAL, "bad conv geometry");
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.b = w;
  p.ldb = k * cin_g;
  p.m = batch * t;
  p.n = cout;
  p.k = k * cin_g;
  p.bias = bias;
  p.c = y;
  p.ldc = ldy;
  p.epi = epi ? *epi : cv3_epilogue{};
  p.conv_t = (int)t;
  p.conv_cg = (int)cin_g;
  p.conv_pad = (int)pad_l;
  const int64_t tiles_m = ceil_div(p.m, BM), tiles_n = cout / BN;
  if (tiles_m * tiles_n <= 256)
    hipLaunchKernelGGL((k_gemm8<B_F32, A_CONV>), dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, st, p,
                       (int)tiles_m);
  else
    hipLaunchKernelGGL((k_gemm<B_F32, true, A_CONV>), dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st, p, 1,
                       1, (int)tiles_m, 0);
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // namespace cv3
