// Scaled dot-product attention (cv3cpu/ops.py:244-310) on strided q/k/v.
//
//   out[b, h, n, :] = softmax_m((q[b, h, n] * scale) . k[b, h', m]  + mask) . v[b, h', m]
//   with h' = h / (H / Hk) (grouped-query attention, ops.py:279-283) and masks
//   none / ("causal", offset) / ("chunk", size, left) (ops.py:244-264).
//
// The reference takes one ordinary softmax per query tile; here the softmax is
// streamed over key tiles (online max/sum rescaling), which changes only
// rounding.  The head_dim == 64 path runs on the matrix cores with
// v_mfma_f32_16x16x4_f32.  It computes S^T = K . Q^T so that each lane's
// accumulator registers already hold P^T in the B-operand layout of the next
// MFMA, O^T += V^T . P^T: no LDS round trip for the probabilities.
#include "bf16x3.hpp"
#include "common.hpp"

using namespace cv3;

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct AttnParams {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t q_sb, q_sh, q_sn;
  int64_t k_sb, k_sh, k_sm;
  int64_t v_sb, v_sh, v_sm;
  int64_t o_sb, o_sh, o_sn;
  int h, hk;
  int64_t n, m;
  int d;
  float scale;
  int mask_kind;  // 0 none, 1 causal(a = offset), 2 chunk(a = size, b = left)
  int64_t mask_a, mask_b;
};

// Every mask spec leaves query qi an interval of visible keys [lo, hi):
//   none  -> [0, m);   ("causal", a) -> [0, qi + a + 1);
//   ("chunk", size, left) -> [max((qi/size - left) * size, 0), (qi/size + 1) * size), left < 0: from 0.
// (ops.py:244-264.)  Computed once per query, applied with selects.
__device__ __forceinline__ void visible_keys(const AttnParams& p, int64_t qi, int64_t& lo, int64_t& hi) {
  lo = 0;
  hi = p.m;
  if (p.mask_kind == 1) {
    hi = min(hi, qi + p.mask_a + 1);
  } else if (p.mask_kind == 2) {
    const int64_t c = qi / p.mask_a;
    hi = min(hi, (c + 1) * p.mask_a);
    if (p.mask_b >= 0) lo = max((int64_t)0, (c - p.mask_b) * p.mask_a);
  }
}

constexpr int KT = 64;        // keys per LDS tile
constexpr float kLog2E = 1.4426950408889634f;
constexpr int KS = 68;        // LDS row stride (floats) for K and V tiles
constexpr int QW = 16;        // queries per wave
constexpr int QT = 64;        // queries per workgroup

// 4 * NKG waves: wave w takes queries (w % 4) * 16 .. +15 of the workgroup's 64 and
// key group kg = w / 4.  Each stage stages NKG tiles of 64 keys; key group kg works
// on tile NKG * stage + kg, so every SIMD runs NKG waves (one per key group) and the
// key range is split between them.  Each wave keeps its own online softmax
// (max, sum, output) and the groups merge in LDS at the end:
//   M = max_g m_g, l = sum_g l_g e^{m_g-M}, o = sum_g o_g e^{m_g-M}.
// NKG = 4 (1024 threads, 139 KB of LDS) hides the per-tile latency chain better on
// long key ranges (1024 keys and up); shorter ones keep NKG = 2.
// Per tile a wave scores all 64 keys (64 MFMAs), rescales its running state once,
// then accumulates P V (64 MFMAs).  V is staged transposed ([dim][key]) so the
// P V operands of four consecutive keys are one 16-byte LDS read.
// Scores are kept in base-2 units: q is scaled by log2(e) after the reference's
// (q * scale), so every exponential is one v_exp_f32 (2^x) instead of an expf
// range reduction; e^{s - m} = 2^{s log2 e - m log2 e}, to within a few ulp.
//
// The grid is one-dimensional, nq query tiles x h heads x batch.  Workgroup w runs on XCD w % 8
// (round-robin dispatch), and each XCD has its own L2: when the tile count divides by 8, XCD x
// takes the x-th eighth of the tiles in (batch, head)-major order, so each head's K / V rows
// are fetched into one L2 and re-read from there by that head's query tiles (otherwise every
// XCD would hold a query tile of every head and fetch all of K / V).
template <int NKG>
__global__ __launch_bounds__(256 * NKG) void k_flash64(AttnParams p, int nq) {
  __shared__ float Ks[NKG][KT * KS];
  __shared__ float Vs[NKG][KT * KS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qw = wave & 3, kg = wave >> 2;
  const int ntiles = (int)gridDim.x;
  const int wg = (int)blockIdx.x;
  const int tile = (ntiles & 7) == 0 ? (wg & 7) * (ntiles >> 3) + (wg >> 3) : wg;
  const int qt = tile % nq, bh = tile / nq;
  const int b = bh / p.h, hq = bh % p.h;
  const int hkv = hq / (p.h / p.hk);
  const int64_t q0 = (int64_t)qt * QT + qw * QW;
  const int c16 = lane & 15, g = lane >> 4;
  const int64_t qi = q0 + c16;
  const bool qvalid = qi < p.n;
  int64_t klo64, khi64;
  visible_keys(p, qi, klo64, khi64);
  const int klo = (int)klo64, khi = (int)khi64;  // the host bounds m below 2^31 - 64

  // Q fragments, pre-scaled like the reference's (q * scale) (ops.py:292)
  f32x4 qf[4];
  const float* qrow = p.q + b * p.q_sb + hq * p.q_sh + (qvalid ? qi : 0) * p.q_sn;
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) {
    const float4 t = qvalid ? *reinterpret_cast<const float4*>(qrow + s4 * 16 + g * 4) : make_float4(0, 0, 0, 0);
    qf[s4] = f32x4{(t.x * p.scale) * kLog2E, (t.y * p.scale) * kLog2E, (t.z * p.scale) * kLog2E,
                   (t.w * p.scale) * kLog2E};
  }

  f32x4 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  const float* kbase = p.k + b * p.k_sb + hkv * p.k_sh;
  const float* vbase = p.v + b * p.v_sb + hkv * p.v_sh;
  const int64_t nstages = ceil_div(p.m, NKG * KT);
  // The next stage's NKG * 64 K/V rows are loaded into registers while the current stage
  // is computed.  Rows past m are clamped to m - 1 (always in bounds); their scores
  // are masked to -inf below, so the loads carry no predicates.
  // K: thread -> tile tid/256, keys (tid%256)/16 + 16r (r < 4), dims (tid%16)*4 .. +3.
  // V: thread -> tile tid/256, key tid%64, dims ((tid/64)%4)*16 .. +15, so the transposed
  // LDS stores of one wave hit 64 consecutive keys of a dim row.
  const int ltile = tid >> 8, lkey = (tid & 255) >> 4, ld4 = (tid & 15) * 4;
  const int vkey = tid & 63, vd = ((tid >> 6) & 3) * 16;
  float4 k0r, k1r, k2r, k3r, v0r, v1r, v2r, v3r;
#define CV3_KV_LOAD(KOFF)                                                                        \
  {                                                                                              \
    const int64_t kb0 = (KOFF) + ltile * KT + lkey;                                              \
    const int64_t j0 = min(kb0, p.m - 1), j1 = min(kb0 + 16, p.m - 1);                           \
    const int64_t j2 = min(kb0 + 32, p.m - 1), j3 = min(kb0 + 48, p.m - 1);                      \
    k0r = *reinterpret_cast<const float4*>(kbase + j0 * p.k_sm + ld4);                           \
    k1r = *reinterpret_cast<const float4*>(kbase + j1 * p.k_sm + ld4);                           \
    k2r = *reinterpret_cast<const float4*>(kbase + j2 * p.k_sm + ld4);                           \
    k3r = *reinterpret_cast<const float4*>(kbase + j3 * p.k_sm + ld4);                           \
    const float* vr_ = vbase + min((KOFF) + ltile * KT + vkey, p.m - 1) * p.v_sm + vd;            \
    v0r = *reinterpret_cast<const float4*>(vr_);                                                 \
    v1r = *reinterpret_cast<const float4*>(vr_ + 4);                                             \
    v2r = *reinterpret_cast<const float4*>(vr_ + 8);                                             \
    v3r = *reinterpret_cast<const float4*>(vr_ + 12);                                            \
  }
  CV3_KV_LOAD((int64_t)0)
  for (int64_t st = 0; st < nstages; ++st) {
    const int k0i = (int)(st * NKG * KT + kg * KT);  // first key of this wave's tile
    __syncthreads();
    float* kt_ = Ks[ltile];
    float* vt_ = Vs[ltile];
    *reinterpret_cast<float4*>(&kt_[lkey * KS + ld4]) = k0r;
    *reinterpret_cast<float4*>(&kt_[(lkey + 16) * KS + ld4]) = k1r;
    *reinterpret_cast<float4*>(&kt_[(lkey + 32) * KS + ld4]) = k2r;
    *reinterpret_cast<float4*>(&kt_[(lkey + 48) * KS + ld4]) = k3r;
    {
      const float vv[16] = {v0r.x, v0r.y, v0r.z, v0r.w, v1r.x, v1r.y, v1r.z, v1r.w,
                            v2r.x, v2r.y, v2r.z, v2r.w, v3r.x, v3r.y, v3r.z, v3r.w};
#pragma unroll
      for (int e = 0; e < 16; ++e) vt_[(vd + e) * KS + vkey] = vv[e];
    }
    __syncthreads();
    if (st + 1 < nstages) CV3_KV_LOAD((st + 1) * NKG * KT)
    __builtin_amdgcn_sched_barrier(0);  // the prefetch is issued before this stage's math
    const float* Kt = Ks[kg];
    const float* Vt = Vs[kg];

    // S^T for the tile: sub-tile sub holds keys sub*16 + 4g + i (i < 4) for query column c16
    // the four sub-tiles' accumulators are independent: consecutive MFMAs go to different ones
    f32x4 s[KT / 16];
#pragma unroll
    for (int sub = 0; sub < KT / 16; ++sub) s[sub] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      float4 kf[KT / 16];
#pragma unroll
      for (int sub = 0; sub < KT / 16; ++sub)
        kf[sub] = *reinterpret_cast<const float4*>(&Kt[(sub * 16 + c16) * KS + g * 4 + s4 * 16]);
#pragma unroll
      for (int sub = 0; sub < KT / 16; ++sub) s[sub] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[sub].x, qf[s4].x, s[sub], 0, 0, 0);
#pragma unroll
      for (int sub = 0; sub < KT / 16; ++sub) s[sub] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[sub].y, qf[s4].y, s[sub], 0, 0, 0);
#pragma unroll
      for (int sub = 0; sub < KT / 16; ++sub) s[sub] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[sub].z, qf[s4].z, s[sub], 0, 0, 0);
#pragma unroll
      for (int sub = 0; sub < KT / 16; ++sub) s[sub] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[sub].w, qf[s4].w, s[sub], 0, 0, 0);
    }
    // copy out of the accumulators and mask with selects (no divergent writes into them)
    float sc[KT / 16][4];
    float mx = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < KT / 16; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kj = k0i + sub * 16 + 4 * g + i;
        const bool ok = kj >= klo && kj < khi;
        sc[sub][i] = ok ? s[sub][i] : -INFINITY;
        mx = fmaxf(mx, sc[sub][i]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // Branch-free so the wave-wide MFMAs below see uniform control flow: a query
    // column with nothing visible yet keeps alpha = 1 and p = 0.
    const float m_new = fmaxf(m_run, mx);
    const bool none = m_new == -INFINITY;
    const float m_use = none ? 0.f : m_new;
    const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int sub = 0; sub < KT / 16; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[sub][i] = __builtin_amdgcn_exp2f(sc[sub][i] - m_use);
        psum += sc[sub][i];
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
    // O^T += V^T P^T: the A operand of key group i is V^T[db*16 + c16][sub*16 + 4g + i]
#pragma unroll
    for (int sub = 0; sub < KT / 16; ++sub) {
      float4 vf[4];
#pragma unroll
      for (int db = 0; db < 4; ++db)
        vf[db] = *reinterpret_cast<const float4*>(&Vt[(db * 16 + c16) * KS + sub * 16 + 4 * g]);
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[db].x, sc[sub][0], oacc[db], 0, 0, 0);
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[db].y, sc[sub][1], oacc[db], 0, 0, 0);
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[db].z, sc[sub][2], oacc[db], 0, 0, 0);
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[db].w, sc[sub][3], oacc[db], 0, 0, 0);
    }
  }
#undef CV3_KV_LOAD
  // merge the key groups through LDS (each lane's state is per query column)
  __syncthreads();
  float* mb = &Ks[0][0];  // (NKG - 1) x 4 waves x 64 lanes x 18 floats <= NKG * 64 * 68
  static_assert((NKG - 1) * 4 * 64 * 18 <= NKG * KT * KS, "merge slots fit the K tiles");
  if (kg > 0) {
    float* slot = mb + (((kg - 1) * 4 + qw) * 64 + lane) * 18;
    slot[0] = m_run;
    slot[1] = l_run;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) slot[2 + db * 4 + i] = oacc[db][i];
  }
  __syncthreads();
  if (kg > 0) return;
  float M = m_run;
#pragma unroll
  for (int g2 = 1; g2 < NKG; ++g2) M = fmaxf(M, mb[(((g2 - 1) * 4 + qw) * 64 + lane) * 18]);
  const float a0 = M == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - M);
  l_run = l_run * a0;
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] *= a0;
#pragma unroll
  for (int g2 = 1; g2 < NKG; ++g2) {
    const float* slot = mb + (((g2 - 1) * 4 + qw) * 64 + lane) * 18;
    const float ag = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(slot[0] - M);
    l_run += slot[1] * ag;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[db][i] += slot[2 + db * 4 + i] * ag;
  }
  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!qvalid) return;
  float* orow = p.o + b * p.o_sb + hq * p.o_sh + qi * p.o_sn;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) orow[db * 16 + 4 * g + i] = oacc[db][i] / l_tot;
}

// The same flash attention on the bfloat16 matrix cores (v_mfma_f32_16x16x32_bf16): q, k, v
// and the probabilities split into three bfloat16 planes each (bf16x3.hpp), every product
// as the six plane products of weight >= 2^-16, hh into one accumulator and the other five
// into a second, added where the float32 kernel reads its accumulator.  Two key groups of
// four waves (one 64-key tile each per stage), 16 queries per wave, as k_flash64<2>.
//
// LDS holds each tile's planes as 64 rows of 128 bytes (8 chunks of 8 bf16, chunk c of row r
// in slot r * 8 + (c ^ (r / 2) % 8)): K as [key][dim] with key 4c + s in row 16 s + c, V^T as
// [dim][key].  Score sub-tile s (MFMA rows r = LDS rows 16 s + r) then holds keys 4 r + s, so
// lane (c16, g) ends with keys 16 g + 4 i + s (i, s < 4): the 16 consecutive keys 16 g .. + 15
// of its query column.  P V step j takes keys 16 g + 8 j + t (t < 8) from lane group g, which
// are the lane's own values sc[t % 4][2 j + t / 4] as the B operand (k index 8 g + t), and
// V^T row d, chunk 2 g + j as the A operand: no data moves between the two products.
__device__ __forceinline__ int xkv(int row, int chunk) { return row * 8 + (chunk ^ ((row >> 1) & 7)); }
// V^T rows (64 dims of 8 16-byte key chunks) of k_flash64x: chunk c of row d at slot
// (d / 2) 16 + ((8 (d % 2) + c) ^ f(d)), f(d) = 8 b5 + ((d / 2) % 8 ^ b4) with b4, b5 bits 4 and 5 of d.
// A row pair fills 16 slots (256 bytes, one bank window).  The P.V reads (16 consecutive rows, one
// chunk) and the staging writes (rows 4 q + e for q = 0..15, one chunk, 8 bytes each) both land on
// 16 distinct slots of a window.
__device__ __forceinline__ int vslot(int d, int c) {
  const int f = (((d >> 5) & 1) << 3) | (((d >> 1) & 7) ^ ((d >> 4) & 1));
  return (d >> 1) * 16 + (((d & 1) * 8 + c) ^ f);
}

__device__ __forceinline__ void mfma6(const bf16x8_t& ah, const bf16x8_t& am, const bf16x8_t& al,
                                      const bf16x8_t& bh, const bf16x8_t& bm, const bf16x8_t& bl, f32x4& big,
                                      f32x4& small) {
  big = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, big, 0, 0, 0);
  small = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bm, small, 0, 0, 0);
  small = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bh, small, 0, 0, 0);
  small = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, small, 0, 0, 0);
  small = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bm, small, 0, 0, 0);
  small = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, small, 0, 0, 0);
}

__global__ __launch_bounds__(512) void k_flash64x(AttnParams p, int nq) {
  constexpr int NKG = 2;
  __shared__ uint4 Ks[NKG][3][KT * 8];
  __shared__ uint4 Vs[NKG][3][KT * 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qw = wave & 3, kg = wave >> 2;
  const int ntiles = (int)gridDim.x;
  const int wg = (int)blockIdx.x;
  const int tile = (ntiles & 7) == 0 ? (wg & 7) * (ntiles >> 3) + (wg >> 3) : wg;
  const int qt = tile % nq, bh = tile / nq;
  const int b = bh / p.h, hq = bh % p.h;
  const int hkv = hq / (p.h / p.hk);
  const int64_t q0 = (int64_t)qt * QT + qw * QW;
  const int c16 = lane & 15, g = lane >> 4;
  const int64_t qi = q0 + c16;
  const bool qvalid = qi < p.n;
  int64_t klo64, khi64;
  visible_keys(p, qi, klo64, khi64);
  const int klo = (int)klo64, khi = (int)khi64;  // the host bounds m below 2^31 - 64

  // Q^T fragments: query c16, dims 32 ks + 8 g .. + 7, pre-scaled like the reference's
  // (q * scale) (ops.py:292), in base-2 units, as planes
  bf16x8_t qh[2], qm[2], ql[2];
  const float* qrow = p.q + b * p.q_sb + hq * p.q_sh + (qvalid ? qi : 0) * p.q_sn;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    float4 t0 = qvalid ? *reinterpret_cast<const float4*>(qrow + 32 * ks + 8 * g) : make_float4(0, 0, 0, 0);
    float4 t1 = qvalid ? *reinterpret_cast<const float4*>(qrow + 32 * ks + 8 * g + 4) : make_float4(0, 0, 0, 0);
    t0 = make_float4((t0.x * p.scale) * kLog2E, (t0.y * p.scale) * kLog2E, (t0.z * p.scale) * kLog2E,
                     (t0.w * p.scale) * kLog2E);
    t1 = make_float4((t1.x * p.scale) * kLog2E, (t1.y * p.scale) * kLog2E, (t1.z * p.scale) * kLog2E,
                     (t1.w * p.scale) * kLog2E);
    uint4 h4, m4, l4;
    split_x3(t0, t1, h4, m4, l4);
    qh[ks] = __builtin_bit_cast(bf16x8_t, h4);
    qm[ks] = __builtin_bit_cast(bf16x8_t, m4);
    ql[ks] = __builtin_bit_cast(bf16x8_t, l4);
  }

  f32x4 ob[4], os[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) ob[db] = os[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  const float* kbase = p.k + b * p.k_sb + hkv * p.k_sh;
  const float* vbase = p.v + b * p.v_sb + hkv * p.v_sh;
  const int64_t nstages = ceil_div(p.m, NKG * KT);
  // Staging (next stage's rows in registers while this one is computed; rows past m clamp
  // to m - 1 and are masked to -inf below):
  // K: thread -> tile tid/256, key (tid%256)/4, dims 16 (tid%4) .. + 15 (two chunks);
  // V: thread -> tile tid/256, keys 4 kq .. + 3 (kq = (tid%256)/16), dims 4 dq .. + 3 (dq = tid%16):
  //    each dim's four keys are one 8-byte half-chunk of a V^T row.
  const int ltile = tid >> 8, lkey = (tid & 255) >> 2, ld16 = (tid & 3) * 16;
  const int lrow = (lkey & 3) * 16 + (lkey >> 2);
  const int dq = tid & 15, kq = (tid & 255) >> 4;
  float4 kr[4], vv[4];
#define CV3_KVX_LOAD(KOFF)                                                                 \
  {                                                                                        \
    const int64_t jk = min((KOFF) + ltile * KT + lkey, p.m - 1);                           \
    const float* kr_ = kbase + jk * p.k_sm + ld16;                                         \
    kr[0] = *reinterpret_cast<const float4*>(kr_);                                         \
    kr[1] = *reinterpret_cast<const float4*>(kr_ + 4);                                     \
    kr[2] = *reinterpret_cast<const float4*>(kr_ + 8);                                     \
    kr[3] = *reinterpret_cast<const float4*>(kr_ + 12);                                    \
    _Pragma("unroll") for (int r_ = 0; r_ < 4; ++r_) {                                     \
      const int64_t jv = min((KOFF) + ltile * KT + 4 * kq + r_, p.m - 1);                  \
      vv[r_] = *reinterpret_cast<const float4*>(vbase + jv * p.v_sm + 4 * dq);             \
    }                                                                                      \
  }
  CV3_KVX_LOAD((int64_t)0)
  for (int64_t st = 0; st < nstages; ++st) {
    const int k0i = (int)(st * NKG * KT + kg * KT);  // first key of this wave's tile
    __syncthreads();
    {
      uint4 h4, m4, l4;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        split_x3(kr[2 * half], kr[2 * half + 1], h4, m4, l4);
        const int slot = xkv(lrow, (ld16 >> 3) + half);
        Ks[ltile][0][slot] = h4;
        Ks[ltile][1][slot] = m4;
        Ks[ltile][2][slot] = l4;
      }
      const float vr[4][4] = {{vv[0].x, vv[0].y, vv[0].z, vv[0].w}, {vv[1].x, vv[1].y, vv[1].z, vv[1].w},
                              {vv[2].x, vv[2].y, vv[2].z, vv[2].w}, {vv[3].x, vv[3].y, vv[3].z, vv[3].w}};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint2 hh, mm, ll;
        split_x3(vr[0][e], vr[1][e], hh.x, mm.x, ll.x);  // keys 4 kq, 4 kq + 1
        split_x3(vr[2][e], vr[3][e], hh.y, mm.y, ll.y);  // keys 4 kq + 2, 4 kq + 3
        const int sl = vslot(4 * dq + e, kq >> 1);
        reinterpret_cast<uint2*>(&Vs[ltile][0][sl])[kq & 1] = hh;
        reinterpret_cast<uint2*>(&Vs[ltile][1][sl])[kq & 1] = mm;
        reinterpret_cast<uint2*>(&Vs[ltile][2][sl])[kq & 1] = ll;
      }
    }
    __syncthreads();
    if (st + 1 < nstages) CV3_KVX_LOAD((st + 1) * NKG * KT)
    __builtin_amdgcn_sched_barrier(0);  // the prefetch is issued before this stage's math

    // S^T sub-tiles: sub-tile s holds keys 4 r + s in MFMA row r; k = dims
    f32x4 sb[4], ss[4];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) sb[sub] = ss[sub] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        const int slot = xkv(sub * 16 + c16, 4 * ks + g);
        const bf16x8_t kh = __builtin_bit_cast(bf16x8_t, Ks[kg][0][slot]);
        const bf16x8_t km = __builtin_bit_cast(bf16x8_t, Ks[kg][1][slot]);
        const bf16x8_t kl = __builtin_bit_cast(bf16x8_t, Ks[kg][2][slot]);
        mfma6(kh, km, kl, qh[ks], qm[ks], ql[ks], sb[sub], ss[sub]);
      }
    }
    // lane (c16, g): sc[s][i] = score of key k0i + 16 g + 4 i + s for query c16; a tile that every
    // query of the wave sees whole skips the per-key selects
    float sc[4][4];
    float mx = -INFINITY;
    if (__all(k0i >= klo && k0i + KT <= khi)) {
#pragma unroll
      for (int sub = 0; sub < 4; ++sub)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[sub][i] = sb[sub][i] + ss[sub][i];
          mx = fmaxf(mx, sc[sub][i]);
        }
    } else {
#pragma unroll
      for (int sub = 0; sub < 4; ++sub)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kj = k0i + 16 * g + 4 * i + sub;
          const bool ok = kj >= klo && kj < khi;
          sc[sub][i] = ok ? sb[sub][i] + ss[sub][i] : -INFINITY;
          mx = fmaxf(mx, sc[sub][i]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const bool none = m_new == -INFINITY;
    const float m_use = none ? 0.f : m_new;
    const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[sub][i] = __builtin_amdgcn_exp2f(sc[sub][i] - m_use);
        psum += sc[sub][i];
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      ob[db] *= alpha;
      os[db] *= alpha;
    }
    // O^T += V^T P^T over keys 16 g + 8 j + t: P^T's B operand is the lane's own values
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float4 p0 = make_float4(sc[0][2 * j], sc[1][2 * j], sc[2][2 * j], sc[3][2 * j]);
      const float4 p1 = make_float4(sc[0][2 * j + 1], sc[1][2 * j + 1], sc[2][2 * j + 1], sc[3][2 * j + 1]);
      uint4 h4, m4, l4;
      split_x3(p0, p1, h4, m4, l4);
      const bf16x8_t ph = __builtin_bit_cast(bf16x8_t, h4);
      const bf16x8_t pm = __builtin_bit_cast(bf16x8_t, m4);
      const bf16x8_t pl = __builtin_bit_cast(bf16x8_t, l4);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int slot = vslot(db * 16 + c16, 2 * g + j);
        const bf16x8_t vh = __builtin_bit_cast(bf16x8_t, Vs[kg][0][slot]);
        const bf16x8_t vm = __builtin_bit_cast(bf16x8_t, Vs[kg][1][slot]);
        const bf16x8_t vl = __builtin_bit_cast(bf16x8_t, Vs[kg][2][slot]);
        mfma6(vh, vm, vl, ph, pm, pl, ob[db], os[db]);
      }
    }
  }
#undef CV3_KVX_LOAD
  f32x4 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = ob[db] + os[db];
  // merge the key groups through LDS, as k_flash64
  __syncthreads();
  float* mb = reinterpret_cast<float*>(&Ks[0][0][0]);
  static_assert((NKG - 1) * 4 * 64 * 18 * 4 <= (int)sizeof(Ks), "merge slots fit the K tiles");
  if (kg > 0) {
    float* slot = mb + (((kg - 1) * 4 + qw) * 64 + lane) * 18;
    slot[0] = m_run;
    slot[1] = l_run;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) slot[2 + db * 4 + i] = oacc[db][i];
  }
  __syncthreads();
  if (kg > 0) return;
  float M = m_run;
#pragma unroll
  for (int g2 = 1; g2 < NKG; ++g2) M = fmaxf(M, mb[(((g2 - 1) * 4 + qw) * 64 + lane) * 18]);
  const float a0 = M == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - M);
  l_run = l_run * a0;
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] *= a0;
#pragma unroll
  for (int g2 = 1; g2 < NKG; ++g2) {
    const float* slot = mb + (((g2 - 1) * 4 + qw) * 64 + lane) * 18;
    const float ag = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(slot[0] - M);
    l_run += slot[1] * ag;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[db][i] += slot[2 + db * 4 + i] * ag;
  }
  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!qvalid) return;
  float* orow = p.o + b * p.o_sb + hq * p.o_sh + qi * p.o_sn;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) orow[db * 16 + 4 * g + i] = oacc[db][i] / l_tot;
}

// Generic path for any head dim <= 256: one wave per query row, 64 keys per step.
__global__ __launch_bounds__(256) void k_attn_generic(AttnParams p) {
  extern __shared__ float qs_all[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.z, hq = blockIdx.y;
  const int hkv = hq / (p.h / p.hk);
  const int64_t qi = (int64_t)blockIdx.x * 4 + wave;
  float* qs = qs_all + wave * p.d;
  const bool qvalid = qi < p.n;
  const float* qrow = p.q + b * p.q_sb + hq * p.q_sh + (qvalid ? qi : 0) * p.q_sn;
  for (int d = lane; d < p.d; d += 64) qs[d] = qvalid ? qrow[d] * p.scale : 0.f;
  __syncthreads();
  if (!qvalid) return;
  const float* kbase = p.k + b * p.k_sb + hkv * p.k_sh;
  const float* vbase = p.v + b * p.v_sb + hkv * p.v_sh;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  int64_t klo, khi;
  visible_keys(p, qi, klo, khi);
  for (int64_t c0 = 0; c0 < p.m; c0 += 64) {
    const int64_t kj = c0 + lane;
    float s = -INFINITY;
    if (kj >= klo && kj < khi) {
      const float* kr = kbase + kj * p.k_sm;
      float t = 0.f;
      for (int d = 0; d < p.d; ++d) t = fmaf(qs[d], kr[d], t);
      s = t;
    }
    const float mx = wave_max(s);
    const float m_new = fmaxf(m_run, mx);
    if (m_new == -INFINITY) continue;
    const float alpha = expf(m_run - m_new);
    const float pj = expf(s - m_new);
    l_run = l_run * alpha + wave_sum(pj);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] *= alpha;
    const int64_t cnt = p.m - c0 < 64 ? p.m - c0 : 64;
    for (int jj = 0; jj < cnt; ++jj) {
      const float pb = __shfl(pj, jj, 64);
      const float* vr = vbase + (c0 + jj) * p.v_sm;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = lane + 64 * r;
        if (d < p.d) acc[r] = fmaf(pb, vr[d], acc[r]);
      }
    }
    m_run = m_new;
  }
  float* orow = p.o + b * p.o_sb + hq * p.o_sh + qi * p.o_sn;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int d = lane + 64 * r;
    if (d < p.d) orow[d] = acc[r] / l_run;
  }
}

}  // namespace

static int attention(bool x3, const float* q, const float* k, const float* v, float* out, int64_t batch, int h,
                     int hk, int64_t n, int64_t m, int d, const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides, float scale, int mask_kind, int64_t mask_a,
                     int64_t mask_b, cv3_stream_t s) {
  CV3_REQUIRE(h > 0 && hk > 0, CV3_EINVAL, "head counts must be positive");
  CV3_REQUIRE(h % hk == 0, CV3_EINVAL, "%d query heads is not a multiple of %d kv heads", h, hk);
  CV3_REQUIRE(d > 0 && d <= 256, CV3_EUNSUPPORTED, "head dim %d not supported (max 256)", d);
  CV3_REQUIRE(mask_kind >= 0 && mask_kind <= 2, CV3_EINVAL, "unknown mask spec kind %d", mask_kind);
  CV3_REQUIRE(mask_kind != 2 || mask_a > 0, CV3_EINVAL, "chunk mask needs a positive chunk size");
  if (batch <= 0 || n <= 0) return CV3_OK;
  CV3_REQUIRE(m > 0, CV3_EINVAL, "attention over zero keys");
  AttnParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = out;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_sn = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_sm = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_sm = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_sn = o_strides[2];
  p.h = h;
  p.hk = hk;
  p.n = n;
  p.m = m;
  p.d = d;
  p.scale = scale;
  p.mask_kind = mask_kind;
  p.mask_a = mask_a;
  p.mask_b = mask_b;
  hipStream_t st = stream_of(s);
  const bool aligned16 = ((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0) &&
                         (p.q_sb % 4 == 0) && (p.q_sh % 4 == 0) && (p.q_sn % 4 == 0) && (p.k_sb % 4 == 0) &&
                         (p.k_sh % 4 == 0) && (p.k_sm % 4 == 0) && (p.v_sb % 4 == 0) && (p.v_sh % 4 == 0) &&
                         (p.v_sm % 4 == 0);
  if (d == 64 && aligned16) {
    CV3_REQUIRE(m < (1ll << 31) - 4 * 64, CV3_EUNSUPPORTED, "attention over 2^31 keys or more");
    const int64_t nq = ceil_div(n, QT);
    CV3_REQUIRE(nq * h * batch < (int64_t)1 << 31, CV3_EUNSUPPORTED, "attention grid too large");
    const dim3 grid((unsigned)(nq * h * batch));
    if (x3)
      hipLaunchKernelGGL(k_flash64x, grid, dim3(512), 0, st, p, (int)nq);
    else if (m >= 16 * KT)  // 1024 keys and up: 8 % faster at 1500 keys, no gain at 500
      hipLaunchKernelGGL(k_flash64<4>, grid, dim3(1024), 0, st, p, (int)nq);
    else
      hipLaunchKernelGGL(k_flash64<2>, grid, dim3(512), 0, st, p, (int)nq);
  } else {
    const dim3 grid((unsigned)ceil_div(n, 4), (unsigned)h, (unsigned)batch);
    hipLaunchKernelGGL(k_attn_generic, grid, dim3(256), 4 * d * sizeof(float), st, p);
  }
  CV3_LAUNCHED();
  return CV3_OK;
}

extern "C" int cv3_attention(const float* q, const float* k, const float* v, float* out, int64_t batch, int h,
                             int hk, int64_t n, int64_t m, int d, const int64_t* q_strides,
                             const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
                             float scale, int mask_kind, int64_t mask_a, int64_t mask_b, cv3_stream_t s) {
  CV3_ALIVE();
  return attention(false, q, k, v, out, batch, h, hk, n, m, d, q_strides, k_strides, v_strides, o_strides, scale,
                   mask_kind, mask_a, mask_b, s);
}

extern "C" int cv3_attention_x3(const float* q, const float* k, const float* v, float* out, int64_t batch, int h,
                                int hk, int64_t n, int64_t m, int d, const int64_t* q_strides,
                                const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
                                float scale, int mask_kind, int64_t mask_a, int64_t mask_b, cv3_stream_t s) {
  CV3_ALIVE();
  return attention(true, q, k, v, out, batch, h, hk, n, m, d, q_strides, k_strides, v_strides, o_strides, scale,
                   mask_kind, mask_a, mask_b, s);
}
