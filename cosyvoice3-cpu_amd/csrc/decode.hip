// Qwen2 single-token decode step, resident on the device (cv3cpu/models/qwen2.py:139-179,
// cv3cpu/models/llm.py:68-77,112-123 with greedy selection).
//
// One token costs 5 kernels per layer plus 2 at the end, all enqueued by
// cv3_qwen2_decode_step so the whole step can be captured into one HIP graph and
// replayed: the position and the last token live in device memory, so every
// token's launch sequence is identical.
//
//   per layer
//     qkv   : RMSNorm prologue -> int8 GEMV of [q; k; v] + bias -> half-split
//             rotary on q and k -> k, v appended to the cache at `pos`
//     attn  : GQA decode attention over keys [0, pos], split over key chunks;
//             the last workgroup of each kv head merges the chunks
//     o     : int8 GEMV, x += W_o . attn
//     mlp   : RMSNorm prologue -> int8 GEMV of [gate; up] -> silu(gate) * up
//     down  : int8 GEMV, x += W_down . h
//   end
//     head  : final RMSNorm prologue -> int8 GEMV + bias -> logits
//     next  : argmax (ties to the lowest index, np.argsort(-p, stable)[0]),
//             history[pos + 1] = id, x = speech_embedding[id], pos += 1
//
// The quantised GEMV (the HBM-bound part, cv3cpu/quant.py:172-204 at m = 1): a row
// group of LPR lanes owns one weight row; each lane streams CPL 16-byte chunks
// of it (128 contiguous bytes per 8 lanes), issued before the activation vector
// is staged into LDS so the two memory latencies overlap.  Codes are widened in
// registers; per-row float32 scales are applied once after the dot product,
// block float16 scales once per chunk (a chunk never straddles a block).
// A chunk holds 16 int8 codes (q8, block % 16 == 0) or one 32-code q4 block of
// packed nibbles (byte j: code j in the low nibble, code j + 16 in the high one,
// stored +8; quant.py:70-86,123-131), so the tiny profile's body layers stream
// half the bytes through the same kernels.
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "decode_common.hpp"
#include "epilogue.hpp"

using namespace cv3;

namespace {


// Chunk dot products.  q8: 16 int8 codes, each sign-extended from its byte.
// q4: one 32-code block; word d holds codes 4d..4d+3 in its low nibbles and
// 16+4d..16+4d+3 in its high nibbles, each stored + 8.  Flipping bit 3 of a
// nibble n gives the 4-bit two's complement of n - 8 (n ^ 8 = n - 8 for n >= 8,
// n + 8 = (n - 8) + 16 below); moved to the top of a byte it reads as the int8
// 16 * (n - 8), so both nibble sets widen like q8 bytes and dot32_q4 returns
// 16 x the chunk's dot product (the caller scales by 1/16, exactly).
__device__ __forceinline__ float sext(uint32_t u, int lsb, int bits) {
  return (float)((int32_t)(u << (32 - lsb - bits)) >> (32 - bits));
}

__device__ __forceinline__ float dot32_q4(const u32x4 v, const float* __restrict__ xs) {
  const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
  float a = 0.f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float4 xl = *reinterpret_cast<const float4*>(xs + 4 * d);
    const float4 xh = *reinterpret_cast<const float4*>(xs + 16 + 4 * d);
    const uint32_t u = ws[d] ^ 0x88888888u;
    const uint32_t lo = (u << 4) & 0xF0F0F0F0u, hi = u & 0xF0F0F0F0u;
    a = fmaf(sext(lo, 0, 8), xl.x, a);
    a = fmaf(sext(lo, 8, 8), xl.y, a);
    a = fmaf(sext(lo, 16, 8), xl.z, a);
    a = fmaf(sext(lo, 24, 8), xl.w, a);
    a = fmaf(sext(hi, 0, 8), xh.x, a);
    a = fmaf(sext(hi, 8, 8), xh.y, a);
    a = fmaf(sext(hi, 16, 8), xh.z, a);
    a = fmaf(sext(hi, 24, 8), xh.w, a);
  }
  return a;
}

__device__ __forceinline__ float dot16(const u32x4 v, const float* __restrict__ xs) {
  const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
  float a = 0.f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float4 xv = *reinterpret_cast<const float4*>(xs + 4 * d);
    const uint32_t u = ws[d];
    a = fmaf(sext(u, 0, 8), xv.x, a);
    a = fmaf(sext(u, 8, 8), xv.y, a);
    a = fmaf(sext(u, 16, 8), xv.z, a);
    a = fmaf(sext(u, 24, 8), xv.w, a);
  }
  return a;
}

// Stage x[0:k) into LDS (zero padded to kx), optionally RMS-normalised with weight
// rms_w: x * (1 / sqrt(mean(x^2) + eps)) * w (cv3cpu/ops.py:101-104).
// load() issues every float4 load of this thread at once (NV per thread, clamped
// indices, no predicates); kernels call it BEFORE issuing their weight stream,
// because loads complete in issue order: a vector loaded after the weights would
// wait for all of them.  finish_folded() writes LDS and synchronises.
// Needs k % 4 == 0 and 16-byte aligned x / rms_w.
template <int NV>
struct VecStage {
  float4 v[NV], w[NV];
  __device__ __forceinline__ void load(const float* __restrict__ x, int64_t k, const float* __restrict__ rms_w) {
    const int64_t k4 = k / 4;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* w4 = reinterpret_cast<const float4*>(rms_w ? rms_w : x);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t idx = min((int64_t)threadIdx.x + (int64_t)i * blockDim.x, k4 - 1);
      v[i] = x4[idx];
      w[i] = w4[idx];
    }
  }
  // Stage with the norm folded out of the vector: xs = x * w, and the returned
  // 1 / sqrt(mean(x^2) + eps) scales each row's dot product afterwards
  // (W . (x * inv * w) = inv * (W . (x * w))).  The statistic's cross-wave sum rides on
  // the staging barrier, so the dot products do not wait for a reduction.
  __device__ __forceinline__ float finish_folded(int64_t k, int64_t kx, bool rms, float eps, float* xs, float* red) {
    const int64_t k4 = k / 4, n4 = kx / 4;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t idx = threadIdx.x + (int64_t)i * blockDim.x;
      if (idx >= k4) v[i] = z;
    }
    float ss = 0.f;
    if (rms) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        ss = fmaf(v[i].x, v[i].x, ss);
        ss = fmaf(v[i].y, v[i].y, ss);
        ss = fmaf(v[i].z, v[i].z, ss);
        ss = fmaf(v[i].w, v[i].w, ss);
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t idx = threadIdx.x + (int64_t)i * blockDim.x;
      float4 o = v[i];
      if (rms) {
        o.x = o.x * w[i].x;
        o.y = o.y * w[i].y;
        o.z = o.z * w[i].z;
        o.w = o.w * w[i].w;
      }
      if (idx < n4) reinterpret_cast<float4*>(xs)[idx] = o;
    }
    if (rms) {
      ss = wave_sum(ss);
      if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    if (!rms) return 1.f;
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
    return 1.0f / sqrtf(t / (float)k + eps);
  }
};

// Codes per 16-byte chunk.
template <bool Q4>
constexpr int kCodes = Q4 ? 32 : 16;

// Dot products of one row group: lanes [g*LPR, g*LPR + LPR) cover row `row`.
// load() issues the lane's CPL 16-byte chunks and their scales (one per chunk: the
// per-row layout repeats the row's scale) with no predicates; dot() consumes them.
// Chunks past the row are clamped to its last chunk and meet the zero padding of
// the staged vector (xs is zero from K up to LPR * CPL * kCodes), so they add
// exactly 0 (q4: (n - 8) * 0); nothing selects on a loaded value, which would wait
// for the load right there.
// A dead row group (`row` clamped to a valid row) computes a value nobody stores.
template <int LPR, int CPL, bool SF16, bool Q4>
struct RowDot {
  static constexpr int CPC = kCodes<Q4>;
  u32x4 wv[CPL];
  float sc[CPL];
  __device__ __forceinline__ void load(const QW& w, int64_t row, int sub, bool /*live*/) {
    const int64_t row_bytes = Q4 ? w.kp / 2 : w.kp;
    const u32x4* base = reinterpret_cast<const u32x4*>(w.q + row * row_bytes);
    const int nch = (int)(row_bytes / 16);
    const unsigned cpb = (unsigned)(w.block / CPC);
    const int64_t srow = row * (w.kp / w.block);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = min(sub + i * LPR, nch - 1);
      wv[i] = __builtin_nontemporal_load(base + c);
      const int64_t si = srow + (int64_t)((unsigned)c / cpb);
      if constexpr (SF16)
        sc[i] = __half2float(reinterpret_cast<const __half*>(w.scales)[si]);
      else
        sc[i] = reinterpret_cast<const float*>(w.scales)[si];
    }
  }
  // full row dot product, reduced over the row group (every lane of the group gets it)
  __device__ __forceinline__ float dot(const float* xs, int sub) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const float* xc = xs + (sub + i * LPR) * CPC;
      acc = fmaf(Q4 ? dot32_q4(wv[i], xc) : dot16(wv[i], xc), sc[i], acc);
    }
    if (Q4) acc *= 0.0625f;
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    return acc;
  }
};

// A q4 row of the one-launch step over 64 lanes, half a 32-code block per lane (16 codes, the
// per-lane work of a q8 chunk): lane l holds bytes 8 (l % 2) .. + 7 of block l / 2, i.e. codes
// 8 (l % 2) .. + 7 in their low nibbles and 16 + 8 (l % 2) .. + 7 in their high ones (each
// stored + 8, quant.py:70-86,123-131), and its block's scale.  Halves past the row are clamped
// to its last half and meet the zero padding of the staged vector.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <bool SF16>
struct RowQ4H {
  u32x2 wv;
  float sc;
  __device__ __forceinline__ void load(const QW& w, int64_t row, int lane, bool /*live*/) {
    const int64_t row_bytes = w.kp / 2;
    const u32x2* base = reinterpret_cast<const u32x2*>(w.q + row * row_bytes);
    const int c = min(lane, (int)(row_bytes / 8) - 1);
    wv = __builtin_nontemporal_load(base + c);
    const int64_t si = row * (w.kp / w.block) + (int64_t)((unsigned)(c >> 1) / (unsigned)(w.block / 32));
    if constexpr (SF16)
      sc = __half2float(reinterpret_cast<const __half*>(w.scales)[si]);
    else
      sc = reinterpret_cast<const float*>(w.scales)[si];
  }
};
// 16 x the dot of a half block with its 16 staged values: xs[0..7] meet the low nibbles,
// xs[8..15] the high ones (widened as in dot32_q4).
__device__ __forceinline__ float dot16_q4h(const u32x2 v, const float* __restrict__ xs) {
  const uint32_t ws[2] = {v.x, v.y};
  float a = 0.f;
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const float4 xl = *reinterpret_cast<const float4*>(xs + 4 * d);
    const float4 xh = *reinterpret_cast<const float4*>(xs + 8 + 4 * d);
    const uint32_t u = ws[d] ^ 0x88888888u;
    const uint32_t lo = (u << 4) & 0xF0F0F0F0u, hi = u & 0xF0F0F0F0u;
    a = fmaf(sext(lo, 0, 8), xl.x, a);
    a = fmaf(sext(lo, 8, 8), xl.y, a);
    a = fmaf(sext(lo, 16, 8), xl.z, a);
    a = fmaf(sext(lo, 24, 8), xl.w, a);
    a = fmaf(sext(hi, 0, 8), xh.x, a);
    a = fmaf(sext(hi, 8, 8), xh.y, a);
    a = fmaf(sext(hi, 16, 8), xh.z, a);
    a = fmaf(sext(hi, 24, 8), xh.w, a);
  }
  return a;
}

// ---------------------------------------------------------------------------
// Generic GEMV y = epi(W . vec): 256 threads, RPW = 64 / LPR rows per wave.
//   mode 0: y[r] = acc + bias[r]             (head)
//   mode 1: y[r] = y[r] + acc                (o / down: residual add, in place)
//   mode 2: y[r] = silu(acc_gate) * acc_up   (gate rows r, up rows r + n)
// ---------------------------------------------------------------------------
struct GemvArgs {
  QW w;
  int64_t layer_row0;   // first weight row of this layer (layer * rows)
  int64_t n;            // outputs
  const float* x;
  const float* rms_w;
  float eps;
  const float* bias;
  float* y;
  int mode;
};

template <int LPR, int CPL, int MODE, bool SF16, bool Q4>
__global__ __launch_bounds__(256) void k_dec_gemv(GemvArgs a) {
  extern __shared__ float xs[];
  __shared__ float red[4];
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPR, sub = lane % LPR;
  constexpr bool swiglu = MODE == 2;
  // output column handled by this row group
  const int64_t outs_per_wave = swiglu ? RPW / 2 : RPW;
  const int64_t col = ((int64_t)blockIdx.x * 4 + wave) * outs_per_wave + (swiglu ? grp / 2 : grp);
  const bool live = col < a.n;
  const int64_t wrow = a.layer_row0 + (swiglu ? ((grp & 1) ? col + a.n : col) : col);
  constexpr int WIDTH = LPR * CPL * kCodes<Q4>;  // staged (zero-padded) vector length
  VecStage<(WIDTH / 4 + 255) / 256> vs;
  vs.load(a.x, a.w.k, a.rms_w);
  const float yres = MODE == 1 ? a.y[live ? col : 0] : 0.f;
  __builtin_amdgcn_sched_barrier(0);  // the vector's loads go out before the weight stream
  RowDot<LPR, CPL, SF16, Q4> rd;
  rd.load(a.w, live ? wrow : a.layer_row0, sub, live);
  __builtin_amdgcn_sched_barrier(0);
  const float inv = vs.finish_folded(a.w.k, WIDTH, a.rms_w != nullptr, a.eps, xs, red);
  const float acc = rd.dot(xs, sub) * inv;
  if (swiglu) {
    const float up = __shfl_xor(acc, LPR, 64);  // partner row group (gate <-> up)
    if (live && sub == 0 && (grp & 1) == 0) a.y[col] = (acc / (1.0f + expf(-acc))) * up;
  } else if (live && sub == 0) {
    if constexpr (MODE == 1)
      a.y[col] = yres + acc;
    else
      a.y[col] = acc + (a.bias ? a.bias[col] : 0.f);
  }
}

// ---------------------------------------------------------------------------
// QKV: RMSNorm prologue, GEMV of the stacked [q; k; v] rows (+ bias), half-split
// rotary on q and k (qwen2.py:64-71), k and v written to the cache at `pos`.
// A wave owns 4 rotary pairs (rows h*64 + j and h*64 + 32 + j), LPR = 8.
// ---------------------------------------------------------------------------
struct QkvArgs {
  QW w;
  int64_t layer_row0;
  const float* x;
  const float* rms_w;
  float eps;
  const float* bias;       // layer's [q; k; v] bias
  int heads, kv_heads, dh;
  const float* cos_t;      // [cap, dh]
  const float* sin_t;
  const int64_t* pos;
  float* q_out;            // [heads * dh]
  float* k_cache;          // layer's [kv_heads, cap, dh]
  float* v_cache;
  int64_t cap;
};

template <int CPL, bool SF16, bool Q4>
__global__ __launch_bounds__(256) void k_dec_qkv(QkvArgs a) {
  extern __shared__ float xs[];
  __shared__ float red[4];
  constexpr int LPR = 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPR, sub = lane % LPR;
  const int half = a.dh / 2;
  const int64_t nrows = (int64_t)(a.heads + 2 * a.kv_heads) * a.dh;
  // pair index p covers rows (head, j) and (head, j + half); 4 pairs per wave
  const int64_t pair = ((int64_t)blockIdx.x * 4 + wave) * 4 + grp / 2;
  const int64_t head = pair / half, j = pair % half;
  const bool live = head * a.dh < nrows;
  const int64_t r = head * a.dh + j + ((grp & 1) ? half : 0);
  const int64_t wrow = a.layer_row0 + (live ? r : 0);
  const int64_t p = *a.pos;  // issued first: the rotary tables depend on it
  constexpr int WIDTH = LPR * CPL * kCodes<Q4>;
  VecStage<(WIDTH / 4 + 255) / 256> vs;
  vs.load(a.x, a.w.k, a.rms_w);
  __builtin_amdgcn_sched_barrier(0);
  RowDot<LPR, CPL, SF16, Q4> rd;
  rd.load(a.w, wrow, sub, live);
  const float bias = a.bias[live ? r : 0];
  __builtin_amdgcn_sched_barrier(0);
  // the row's rotary table entries: they wait for `pos`, so they go out after the
  // weight stream and arrive while the RMSNorm and the dot product run
  const bool upper = grp & 1;
  const int jj = (int)j + (upper ? half : 0);
  const float rc = a.cos_t[p * a.dh + jj], rs = a.sin_t[p * a.dh + jj];
  const float inv = vs.finish_folded(a.w.k, WIDTH, a.rms_w != nullptr, a.eps, xs, red);
  float v = rd.dot(xs, sub) * inv;
  if (live) v += bias;
  const float other = __shfl_xor(v, LPR, 64);  // the pair partner
  if (!live || sub != 0) return;
  const int64_t nq = a.heads, nk = a.kv_heads;
  float out = v;
  if (head < nq + nk) {
    // x cos + rotate_half(x) sin, rotate_half = concat(-x2, x1)
    out = upper ? v * rc + other * rs : v * rc + (-other) * rs;
  }
  if (head < nq) {
    a.q_out[head * a.dh + jj] = out;
  } else if (head < nq + nk) {
    a.k_cache[((head - nq) * a.cap + p) * a.dh + jj] = out;
  } else {
    a.v_cache[((head - nq - nk) * a.cap + p) * a.dh + jj] = out;
  }
}

// ---------------------------------------------------------------------------
// Decode attention (cv3cpu/ops.py:267-300 with one query and no mask,
// qwen2.py:148,169): the G = heads / kv_heads query heads of one kv head
// against keys [0, pos].  Workgroup (split, g) covers keys [split*64, split*64+64)
// and writes, per query head, the chunk's max score m_s, sum l_s = sum e^{s - m_s}
// and unnormalised output o_s = sum e^{s - m_s} v.  The o_proj kernel merges the
// chunks when it stages its input (out = sum_s e^{m_s - M} o_s / sum_s e^{m_s - M} l_s),
// so no workgroup ever waits on another inside a kernel.
// ---------------------------------------------------------------------------
constexpr int KCH = 64;      // keys per chunk
constexpr int64_t kWsQ = 1024;  // q slot of the workspace
constexpr int NSMAX = 16;    // chunks per head: cache capacity <= 1024
struct AttnArgs {
  const float* q;          // [heads * dh]
  const float* k_cache;    // layer's [kv_heads, cap, dh]
  const float* v_cache;
  int heads, kv_heads, dh;
  int64_t cap;
  const int64_t* pos;
  float scale;
  float* part_o;           // [heads, NSMAX, 64]
  float* part_ml;          // [heads, NSMAX, 2]
};

__global__ __launch_bounds__(512) void k_dec_attn(AttnArgs a) {
  __shared__ float Kt[64 * (KCH + 1)];   // K^T: [d][key], padded
  __shared__ float Vs[KCH * 64];         // V: [key][d]
  __shared__ float qs[8 * 64];
  __shared__ float ps[8 * KCH];          // probabilities, one row per head
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;  // wave = query head within the group
  const int split = blockIdx.x, g = blockIdx.y;
  const int G = a.heads / a.kv_heads;
  // Every load is issued before the position is known: keys are clamped to the
  // cache (rows < cap), masked once L is in.
  const int64_t pos = *a.pos;
  const int64_t k0 = (int64_t)split * KCH;
  const float* kb = a.k_cache + (int64_t)g * a.cap * a.dh;
  const float* vb = a.v_cache + (int64_t)g * a.cap * a.dh;
  const int d4n = a.dh / 4;  // float4 per key row
  float4 kr[2], vr[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = threadIdx.x + 512 * r;  // (key, d4) over 64 x 16
    const int key = idx >> 4, d4 = min(idx & 15, d4n - 1);
    const int64_t row = min(k0 + key, a.cap - 1);
    kr[r] = reinterpret_cast<const float4*>(kb + row * a.dh)[d4];
    vr[r] = reinterpret_cast<const float4*>(vb + row * a.dh)[d4];
  }
  // q of the G <= 8 heads: (head, d4) over 8 x 16 float4, one per thread of the first 128
  const int qh = threadIdx.x >> 4, qd4 = threadIdx.x & 15;
  const float4 qraw =
      reinterpret_cast<const float4*>(a.q + (g * G + min(qh, G - 1)) * a.dh)[min(qd4, d4n - 1)];
  const float4 qv = (threadIdx.x < 128 && qh < G && qd4 < d4n) ? qraw : make_float4(0.f, 0.f, 0.f, 0.f);
  const int64_t L = pos + 1;
  const int active = (int)((L + KCH - 1) / KCH);
  if (split >= active) return;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = threadIdx.x + 512 * r;
    const int key = idx >> 4, d4 = idx & 15;
    if (k0 + key >= L || d4 >= d4n) {
      kr[r] = make_float4(0.f, 0.f, 0.f, 0.f);
      vr[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int d = d4 * 4;
    Kt[(d + 0) * (KCH + 1) + key] = kr[r].x;
    Kt[(d + 1) * (KCH + 1) + key] = kr[r].y;
    Kt[(d + 2) * (KCH + 1) + key] = kr[r].z;
    Kt[(d + 3) * (KCH + 1) + key] = kr[r].w;
    reinterpret_cast<float4*>(Vs)[idx] = vr[r];
  }
  if (threadIdx.x < 128)  // (q * scale) first (ops.py:292)
    reinterpret_cast<float4*>(qs)[threadIdx.x] = make_float4(qv.x * a.scale, qv.y * a.scale, qv.z * a.scale,
                                                             qv.w * a.scale);
  __syncthreads();
  const int h = wave;
  if (h >= G) return;
  // score of key `lane` for head h; q read as broadcast float4s
  float s = 0.f;
  const float4* q4 = reinterpret_cast<const float4*>(qs + h * 64);
#pragma unroll
  for (int d4 = 0; d4 < 16; ++d4) {
    const float4 qq = q4[d4];
    s = fmaf(qq.x, Kt[(4 * d4 + 0) * (KCH + 1) + lane], s);
    s = fmaf(qq.y, Kt[(4 * d4 + 1) * (KCH + 1) + lane], s);
    s = fmaf(qq.z, Kt[(4 * d4 + 2) * (KCH + 1) + lane], s);
    s = fmaf(qq.w, Kt[(4 * d4 + 3) * (KCH + 1) + lane], s);
  }
  if (k0 + lane >= L) s = -INFINITY;
  const float m = wave_max(s);
  const float p = expf(s - m);
  const float l = wave_sum(p);
  ps[h * KCH + lane] = p;  // read back by the same wave only
  // o[d = lane] = sum_key p[key] v[key][d]; p read as broadcast float4s
  float o = 0.f;
  const float4* p4 = reinterpret_cast<const float4*>(ps + h * KCH);
#pragma unroll
  for (int k4 = 0; k4 < KCH / 4; ++k4) {
    const float4 pp = p4[k4];
    o = fmaf(pp.x, Vs[(4 * k4 + 0) * 64 + lane], o);
    o = fmaf(pp.y, Vs[(4 * k4 + 1) * 64 + lane], o);
    o = fmaf(pp.z, Vs[(4 * k4 + 2) * 64 + lane], o);
    o = fmaf(pp.w, Vs[(4 * k4 + 3) * 64 + lane], o);
  }
  const int hq = g * G + h;
  a.part_o[((int64_t)hq * NSMAX + split) * 64 + lane] = o;
  if (lane == 0) {
    a.part_ml[((int64_t)hq * NSMAX + split) * 2] = m;
    a.part_ml[((int64_t)hq * NSMAX + split) * 2 + 1] = l;
  }
}

// ---------------------------------------------------------------------------
// o_proj with the attention merge as its prologue: stage
// attn[h*dh + d] = sum_s e^{m_s - M_h} o_s[d] / sum_s e^{m_s - M_h} l_s  (H*dh <= 1024),
// then x += W_o . attn (mode-1 GEMV, LPR = 8).
// ---------------------------------------------------------------------------
struct OprojArgs {
  QW w;
  int64_t layer_row0;
  int64_t n;
  const float* part_o;
  const float* part_ml;
  int heads, dh;
  const int64_t* pos;
  float* x;                // residual stream, updated in place
};

template <int CPL, bool SF16, bool Q4>
__global__ __launch_bounds__(256) void k_dec_oproj(OprojArgs a) {
  extern __shared__ float xs[];
  constexpr int LPR = 8, RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPR, sub = lane % LPR;
  const int64_t col = ((int64_t)blockIdx.x * 4 + wave) * RPW + grp;
  const bool live = col < a.n;
  const int64_t wrow = a.layer_row0 + (live ? col : 0);
  // the attention partials (every chunk, unconditionally), then the weight stream;
  // the chunk count is applied after the loads are out
  const int t = threadIdx.x;
  const int64_t pos = *a.pos;
  const float xres = a.x[live ? col : 0];
  const float2 mlraw = reinterpret_cast<const float2*>(a.part_ml)[min(t, a.heads * NSMAX - 1)];
  const int d4n = a.dh / 4;
  const int oh = t / 16, od4 = t % 16;
  const bool owns = oh < a.heads && od4 < d4n;
  float4 ov[NSMAX];
#pragma unroll
  for (int s2 = 0; s2 < NSMAX; ++s2)
    ov[s2] = reinterpret_cast<const float4*>(a.part_o + ((int64_t)min(oh, a.heads - 1) * NSMAX + s2) * 64)
        [min(od4, d4n - 1)];
  __builtin_amdgcn_sched_barrier(0);
  RowDot<LPR, CPL, SF16, Q4> rd;
  rd.load(a.w, wrow, sub, live);
  __builtin_amdgcn_sched_barrier(0);
  // Chunk weights: thread t holds (m, l) of head t / 16, chunk t % 16.  A head's 16
  // chunks are 16 adjacent lanes, so its max M and denominator sum_s e^{m_s - M} l_s
  // are shuffle reductions; each weight e^{m_s - M} is computed once and shared.
  static_assert(NSMAX == 16, "one lane per chunk in 16-lane head groups");
  __shared__ float wl[16 * NSMAX];
  __shared__ float dl[16];
  const int active = (int)((pos + 1 + KCH - 1) / KCH);
  const int sl = t % NSMAX;
  const bool valid = t < a.heads * NSMAX && sl < active;
  const float mm = valid ? mlraw.x : -INFINITY;
  float M = mm;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  const float wgt = valid ? expf(mm - M) : 0.f;
  float den = valid ? mlraw.y * wgt : 0.f;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
  wl[t] = wgt;
  if (sl == 0) dl[t / NSMAX] = den;
  __syncthreads();
  constexpr int WIDTH = LPR * CPL * kCodes<Q4>;
  if (owns) {
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s2 = 0; s2 < NSMAX; ++s2) {
      if (s2 < active) {  // uniform: stale slots past the active count are never touched
        const float w = wl[oh * NSMAX + s2];
        num.x = fmaf(ov[s2].x, w, num.x);
        num.y = fmaf(ov[s2].y, w, num.y);
        num.z = fmaf(ov[s2].z, w, num.z);
        num.w = fmaf(ov[s2].w, w, num.w);
      }
    }
    const float dsum = dl[oh];
    reinterpret_cast<float4*>(xs + oh * a.dh)[od4] =
        make_float4(num.x / dsum, num.y / dsum, num.z / dsum, num.w / dsum);
  }
  // zero padding up to the staged width (chunks past the row read zeros)
  for (int64_t c = (int64_t)a.heads * a.dh + t; c < WIDTH; c += 256) xs[c] = 0.f;
  __syncthreads();
  const float acc = rd.dot(xs, sub);
  if (live && sub == 0) a.x[col] = xres + acc;
}

// ---------------------------------------------------------------------------
// Greedy selection and the next input row.
// ---------------------------------------------------------------------------
struct NextArgs {
  const float* logits;
  int64_t vocab;
  QW emb;                  // speech_embedding [vocab, hidden] (q8)
  float* x;                // next input, [hidden]
  int64_t* pos;
  int64_t* history;        // [cap]
  int64_t* token;
};

__global__ __launch_bounds__(1024) void k_dec_next(NextArgs a) {
  __shared__ float bv[16];
  __shared__ int64_t bi[16];
  __shared__ int64_t pick;
  float best = -INFINITY;
  int64_t bidx = 0x7fffffffffffffffll;
  // the first 8 * 1024 logits in one batch of loads, any rest in a loop
  float lv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) lv[j] = a.logits[min((int64_t)threadIdx.x + 1024 * j, a.vocab - 1)];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t i = threadIdx.x + 1024 * j;
    if (i < a.vocab && (lv[j] > best || (lv[j] == best && i < bidx))) {
      best = lv[j];
      bidx = i;
    }
  }
  for (int64_t i = threadIdx.x + 8 * 1024; i < a.vocab; i += blockDim.x) {
    const float v = a.logits[i];
    if (v > best || (v == best && i < bidx)) {
      best = v;
      bidx = i;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int64_t oi = __shfl_xor(bidx, o, 64);
    if (ov > best || (ov == best && oi < bidx)) {
      best = ov;
      bidx = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = bidx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = bv[0];
    int64_t id = bi[0];
    for (int w = 1; w < (int)(blockDim.x / 64); ++w)
      if (bv[w] > b || (bv[w] == b && bi[w] < id)) {
        b = bv[w];
        id = bi[w];
      }
    if (id >= a.vocab) id = 0;  // all-NaN logits: keep a valid row
    pick = id;
  }
  __syncthreads();
  const int64_t id = pick;
  // x = dequant(speech_embedding[id])  (cv3cpu/ops.py:126-144, llm.py:121)
  for (int64_t c = threadIdx.x; c < a.emb.k; c += blockDim.x)
    a.x[c] = (float)a.emb.q[id * a.emb.kp + c] * sc_at(a.emb, id, c);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t p = *a.pos;
    a.history[p + 1] = id;
    *a.token = id;
    *a.pos = p + 1;
  }
}

__global__ void k_dec_embed(QW emb, const int64_t* token, float* x) {
  const int64_t id = *token;
  for (int64_t c = threadIdx.x; c < emb.k; c += blockDim.x) x[c] = (float)emb.q[id * emb.kp + c] * sc_at(emb, id, c);
}

// ---------------------------------------------------------------------------
// Sampling (cv3cpu/models/llm.py:37-49,125-149) on the device.
//
// NumPy's Generator draws from PCG64: a 128-bit LCG (multiplier below, the
// stream's odd increment) whose 64-bit output is the XOR of the state's halves
// rotated right by its top 6 bits; random() is (next >> 11) * 2^-53.  The state
// is the Generator's own, copied in and out by the host, so the device consumes
// exactly the draws the reference would and the host Generator continues after.
//
// Per token, in one 1024-thread workgroup, the reference's steps in order:
//   logp = log_softmax(logits); below min_len the eos id (or every stop id)
//   goes to -inf; probs = softmax(logp); the top_k entries in stable descending
//   order (ties to the lower id); the nucleus: entries while their float64 sum
//   is below top_p; p = probs / sum(probs) (NumPy's pairwise sum), cdf =
//   cumsum(p) / cdf[-1], pick = first cdf > random().  If the pick occurs at
//   least win_size * tau_r times among the last win_size tokens of this
//   generation, it is masked and a second draw is taken from the full
//   renormalised softmax the same way.  A stop id ends the generation: the step
//   is recorded and later steps leave everything untouched.
// ---------------------------------------------------------------------------
constexpr int kSampleThreads = 1024;
constexpr int kSamplePerThread = 8;      // vocab <= 8192, ids t*8 .. t*8+7 per thread
constexpr int kTopKMax = 64;
constexpr int kStopIds = 200;            // llm.py:64
constexpr int kCandCap = (kSampleThreads / 64) * kTopKMax;  // gathered top-k candidates

__device__ __forceinline__ uint64_t pcg64_next(uint64_t* st) {
  typedef unsigned __int128 u128;
  const u128 mult = ((u128)2549297995355413924ull << 64) | (u128)4865540595714422341ull;
  u128 state = ((u128)st[0] << 64) | (u128)st[1];
  const u128 inc = ((u128)st[2] << 64) | (u128)st[3];
  state = state * mult + inc;
  st[0] = (uint64_t)(state >> 64);
  st[1] = (uint64_t)state;
  const uint64_t x = (uint64_t)(state >> 64) ^ (uint64_t)state;
  const unsigned rot = (unsigned)(state >> 122);
  return (x >> rot) | (x << ((64u - rot) & 63u));
}

__device__ __forceinline__ double pcg64_double(uint64_t* st) {
  return (double)(pcg64_next(st) >> 11) * (1.0 / 9007199254740992.0);
}

__global__ void k_pcg64_random(uint64_t* pcg, int64_t n, double* out) {
  uint64_t st[4] = {pcg[0], pcg[1], pcg[2], pcg[3]};
  for (int64_t i = 0; i < n; ++i) out[i] = pcg64_double(st);
  for (int i = 0; i < 4; ++i) pcg[i] = st[i];
}

struct SampleArgs {
  NextArgs n;
  double top_p, rep_threshold;
  int64_t top_k, win_size, speech_token_size, min_len;
  int strict_min_len;
  int64_t* ctl;  // [start, stop step + 1 (0 while running), pcg state hi, lo, inc hi, lo]
};


// (probability, id) as one integer whose order is the stable descending sort's:
// larger probability first (non-negative floats order as their bits), then the
// lower id.  0 marks an empty slot.
__device__ __forceinline__ uint64_t rank_key(float p, int id) {
  return ((uint64_t)__float_as_uint(p) << 32) | (uint32_t)(0x7fffffff - id) | (1ull << 31);
}
__device__ __forceinline__ int key_id(uint64_t k) { return 0x7fffffff - (int)((uint32_t)k & 0x7fffffffu); }
__device__ __forceinline__ float key_p(uint64_t k) { return __uint_as_float((uint32_t)(k >> 32)); }

__device__ float blk_max(float v, float* red) {
  v = wave_max_dpp(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
  for (int w = 1; w < kSampleThreads / 64; ++w) t = fmaxf(t, red[w]);
  return t;
}

__device__ float blk_sum(float v, float* red) {
  v = wave_sum_dpp(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < kSampleThreads / 64; ++w) t += red[w];
  return t;
}

__device__ double blk_sum_d(double v, double* red) {
  v = wave_sum_d(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < kSampleThreads / 64; ++w) t += red[w];
  return t;
}

// Exclusive prefix of v over the block in thread order.
__device__ double blk_exclusive_scan_d(double v, double* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  double incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  __syncthreads();
  if (lane == 63) red[wave] = incl;
  __syncthreads();
  double base = 0.0;
  for (int w = 0; w < wave; ++w) base += red[w];
  return base + incl - v;
}

// softmax(sc) over the block as float32 (ops.py:84-87): e = exp(x - max), e / sum(e)
__device__ void blk_softmax(const float* sc, float* p, float* red) {
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kSamplePerThread; ++j) m = fmaxf(m, sc[j]);
  m = blk_max(m, red);
  float e[kSamplePerThread], s = 0.f;
#pragma unroll
  for (int j = 0; j < kSamplePerThread; ++j) {
    e[j] = expf(sc[j] - m);
    s += e[j];
  }
  s = blk_sum(s, red);
#pragma unroll
  for (int j = 0; j < kSamplePerThread; ++j) p[j] = e[j] / s;
}

__global__ __launch_bounds__(kSampleThreads) void k_dec_sample(SampleArgs a) {
  __shared__ float red[kSampleThreads / 64];
  __shared__ double redd[kSampleThreads / 64];
  __shared__ int redi[kSampleThreads / 64];
  __shared__ uint64_t cand[kCandCap];
  __shared__ float rowmax[kSampleThreads / 16];
  __shared__ float thresh;
  __shared__ int ncand;
  __shared__ uint64_t sorted[64];
  __shared__ double draw_u;
  __shared__ int64_t pick;
  __shared__ int resample;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t vocab = a.n.vocab;
  const int base = tid * kSamplePerThread;
  // the logits go out first: nothing they need has to arrive before them
  float x[kSamplePerThread];
  if (base + kSamplePerThread <= vocab) {
    const float4 x0 = reinterpret_cast<const float4*>(a.n.logits + base)[0];
    const float4 x1 = reinterpret_cast<const float4*>(a.n.logits + base)[1];
    x[0] = x0.x, x[1] = x0.y, x[2] = x0.z, x[3] = x0.w, x[4] = x1.x, x[5] = x1.y, x[6] = x1.z, x[7] = x1.w;
  } else {
#pragma unroll
    for (int j = 0; j < kSamplePerThread; ++j) x[j] = base + j < vocab ? a.n.logits[base + j] : -INFINITY;
  }
  if (a.ctl[1] != 0) return;  // a stop id was drawn earlier: the generation is over
  const int64_t pos = *a.n.pos, start = a.ctl[0], step = pos - start;
  // decoded[-win_size:] of the tokens drawn so far (win_size 0 slices them all): wave 0
  // fetches the first 64 now, while the distribution is formed
  const int64_t w = a.win_size > 0 ? min(a.win_size, step) : step;
  const int64_t w0 = pos - w + 1;
  const int64_t hist0 = (wave == 0 && lane < w) ? a.n.history[w0 + lane] : -1;
  // log_softmax (ops.py:90-93), then the eos mask of the first min_len steps
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kSamplePerThread; ++j) m = fmaxf(m, x[j]);
  m = blk_max(m, red);
  float z[kSamplePerThread], s = 0.f;
#pragma unroll
  for (int j = 0; j < kSamplePerThread; ++j) {
    z[j] = x[j] - m;
    s += expf(z[j]);
  }
  const float ls = logf(blk_sum(s, red));
  float sc[kSamplePerThread];
  const bool ignore_eos = step < a.min_len;
  const int64_t sts = a.speech_token_size;
#pragma unroll
  for (int j = 0; j < kSamplePerThread; ++j) {
    const int64_t id = base + j;
    sc[j] = z[j] - ls;
    if (id >= vocab) sc[j] = -INFINITY;
    if (ignore_eos && (a.strict_min_len ? (id >= sts && id < sts + kStopIds) : id == sts)) sc[j] = -INFINITY;
  }
  float p[kSamplePerThread];
  blk_softmax(sc, p, red);
  // top_k in stable descending order.  A lower bound of the k-th largest
  // probability is the k-th largest of the 64 row maxima (16 lanes x 8 ids per
  // row): k rows hold an entry at least that large.  The entries at or above it
  // are gathered, and wave 0 picks the k best of those (ties to the lower id).
  // A flat distribution that leaves more candidates than the gather holds takes
  // the exhaustive path: every wave its own k best, then wave 0 merges.
  const int k = (int)min(a.top_k, vocab);
  uint64_t key[kSamplePerThread];
  float lmax = 0.f;
#pragma unroll
  for (int j = 0; j < kSamplePerThread; ++j) {
    key[j] = base + j < vocab ? rank_key(p[j], base + j) : 0ull;
    if (base + j < vocab) lmax = fmaxf(lmax, p[j]);
  }
  lmax = fmaxf(lmax, __uint_as_float(dpp32<kDppXor1>(__float_as_uint(lmax))));
  lmax = fmaxf(lmax, __uint_as_float(dpp32<kDppXor2>(__float_as_uint(lmax))));
  lmax = fmaxf(lmax, __uint_as_float(dpp32<kDppHalfMirror>(__float_as_uint(lmax))));
  lmax = fmaxf(lmax, __uint_as_float(dpp32<kDppMirror>(__float_as_uint(lmax))));
  if ((lane & 15) == 0) rowmax[wave * 4 + (lane >> 4)] = lmax;
  if (tid == 0) ncand = 0;
  __syncthreads();
  if (wave == 0) {  // the k-th largest row maximum: the row whose key has k - 1 above it
    const uint64_t rk = rank_key(rowmax[lane], lane);
    int above = 0;
#pragma unroll
    for (int q = 0; q < 64; ++q) above += readlane64(rk, q) > rk;
    const uint64_t hit = __ballot(above == k - 1);
    if (lane == 0) thresh = rowmax[__ffsll((unsigned long long)hit) - 1];
  }
  __syncthreads();
  const float T = thresh;
  int mine_n = 0;
#pragma unroll
  for (int j = 0; j < kSamplePerThread; ++j) mine_n += (key[j] != 0 && p[j] >= T);
  if (mine_n) {
    int slot = atomicAdd(&ncand, mine_n);
#pragma unroll
    for (int j = 0; j < kSamplePerThread; ++j)
      if (key[j] != 0 && p[j] >= T) {
        if (slot < kCandCap) cand[slot] = key[j];
        ++slot;
      }
  }
  __syncthreads();
  const int C = ncand;
  constexpr int kPerLane = kCandCap / 64;
  if (C > kCandCap) {  // uniform
    __syncthreads();   // every gather write has landed before the slots are reused
    for (int r = 0; r < k; ++r) {
      uint64_t best = 0;
#pragma unroll
      for (int j = 0; j < kSamplePerThread; ++j) best = max(best, key[j]);
      best = wave_max_u64(best);
#pragma unroll
      for (int j = 0; j < kSamplePerThread; ++j)
        if (key[j] == best) key[j] = 0;
      if (lane == 0) cand[wave * kTopKMax + r] = best;
    }
    __syncthreads();
  }
  if (wave == 0 && C <= 64) {  // one candidate per lane: sort by counting the keys above each
    const uint64_t ck = lane < C ? cand[lane] : 0ull;
    int above = 0;
#pragma unroll
    for (int q = 0; q < 64; ++q) above += readlane64(ck, q) > ck;
    if (ck != 0) sorted[above] = ck;
    wave_sync();
  }
  if (wave == 0) {
    const bool all = C > kCandCap;
    uint64_t ck[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int c = lane + 64 * j;  // gathered slot, or (wave, rank) of the exhaustive path
      const bool ok = C > 64 && (all ? (c % kTopKMax) < k : c < C);
      ck[j] = ok ? cand[c] : 0ull;
    }
    const int used = all ? kPerLane : (C + 63) / 64;  // slots per lane worth scanning
    // entry r of the sorted head goes to lane r
    uint64_t mine = 0;
    if (C <= 64) mine = lane < k ? sorted[lane] : 0ull;
    for (int r = 0; r < (C <= 64 ? 0 : k); ++r) {
      uint64_t best = 0;
#pragma unroll
      for (int j = 0; j < kPerLane; ++j)
        if (j < used) best = max(best, ck[j]);
      best = wave_max_u64(best);
#pragma unroll
      for (int j = 0; j < kPerLane; ++j)
        if (ck[j] == best) ck[j] = 0;
      if (lane == r) mine = best;
    }
    const double v = lane < k ? (double)key_p(mine) : 0.0;
    // the nucleus: entries while the float64 running sum is below top_p (llm.py:40-45);
    // every lane runs the same running sums on the values read from lane i
    double cum = 0.0;
    int n = 0;
    for (int i = 0; i < k; ++i) {
      if (cum >= a.top_p) break;
      cum += readlane_d(v, i);
      ++n;
    }
    if (n < 1) n = 1;  // top_p <= 0 leaves no entry (the reference's draw raises; the host rejects it)
    // p / p.sum() with NumPy's pairwise sum (below 8 entries a running sum)
    double tot;
    if (n < 8) {
      tot = 0.0;
      for (int i = 0; i < n; ++i) tot += readlane_d(v, i);
    } else {
      double r[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] = readlane_d(v, j);
      int i = 8;
      for (; i < n - (n % 8); i += 8)
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] += readlane_d(v, i + j);
      tot = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
      for (; i < n; ++i) tot += readlane_d(v, i);
    }
    // Generator.choice: cdf = cumsum(p); cdf /= cdf[-1]; the first cdf > u
    const double q = lane < n ? v / tot : 0.0;
    double c = 0.0, cdf = 0.0;
    for (int i = 0; i < n; ++i) {
      c += readlane_d(q, i);
      if (lane == i) cdf = c;
    }
    const double last = c;
    uint64_t st[4] = {(uint64_t)a.ctl[2], (uint64_t)a.ctl[3], (uint64_t)a.ctl[4], (uint64_t)a.ctl[5]};
    const double u = pcg64_double(st);  // every lane steps its copy; lane 0 stores it
    const uint64_t past = __ballot(lane < n && cdf / last > u);
    const int idx = past ? __ffsll((unsigned long long)past) - 1 : n - 1;
    int64_t top = key_id(readlane64(mine, idx));
    if (top < 0 || top >= vocab) top = 0;  // no finite probability at all: keep a valid row
    // the repetition test over the window (llm.py:142-144)
    int rep = __popcll(__ballot(hist0 == top));
    for (int64_t q0 = w0 + 64; q0 <= pos; q0 += 64) {  // windows beyond 64 tokens
      const int64_t qq = q0 + lane;
      rep += __popcll(__ballot(qq <= pos && a.n.history[min(qq, pos)] == top));
    }
    const bool again = (double)rep >= a.rep_threshold;
    const double u2 = again ? pcg64_double(st) : 0.0;
    if (lane == 0) {
      resample = again;
      draw_u = u2;
      pick = top;
      for (int i = 0; i < 4; ++i) a.ctl[2 + i] = (int64_t)st[i];
    }
  }
  __syncthreads();
  if (resample) {  // uniform
    const int64_t top = pick;
#pragma unroll
    for (int j = 0; j < kSamplePerThread; ++j)
      if (base + j == top) sc[j] = -INFINITY;
    blk_softmax(sc, p, red);
    double d[kSamplePerThread], tsum = 0.0;
#pragma unroll
    for (int j = 0; j < kSamplePerThread; ++j) {
      d[j] = (double)p[j];
      tsum += d[j];
    }
    const double total = blk_sum_d(tsum, redd);
    // cdf over ids in order: this thread's run of 8 after the sum of all earlier runs
    double run = 0.0;
#pragma unroll
    for (int j = 0; j < kSamplePerThread; ++j) run += d[j] / total;
    double c = blk_exclusive_scan_d(run, redd);
    double last = c + run;
    __syncthreads();
    if (tid == kSampleThreads - 1) redd[0] = last;  // cdf[-1]
    __syncthreads();
    last = redd[0];
    const double u = draw_u;
    int first = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kSamplePerThread; ++j) {
      c += d[j] / total;
      if (base + j < vocab && c / last > u && base + j < first) first = base + j;
    }
    // block minimum of the first id past u
    for (int o = 32; o > 0; o >>= 1) first = min(first, __shfl_xor(first, o, 64));
    if (lane == 0) redi[wave] = first;
    __syncthreads();
    if (tid == 0) {
      int f = redi[0];
      for (int w2 = 1; w2 < kSampleThreads / 64; ++w2) f = min(f, redi[w2]);
      pick = f < vocab ? f : vocab - 1;
    }
    __syncthreads();
  }
  const int64_t id = pick;
  // next input row and the bookkeeping of k_dec_next; a stop id ends the generation
  for (int64_t cc = tid; cc < a.n.emb.k; cc += kSampleThreads)
    a.n.x[cc] = (float)a.n.emb.q[id * a.n.emb.kp + cc] * sc_at(a.n.emb, id, cc);
  __syncthreads();
  if (tid == 0) {
    a.n.history[pos + 1] = id;
    *a.n.token = id;
    *a.n.pos = pos + 1;
    if (id >= sts && id < sts + kStopIds) a.ctl[1] = step + 1;
  }
}

// ---------------------------------------------------------------------------
// The whole decode step as one cooperative kernel (q8 weights).
//
// Every dependent kernel boundary of the step above costs about 4.5 us: the
// launch, then the first loads of the next kernel.  Here one workgroup per CU runs
// all layers; the vectors that cross workgroups (x, q/k/v, attention partials,
// x after o_proj, h) travel as 64-bit words (epoch << 32 | float bits) written and
// polled at device scope, and each phase issues its weight (and cache) loads
// BEFORE it waits for its input, so their latency overlaps the exchange.  Per layer:
//   A  all workgroups: RMSNorm(x) -> [q; k; v] row pairs + bias + rotary; k, v
//      also to the cache (read back by later tokens, after the kernel boundary)
//   B  H x 8 workgroups: one query head over one 128-key chunk of the cache
//      (flash-decoding partial: max, sum, unnormalised output); the item of the
//      head's last live chunk merges the head's partials into its 64 outputs
//   C  up to 256 workgroups (224 at hidden 896): o_proj rows + residual -> x_mid
//   D  all workgroups: RMSNorm(x_mid) -> [gate; up] pairs -> h = silu(g) * u
//   E  up to 256 workgroups (224 at hidden 896): down rows + residual -> x for the next layer
// then the head rows, and (greedy) the argmax, speech_embedding row and
// bookkeeping by workgroup 0.
//
// Reuse of the exchange words: every buffer is double-buffered by layer parity,
// so a word of layer l is rewritten in layer l + 2.  Phase D splits the [gate;
// up] pairs so that every workgroup owns at least one (inter >= workgroups), and
// phase E waits for all of h; so once any workgroup is in layer l + 1, every
// workgroup has finished phase D of layer l, and with it every read of a layer-l
// word except phase E's own, which end before x of layer l exists (only the
// workgroups that own down rows wait in E).  The next writer of any layer-l word
// has passed layer l + 1.  Epochs are launch counter * 256 + layer * 8 + phase
// (the host counts launches and clears the words when the counter wraps), so no
// word left by another phase, layer or launch matches.  Every wait is bounded: a
// word that does not arrive sets the error flag, and every other wait ends
// within 256 polls of seeing it.
// ---------------------------------------------------------------------------
constexpr int kPT = 512;                 // threads per workgroup
constexpr int kPMinG = 128;              // workgroups the step needs at least
constexpr int kPOproj = 256;             // workgroups of phase C, at most (64: 4 % slower, 96: 2 %, than 128; 256: 1.5 % faster)
constexpr int kPDown = 256;              // workgroups of phase E, at most (128: 2 % slower)
// Replicas of the exchanged vectors that many workgroups poll (x: all, x_mid: all,
// h: 224, the merged attention output: all): workgroup w reads replica w % n.  Measured
// with the throttled polling below: one copy is 2 % slower; 4 copies of x_mid are 0.5 %
// faster than 2 (8: 0.3 % slower), and 1 or 4 copies of x, h or the attention output
// change nothing (the producers' extra stores sit on their critical path).
constexpr int kRX = 2, kRM = 4, kRH = 2, kRA = 2;

struct PersistArgs {
  QW qkv, o, gu, dn, head, emb;
  const float *ln1, *ln2, *norm, *qkv_bias, *head_bias, *rope_cos, *rope_sin;
  int layers, D, H, Hk, dh, I;
  float eps, scale;
  float *k_cache, *v_cache;
  int64_t cap;
  int64_t *pos, *token, *history;
  float *x, *logits;
  uint64_t *xb, *qkvb, *pb, *ab, *mb, *hb, *arg;  // exchange words, two sets each (arg: one)
  int64_t sx, sp, sa, sm, sh;                    // words between replicas of x, partials, attention, x_mid, h
  int64_t* err;                              // set when a wait gives up
  uint32_t epoch_base;                       // launch counter * 256, from the host
  int select;                                // 1: greedy argmax + next input here
};


// The workgroup reads the words of up to three ranges (n0 words at s0, then n1 at
// s1, n2 at s2), all carrying epoch e, into dst[0 .. n0 + n1 + n2) in LDS: NW
// words per thread per poll, so a wait of up to NW * 512 words is one round trip.
// False for every thread (and the error flag set) if a word never arrives; a wait
// also ends early once another workgroup has set the flag.
struct Ident {
  __device__ __forceinline__ int operator()(int i) const { return i; }
};
template <int NW, class Map = Ident>
__device__ bool ll_get(const uint64_t* s0, int n0, const uint64_t* s1, int n1, const uint64_t* s2, int n2,
                       uint32_t e, float* dst, int64_t* err, Map map = Map()) {
  const int n = n0 + n1 + n2;
  bool ok = true;
  for (int b0 = 0; b0 < n && ok; b0 += kPT * NW) {
    const uint64_t* src[NW];
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const int idx = b0 + (int)threadIdx.x + kPT * j;
      src[j] = idx < n0 ? s0 + idx : idx < n0 + n1 ? s1 + (idx - n0) : s2 + (idx - n0 - n1);
    }
    uint64_t w[NW];
    bool got = false;
    for (int spins = 0; spins < kPSpin; ++spins) {
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        const int idx = b0 + (int)threadIdx.x + kPT * j;
        w[j] = idx < n ? __hip_atomic_load(src[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : ((uint64_t)e << 32);
      }
      got = true;
#pragma unroll
      for (int j = 0; j < NW; ++j) got = got && (uint32_t)(w[j] >> 32) == e;
      if (got) break;
      if ((spins & 255) == 255 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
      // back off after a few misses: hundreds of workgroups polling the same words
      // slow every exchange down (the narrow waits, up to two words per thread, keep
      // the short sleep: 0.6 % faster decode)
      if (spins < 8 || NW <= 2)
        __builtin_amdgcn_s_sleep(1);
      else
        __builtin_amdgcn_s_sleep(8);
    }
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const int idx = b0 + (int)threadIdx.x + kPT * j;
      if (idx < n) dst[map(idx)] = __uint_as_float((uint32_t)w[j]);
    }
    ok = !__syncthreads_or(!got);
  }
  if (!ok && threadIdx.x == 0) atomicOr(reinterpret_cast<unsigned long long*>(err), 1ull);
  return ok;
}
template <int NW, class Map = Ident>
__device__ __forceinline__ bool ll_get(const uint64_t* src, int n, uint32_t e, float* dst, int64_t* err,
                                       Map map = Map()) {
  return ll_get<NW, Map>(src, n, nullptr, 0, nullptr, 0, e, dst, err, map);
}


// The same for one range, polled by the last NPT threads only, so that the waves with weight
// DMAs in flight (loads complete in issue order) do not hold up the poll: the matrix-core phase
// D's wait for x_mid, polled by waves 3-7 while waves 0-2 fetch the [gate; up] rows (0.6 %
// faster decode; the down rows' wait polled by waves 4-7 alone was 6 % slower: fewer waves
// polling 4864 words take longer per round).
template <int NW, int NPT, class Map = Ident>
__device__ bool ll_get_tail(const uint64_t* src, int n, uint32_t e, float* dst, int64_t* err, Map map = Map()) {
  const int pt = (int)threadIdx.x - (kPT - NPT);
  const bool poller = pt >= 0;
  bool ok = true;
  for (int b0 = 0; b0 < n && ok; b0 += NPT * NW) {
    uint64_t w[NW];
    bool got = true;
    if (poller) {
      got = false;
      for (int spins = 0; spins < kPSpin; ++spins) {
#pragma unroll
        for (int j = 0; j < NW; ++j) {
          const int idx = b0 + pt + NPT * j;
          w[j] = idx < n ? __hip_atomic_load(src + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : ((uint64_t)e << 32);
        }
        got = true;
#pragma unroll
        for (int j = 0; j < NW; ++j) got = got && (uint32_t)(w[j] >> 32) == e;
        if (got) break;
        if ((spins & 255) == 255 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
        if (spins < 8 || NW <= 3)
          __builtin_amdgcn_s_sleep(1);
        else
          __builtin_amdgcn_s_sleep(8);
      }
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        const int idx = b0 + pt + NPT * j;
        if (idx < n) dst[map(idx)] = __uint_as_float((uint32_t)w[j]);
      }
    }
    ok = !__syncthreads_or(!got);
  }
  if (!ok && threadIdx.x == 0) atomicOr(reinterpret_cast<unsigned long long*>(err), 1ull);
  return ok;
}


// Dot product of one weight row spread over the whole wave (64 lanes x CPL
// chunks of 16 int8 codes, or of 32 q4 codes), reduced across the wave: every lane
// gets the sum.  (q4: the chunk dots carry the codes x 16, undone once here.)
template <int CPL, bool SF16, bool Q4>
__device__ __forceinline__ float wdot(const RowDot<64, CPL, SF16, Q4>& rd, const float* xs, int lane) {
  constexpr int CPC = kCodes<Q4>;
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const float* xc = xs + (lane + i * 64) * CPC;
    acc = fmaf(Q4 ? dot32_q4(rd.wv[i], xc) : dot16(rd.wv[i], xc), rd.sc[i], acc);
  }
  if (Q4) acc *= 0.0625f;
  return wave_sum_swap(acc);
}
// The same for one chunk per lane (K <= 64 chunks) with the lane's staged values
// already in registers (a wave computing several rows reads its slice once).
template <int CPC>
struct XSlice {
  float v[CPC];
  // the vector is staged chunk-transposed (xslot): float4 i of lane l's chunk at slot 64 i + l, so
  // the 16 lanes of an LDS pass read 16 consecutive 16-byte slots (in lane order a 64- or 128-byte
  // stride put them on 4 or 2 bank groups)
  __device__ __forceinline__ void load(const float* xs, int lane) {
#pragma unroll
    for (int i = 0; i < CPC / 4; ++i)
      reinterpret_cast<float4*>(v)[i] = reinterpret_cast<const float4*>(xs)[64 * i + lane];
  }
};
// The float4 slot of elements 4 t .. 4 t + 3 in a one-chunk-per-lane vector of CPC-code chunks
// staged for XSlice<CPC>.
template <int CPC>
__device__ __forceinline__ int xslot(int t) {
  return (t % (CPC / 4)) * 64 + t / (CPC / 4);
}
// The same for RowQ4H rows: float4 e (e < 8) of block b holds elements 4 e .. 4 e + 3 of the block,
// which lane 2 b + (e / 2) % 2 reads as its float4 2 (e / 4) + e % 2.
__device__ __forceinline__ int xslot_q4h(int t) {
  const int b = t >> 3, e = t & 7;
  return 64 * (2 * (e >> 2) + (e & 1)) + 2 * b + ((e >> 1) & 1);
}
template <bool Q4H>
__device__ __forceinline__ int body_slot(int t) {
  return Q4H ? xslot_q4h(t) : xslot<16>(t);
}
// ll_get destination map: element i of a vector to its staged float in body_slot order
template <bool Q4H>
struct SlotMap {
  __device__ __forceinline__ int operator()(int i) const { return 4 * body_slot<Q4H>(i >> 2) + (i & 3); }
};
template <bool SF16>
__device__ __forceinline__ float wdot(const RowQ4H<SF16>& rd, const XSlice<16>& x) {
  return wave_sum_swap(fmaf(dot16_q4h(rd.wv, x.v), rd.sc, 0.f) * 0.0625f);
}
template <bool SF16, bool Q4>
__device__ __forceinline__ float wdot(const RowDot<64, 1, SF16, Q4>& rd, const XSlice<kCodes<Q4>>& x) {
  const float acc = fmaf(Q4 ? dot32_q4(rd.wv[0], x.v) : dot16(rd.wv[0], x.v), rd.sc[0], 0.f);
  return wave_sum_swap(Q4 ? acc * 0.0625f : acc);
}

// Chunk-transposed staging for rows of NCH chunks of CPC codes (one chunk per lane and
// per 64-lane step): the f-th float4 of chunk c sits at float4 slot f (NCH + 1) + c, so the
// 64 lanes of a wave, reading the same f of chunks c .. c + 63, read 64 consecutive
// float4s (no LDS bank conflicts; the natural layout puts them 4 CPC bytes apart).  The one
// spare slot per f keeps the writes free of conflicts too: the 16 lanes writing the 4 float4s of
// 4 chunks' f-th values land on 16 different banks (at stride NCH they shared 4).
template <int CPC, int NCH>
struct ChunkT {
  __device__ __forceinline__ int operator()(int k) const {
    return ((((k >> 2) & (CPC / 4 - 1)) * (NCH + 1) + k / CPC) << 2) | (k & 3);
  }
};
template <int CPL, bool SF16, bool Q4>
__device__ __forceinline__ float wdot_t(const RowDot<64, CPL, SF16, Q4>& rd, const float* xs, int lane) {
  constexpr int CPC = kCodes<Q4>, NCH = 64 * CPL;
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    float xc[CPC];
#pragma unroll
    for (int f = 0; f < CPC / 4; ++f)
      reinterpret_cast<float4*>(xc)[f] = reinterpret_cast<const float4*>(xs)[f * (NCH + 1) + lane + i * 64];
    acc = fmaf(Q4 ? dot32_q4(rd.wv[i], xc) : dot16(rd.wv[i], xc), rd.sc[i], acc);
  }
  if (Q4) acc *= 0.0625f;
  return wave_sum_swap(acc);
}

// RMSNorm staging with the norm weight loaded ahead (thread t owns float4 t):
// xs[0, width) = x * w, zero past D (width 1024 or 2048: what a one-chunk-per-lane
// row of q8 or q4 codes reads); returns 1 / sqrt(mean(x^2) + eps), which scales each
// row's dot product afterwards.  x is in LDS.
struct NormStage {
  float4 w;
  __device__ __forceinline__ void prefetch(const float* g, int D) {
    const int t = threadIdx.x;
    w = t < D / 4 ? reinterpret_cast<const float4*>(g)[t] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // stages the 1024 floats XSlice<16> reads (zero past D) in the order of its rows: xslot<16>
  // (q8 chunks) or xslot_q4h (RowQ4H halves)
  template <bool Q4H>
  __device__ __forceinline__ float stage(const float* x, int D, float eps, float* xs, float* red) {
    const int t = threadIdx.x;
    const float4 v = t < D / 4 ? reinterpret_cast<const float4*>(x)[t] : make_float4(0.f, 0.f, 0.f, 0.f);
    float ss = 0.f;
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
    if (t < 256)
      reinterpret_cast<float4*>(xs)[body_slot<Q4H>(t)] = make_float4(v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w);
    ss = wave_sum_swap(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kPT / 64; ++i) tot += red[i];
    return 1.0f / sqrtf(tot / (float)D + eps);
  }
};

// A workgroup with nothing to produce before a wait (phase D outside the o_proj
// workgroups, phase A outside the down workgroups) sleeps through about three
// quarters of its previous layer's wait before polling: the layers take the same
// time, and hundreds of idle workgroups polling the same words from the start
// slow the exchange for everyone.  `prev` is that wait in wall-clock ticks
// (0: poll at once), capped.
__device__ __forceinline__ uint64_t idle_wait(uint64_t t0, uint64_t prev) {
  const uint64_t target = min(prev, (uint64_t)4000) * 3 / 4;
  while (wall_clock64() - t0 < target) __builtin_amdgcn_s_sleep(10);
  return t0;
}


// Q4: the body's matrices are q4 (32 codes per 16-byte chunk); the head and the
// speech embedding stay q8, as the reference's converter stores them.
// MX: phase D's [gate; up] rows (q8, one scale per row) run on the matrix cores.  x_mid * w
// is split into four base-128 digit planes against a shared power of two,
// X = rint(v 2^(27 - E)) with every |v| < 2^E, X = d0 + 128 d1 + 128^2 d2 + 128^3 d3,
// d0..d2 the 7-bit fields of X's two's complement (0..127) and d3 = X >> 21 (-64..63),
// all int8; v_mfma_i32_16x16x64_i8 of the planes (A rows 0..3) with 16 weight
// rows (B: lane l holds row l % 16, codes 16 (l / 16) .. +16 of each 64) gives each
// row's four plane sums exactly in int32, combined in float64 into sum_k q_k X_k, then
// times 2^(E - 27), the row's scale and the RMSNorm factor.  The dot product is that
// of the int8 row with v rounded 27 bits below its largest element, and the rows cost
// no per-code VALU work (the VALU path spends two instructions per code).  The rows go
// global -> LDS by DMA (global_load_lds_dwordx4) in the MFMA operand order, so they hold
// no registers while the workgroup waits for x_mid.
constexpr int kMxSteps = 16;  // 64-code steps of a row: hidden <= 1024
// One 16-byte global -> LDS DMA per lane (lane l lands at lds + 16 l).  A function of its own:
// the builtin called directly inside the kernel template's lambda made clang drop that
// instantiation's host stub without a diagnostic (an undefined symbol at load time).
__device__ __forceinline__ void dma16(const void* g, void* lds) { __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0); }
template <bool SF16, bool Q4, bool MX = false>
__global__ __launch_bounds__(kPT) void k_dec_persist(PersistArgs a) {
  constexpr int CPC = kCodes<Q4>;       // codes per chunk of the body rows
  constexpr int kStage = 64 * 16;       // staged width of a body row: 16 codes per lane (q8 chunk, q4 half block)
  constexpr int kDownCPL = Q4 ? 3 : 5;  // chunks per lane of a down row
  constexpr int kXs = (CPC / 4) * (64 * kDownCPL + 1) * 4;  // ChunkT's slots of a down row
  __shared__ __align__(16) float xin[1024];   // x of the layer (raw), for A's norm and C's residual
  __shared__ __align__(16) float xmid[1024];  // x after o_proj (phase D keeps it for E)
  __shared__ __align__(16) float xs[kXs];     // staged (normed, zero-padded) vector of the dot products
  __shared__ __align__(16) float big[8192];   // phase B: q, k, v, per-wave partials, the merge's partials; the head's candidates
  static_assert(1024 + (kPChunks - 1) * kPPart <= 8192, "the merging item's partials fit after B's per-wave partials");
  __shared__ float red[16];
  __shared__ float hb_val[8];
  __shared__ int hb_i[8];
  __shared__ uint64_t hb_key[8];
  // MX: digit planes 1 KB apart, then 64 zero bytes.  (The 16 lanes reading 16 bytes of four
  // planes at four offsets share 4 banks; planes 64 kMxSteps + 64 bytes apart put them on 16,
  // which cut the step's LDS conflict cycles by a fifth and measured 0.3 % slower.)
  constexpr int kPlane = 64 * kMxSteps;
  __shared__ __align__(16) int8_t dpl[MX ? 4 * kPlane + 64 : 16];
  __shared__ __align__(16) int8_t dmw[MX ? 3 * kMxSteps * 1024 : 16];     // MX: phase D's rows, [block][step][lane][16]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps per-wave indices scalar
  const int G = gridDim.x, w = blockIdx.x;
  const int D = a.D, H = a.H, Hk = a.Hk, dh = a.dh, I = a.I;
  const int R = (H + 2 * Hk) * dh;  // [q; k; v] rows per layer
  const int GQ = H / Hk;            // query heads per kv head
  const uint32_t base = a.epoch_base;
  const int64_t pos = *a.pos;
  const int nact = (int)((pos + kPKeys) / kPKeys);  // attention chunks in use
  const int half = dh / 2;
  const int nE = min(kPDown, G);  // phase E's workgroups
  const int nC = min(kPOproj, G);  // phase C's workgroups
  const int rowsC = (D + nC - 1) / nC, rowsE = (D + nE - 1) / nE;
  const bool isB = w < H * kPChunks && (w % kPChunks) < nact;
  // every workgroup waits in C (those without rows then go straight to D's wait: 1.5 % faster
  // than sleeping through most of it, as the idle ones do before A); only those that own rows
  // wait in E
  const bool isC = w < nC, isE = w < nE && w * rowsE < D;
  // phase A's pair of this wave and its rotary factors (the same in every layer)
  const int npairs = R / 2;
  const int pA = w + G * wave;
  const bool liveA = pA < npairs;
  const int hdA = (liveA ? pA : 0) / half, jA = (liveA ? pA : 0) % half;
  const int r0A = hdA * dh + jA, r1A = r0A + half;
  const float c0 = a.rope_cos[pos * dh + jA], s0 = a.rope_sin[pos * dh + jA];
  const float c1 = a.rope_cos[pos * dh + jA + half], s1 = a.rope_sin[pos * dh + jA + half];
  // phase C's rows, phase D's pairs (every workgroup owns at least one: I >= G), phase E's row
  const int raC = w * rowsC + wave, rbC = w * rowsC + wave + 8;
  const bool laC = isC && wave < rowsC && raC < D, lbC = isC && wave + 8 < rowsC && rbC < D;
  const int jbeg = (int)((int64_t)w * I / G), perD = (int)((int64_t)(w + 1) * I / G) - jbeg;
  const int rE = w * rowsE + wave;
  const bool liveE = isE && wave < rowsE && rE < D;

  // Weight loads: each phase issues its own just before its wait, so they arrive
  // while it polls.  (Loads complete in issue order, so a poll also waits for
  // every load issued before it; issuing the next phase's weights any earlier
  // holds up this phase's wait or its compute.)
  using BodyRow = std::conditional_t<Q4, RowQ4H<SF16>, RowDot<64, 1, SF16, false>>;
  BodyRow dA0, dA1, dC0, dC1, dg[MX ? 1 : 3], du[MX ? 1 : 3];
  // MX: wave b < ceil(perD / 8) loads and multiplies pairs 8b .. 8b + 7 of phase D: lane l the
  // gate (l % 16 < 8) or up row of pair 8b + l % 8, codes 16 (l / 16) .. +16 of each 64-code step
  float mxs = 0.f;
  const int nsteps = (D + 63) / 64, nblk = (perD + 7) / 8;
  RowDot<64, kDownCPL, SF16, Q4> dd;
  NormStage ns1, ns2;
  float bA0, bA1;
  auto load_A = [&](int l) {
    dA0.load(a.qkv, (int64_t)l * R + r0A, lane, liveA);
    dA1.load(a.qkv, (int64_t)l * R + r1A, lane, liveA);
    bA0 = a.qkv_bias[(int64_t)l * R + r0A];
    bA1 = a.qkv_bias[(int64_t)l * R + r1A];
    ns1.prefetch(a.ln1 + (int64_t)l * D, D);
  };
  auto load_C = [&](int l) {
    dC0.load(a.o, (int64_t)l * D + (laC ? raC : 0), lane, laC);
    dC1.load(a.o, (int64_t)l * D + (lbC ? rbC : 0), lane, lbC);
  };
  auto load_D = [&](int l) {
    if constexpr (MX) {
      if (wave < nblk) {  // uniform per wave
        const int r16 = lane & 15, pr = wave * 8 + (r16 & 7);
        const int64_t row = (int64_t)l * 2 * I + (r16 < 8 ? 0 : I) + jbeg + (pr < perD ? pr : 0);
        const int8_t* base = a.gu.q + row * a.gu.kp;
        const int nch = (int)(a.gu.kp / 16);
#pragma unroll
        for (int s = 0; s < kMxSteps; ++s)
          if (s < nsteps)
            dma16(base + 16 * min(4 * s + (lane >> 4), nch - 1), dmw + (wave * kMxSteps + s) * 1024);
        mxs = SF16 ? __half2float(reinterpret_cast<const __half*>(a.gu.scales)[row])
                   : reinterpret_cast<const float*>(a.gu.scales)[row];
      }
    } else {
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const bool live = wave + 8 * t < perD;
        const int64_t jr = live ? jbeg + wave + 8 * t : jbeg;
        dg[t].load(a.gu, (int64_t)l * 2 * I + jr, lane, live);
        du[t].load(a.gu, (int64_t)l * 2 * I + I + jr, lane, live);
      }
    }
    ns2.prefetch(a.ln2 + (int64_t)l * D, D);
  };
  auto load_E = [&](int l) { dd.load(a.dn, (int64_t)l * D + (liveE ? rE : 0), lane, liveE); };

  // the dot products read xs up to 64 chunks per lane row: the tail past what a phase stages stays zero
  for (int i = tid; i < kXs; i += kPT) xs[i] = 0.f;
  if constexpr (MX)
    if (tid < 16) reinterpret_cast<uint32_t*>(dpl + 4 * kPlane)[tid] = 0u;
  load_A(0);
  __syncthreads();
  uint64_t waitA = 0, waitD = 0;  // the idle workgroups' previous waits (wall-clock ticks)

  for (int l = 0; l < a.layers; ++l) {
    const int par = l & 1;
    const uint32_t E = base + (uint32_t)l * 8u;
    // ---- A: [q; k; v] pairs (rows head*dh + j and + half) ----
    {
      if (l == 0) {  // its weights went out before the loop
        for (int i = tid; i < D; i += kPT) xin[i] = a.x[i];
        __syncthreads();
      } else {
        load_A(l);
        const uint64_t t0 = isE ? 0 : idle_wait(wall_clock64(), waitA);
        if (!ll_get<2>(a.xb + ((par ^ 1) * kRX + w % kRX) * a.sx, D, E - 8u + 4u, xin, a.err)) return;
        if (!isE) waitA = wall_clock64() - t0;
      }
      const float inv = ns1.stage<Q4>(xin, D, a.eps, xs, red);
      XSlice<16> xv;
      xv.load(xs, lane);
      float v0 = wdot(dA0, xv) * inv + bA0;
      float v1 = wdot(dA1, xv) * inv + bA1;
      if (liveA && lane == 0) {
        if (hdA < H + Hk) {  // rotary on q and k: x cos + rotate_half(x) sin
          const float o0 = v0 * c0 + (-v1) * s0, o1 = v1 * c1 + v0 * s1;
          v0 = o0;
          v1 = o1;
        }
        ll_put(a.qkvb + par * R + r0A, v0, E);
        ll_put(a.qkvb + par * R + r1A, v1, E);
        if (hdA >= H) {  // k or v head: the cache row at pos
          const int kvh = hdA - H;
          float* cache = kvh < Hk ? a.k_cache : a.v_cache;
          const int gh = kvh < Hk ? kvh : kvh - Hk;
          float* row = cache + (((int64_t)l * Hk + gh) * a.cap + pos) * dh;
          row[jA] = v0;
          row[jA + half] = v1;
        }
      }
      __syncthreads();  // xs is reused below
    }
    // ---- B: attention item (query head h, 128-key chunk c) ----
    if (isB) {
      const int h = w / kPChunks, c = w % kPChunks, g = h / GQ;
      const float* kb = a.k_cache + ((int64_t)l * Hk + g) * a.cap * dh;
      const float* vb = a.v_cache + ((int64_t)l * Hk + g) * a.cap * dh;
      const int ipos = (int)pos, last = ipos > 0 ? ipos - 1 : 0;  // rows before pos come from earlier launches
      // scores: wave `wave` has keys kw + lane / 4, a quarter (16 dims) per lane
      const int kw = c * kPKeys + 16 * wave;
      const int key = kw + (lane >> 2);
      const int qd = (lane & 3) * 16;
      float4 kr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) kr[i] = reinterpret_cast<const float4*>(kb + (int64_t)min(key, last) * dh + qd)[i];
      // values: the wave's 16 keys, dim = lane (keys past pos read row `last`: finite, and weighted 0)
      float vr[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) vr[t] = vb[(int64_t)min(kw + t, last) * dh + lane];
      float* qkv = big;  // q [dh], k [dh], v [dh] of this layer
      if (!ll_get<1>(a.qkvb + par * R + h * dh, dh, a.qkvb + par * R + (H + g) * dh, dh,
                     a.qkvb + par * R + (H + Hk + g) * dh, dh, E, qkv, a.err))
        return;
      if (key == ipos) {
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[i] = reinterpret_cast<const float4*>(qkv + dh + qd)[i];
      }
      // scores in base-2 units, (q * scale) first (ops.py:292), then q * log2(e): the
      // softmax weights e^{s - m} become single v_exp_f32 (2^x); the partials' m are in
      // the same units, which only the merge below reads
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 q4 = reinterpret_cast<const float4*>(qkv + qd)[i];
        s = fmaf((q4.x * a.scale) * kLog2E, kr[i].x, s);
        s = fmaf((q4.y * a.scale) * kLog2E, kr[i].y, s);
        s = fmaf((q4.z * a.scale) * kLog2E, kr[i].z, s);
        s = fmaf((q4.w * a.scale) * kLog2E, kr[i].w, s);
      }
      s += __uint_as_float(dpp32<kDppXor1>(__float_as_uint(s)));
      s += __uint_as_float(dpp32<kDppXor2>(__float_as_uint(s)));
      s = key <= ipos ? s : -INFINITY;
      const float mw = wave_max_dpp(s);  // the wave's 16 keys
      const float p = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s - mw);  // 0 for keys past pos
      const float lw = wave_sum_swap((lane & 3) == 0 ? p : 0.f);
      const float vnew = qkv[2 * dh + lane];  // v of this token
      const int tn = ipos - kw;               // its slot in the wave's keys (may lie outside 0..15)
      float o = 0.f;                          // dim = lane
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const float pt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 4 * t));
        o = fmaf(pt, t == tn ? vnew : vr[t], o);
      }
      float* ow = big + 4 * dh;  // [8 waves][dh], then m, l per wave
      ow[wave * dh + lane] = o;
      if (lane == 0) {
        ow[8 * dh + wave] = mw;
        ow[8 * dh + 8 + wave] = lw;
      }
      __syncthreads();
      // the item of the last live chunk merges its head: it waits for the other chunks'
      // partials and publishes the head's 64 outputs, so phase C reads H dh words instead of
      // every partial (nact H 66) and does no merge of its own
      const bool merger = c == nact - 1;
      float M = -INFINITY, L = 0.f, O = 0.f;
      if (wave == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) M = fmaxf(M, ow[8 * dh + i]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float mi = ow[8 * dh + i];
          const float f = mi == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mi - M);
          L = fmaf(ow[8 * dh + 8 + i], f, L);
          O = fmaf(ow[i * dh + lane], f, O);
        }
        if (!merger) {
          uint64_t* out = a.pb + par * a.sp + ((int64_t)h * kPChunks + c) * kPPart;
          if (lane == 0) {
            ll_put(out, M, E + 1u);
            ll_put(out + 1, L, E + 1u);
          }
          ll_put(out + 2 + lane, O, E + 1u);
        }
      }
      if (merger) {
        float* pm = big + 1024;  // [nact - 1][66]: chunks 0 .. nact - 2 of head h
        if (nact > 1 &&
            !ll_get<1>(a.pb + par * a.sp + (int64_t)h * kPChunks * kPPart, (nact - 1) * kPPart, E + 1u, pm, a.err))
          return;
        if (wave == 0) {
          // M = max m_c, den = sum l_c 2^{m_c - M}, out = sum o_c 2^{m_c - M} / den, chunks in order
          float Mx = M;
#pragma unroll
          for (int cc = 0; cc < kPChunks - 1; ++cc)
            if (cc < nact - 1) Mx = fmaxf(Mx, pm[cc * kPPart]);
          float den = 0.f;
#pragma unroll
          for (int cc = 0; cc < kPChunks - 1; ++cc)
            if (cc < nact - 1) den = fmaf(pm[cc * kPPart + 1], __builtin_amdgcn_exp2f(pm[cc * kPPart] - Mx), den);
          den = fmaf(L, __builtin_amdgcn_exp2f(M - Mx), den);
          float att = 0.f;
#pragma unroll
          for (int cc = 0; cc < kPChunks - 1; ++cc)
            if (cc < nact - 1)
              att = fmaf(pm[cc * kPPart + 2 + lane], __builtin_amdgcn_exp2f(pm[cc * kPPart] - Mx) / den, att);
          att = fmaf(O, __builtin_amdgcn_exp2f(M - Mx) / den, att);
#pragma unroll
          for (int rr = 0; rr < kRA; ++rr) ll_put(a.ab + (par * kRA + rr) * a.sa + h * dh + lane, att, E + 5u);
        }
      }
      __syncthreads();  // big is reused below
    }
    // ---- C: o_proj rows + residual -> x_mid ----
    if (isC) {
      load_C(l);
      // the merged attention output (H dh words, from phase B's merging items) goes straight
      // into the staged slots of the o_proj rows; the slots up to kStage stay zero
      static_assert(kStage % kPT == 0, "the staged width is a multiple of the workgroup");
      for (int i = H * dh + tid; i < kStage; i += kPT) xs[4 * body_slot<Q4>(i >> 2) + (i & 3)] = 0.f;
      if (!ll_get<2>(a.ab + (par * kRA + w % kRA) * a.sa, H * dh, E + 5u, xs, a.err, SlotMap<Q4>())) return;
      XSlice<16> xv;
      xv.load(xs, lane);
      const float va = wdot(dC0, xv), vb2 = wdot(dC1, xv);
      if (lane < kRM) {  // lane i writes replica i
        if (laC) ll_put(a.mb + (par * kRM + lane) * a.sm + raC, xin[raC] + va, E + 2u);
        if (lbC) ll_put(a.mb + (par * kRM + lane) * a.sm + rbC, xin[rbC] + vb2, E + 2u);
      }
      __syncthreads();
    }
    // ---- D: [gate; up] pairs -> h ----
    {
      load_D(l);
      const uint64_t t0 = isC ? 0 : idle_wait(wall_clock64(), waitD);
      if (MX ? !ll_get_tail<3, kPT - 192>(a.mb + (par * kRM + w % kRM) * a.sm, D, E + 2u, xmid, a.err)
             : !ll_get<2>(a.mb + (par * kRM + w % kRM) * a.sm, D, E + 2u, xmid, a.err))
        return;
      if (!isC) waitD = wall_clock64() - t0;
      if constexpr (MX) {
        // RMSNorm statistic and max |x_mid * w| in one reduction, then the digit planes
        const int t = tid;
        const float4 v = t < D / 4 ? reinterpret_cast<const float4*>(xmid)[t] : make_float4(0.f, 0.f, 0.f, 0.f);
        float ss = 0.f;
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
        const float vw[4] = {v.x * ns2.w.x, v.y * ns2.w.y, v.z * ns2.w.z, v.w * ns2.w.w};
        float mx = fmaxf(fmaxf(fabsf(vw[0]), fabsf(vw[1])), fmaxf(fabsf(vw[2]), fabsf(vw[3])));
        ss = wave_sum_swap(ss);
        mx = wave_max_dpp(mx);
        if (lane == 0) {
          red[wave] = ss;
          red[8 + wave] = mx;
        }
        __syncthreads();
        float tot = 0.f, m = 0.f;
#pragma unroll
        for (int i = 0; i < kPT / 64; ++i) {
          tot += red[i];
          m = fmaxf(m, red[8 + i]);
        }
        const float inv = 1.0f / sqrtf(tot / (float)D + a.eps);
        int Ex = 0;
        if (m > 0.f) (void)frexpf(m, &Ex);  // m = f 2^Ex, f in [0.5, 1): every |v| < 2^Ex
        Ex = max(Ex, -96);                  // 2^(27 - Ex) stays finite; tiny vectors lose low bits only
        if (t < 16 * kMxSteps) {            // planes to 64 kMxSteps bytes, zero past D
          const float up = ldexpf(1.0f, 27 - Ex);
          int X[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) X[i] = __float2int_rn(vw[i] * up);  // |X| < 2^27
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            uint32_t pk = 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              pk |= (p < 3 ? ((uint32_t)X[i] >> (7 * p)) & 127u : (uint32_t)(X[i] >> 21) & 0xFFu) << (8 * i);
            reinterpret_cast<uint32_t*>(dpl + p * kPlane)[t] = pk;
          }
        }
        __syncthreads();
        if (wave < nblk) {  // uniform per wave
          const int i = lane & 15;
          // lanes of MFMA rows 0..3 read plane i, rows 4..15 the zero bytes
          const int8_t* ab = i < 4 ? dpl + i * kPlane + (lane >> 4) * 16 : dpl + 4 * kPlane;
          const int ast = i < 4 ? 64 : 0;
          const int8_t* wb = dmw + wave * kMxSteps * 1024 + lane * 16;
          __builtin_amdgcn_s_waitcnt(CV3_VMCNT(0));  // this wave's row DMAs (they precede its polls anyway)
          // two register sets of two steps each: one set's fragments are read from LDS while
          // the other's multiply (reads past the last step repeat it and go unused)
          auto fa = [&](int s) { return *reinterpret_cast<const i32x4*>(ab + min(s, nsteps - 1) * ast); };
          auto fb = [&](int s) { return *reinterpret_cast<const i32x4*>(wb + min(s, nsteps - 1) * 1024); };
          i32x4 c = {0, 0, 0, 0};
          i32x4 pa0 = fa(0), pb0 = fb(0), pa1 = fa(1), pb1 = fb(1);
          for (int s = 0; s < nsteps; s += 4) {
            const i32x4 qa0 = fa(s + 2), qb0 = fb(s + 2), qa1 = fa(s + 3), qb1 = fb(s + 3);
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa0, pb0, c, 0, 0, 0);
            if (s + 1 < nsteps) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa1, pb1, c, 0, 0, 0);
            if (s + 2 >= nsteps) break;
            pa0 = fa(s + 4);
            pb0 = fb(s + 4);
            pa1 = fa(s + 5);
            pb1 = fb(s + 5);
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa0, qb0, c, 0, 0, 0);
            if (s + 3 < nsteps) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa1, qb1, c, 0, 0, 0);
          }
          // lanes 0..15: the four plane sums of weight row i
          const double T = (double)c[0] + 128.0 * (double)c[1] + 16384.0 * (double)c[2] + 2097152.0 * (double)c[3];
          const float val = (float)(T * (double)ldexpf(1.0f, Ex - 27) * (double)mxs) * inv;
          const float upv = __shfl_xor(val, 8, 64);  // lanes 0..7: the up row of the same pair
          const int pr = wave * 8 + i;
          if (lane < 8 && pr < perD) {
            const float hv = (val / (1.0f + expf(-val))) * upv;
#pragma unroll
            for (int rr = 0; rr < kRH; ++rr) ll_put(a.hb + (par * kRH + rr) * a.sh + jbeg + pr, hv, E + 3u);
          }
        }
        __syncthreads();
      } else {
      const float inv = ns2.stage<Q4>(xmid, D, a.eps, xs, red);
      XSlice<16> xv;
      xv.load(xs, lane);
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        if (wave + 8 * t < perD) {  // uniform per wave
          const float gv = wdot(dg[t], xv) * inv, uv = wdot(du[t], xv) * inv;
          if (lane < kRH)
            ll_put(a.hb + (par * kRH + lane) * a.sh + jbeg + wave + 8 * t, (gv / (1.0f + expf(-gv))) * uv, E + 3u);
        }
      }
      __syncthreads();  // xs is restaged below
      }
    }
    // ---- E: down rows + residual -> x of the next layer ----
    if (isE) {
      load_E(l);
      // h staged chunk-transposed; the slots of k >= I must be zero (other phases stage
      // their vectors over part of this range)
      const ChunkT<CPC, 64 * kDownCPL> tmap;
      for (int k = I + tid; k < 64 * kDownCPL * CPC; k += kPT) xs[tmap(k)] = 0.f;
      if (!ll_get<10>(a.hb + (par * kRH + w % kRH) * a.sh, I, E + 3u, xs, a.err, tmap)) return;
      const float v = wdot_t(dd, xs, lane);
      if (liveE && lane < kRX) ll_put(a.xb + (par * kRX + lane) * a.sx + rE, xmid[rE] + v, E + 4u);
      __syncthreads();
    }
  }
  // ---- head rows, then the greedy pick ----
  const uint32_t EH = base + (uint32_t)a.layers * 8u;
  {
    const int V = (int)a.head.rows, per = (V + G - 1) / G, rbeg = w * per;
    RowDot<64, 1, SF16, false> dh4[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int rr = rbeg + wave + 8 * t;
      const bool live = wave + 8 * t < per && rr < V;
      dh4[t].load(a.head, live ? rr : 0, lane, live);
    }
    NormStage ns;
    ns.prefetch(a.norm, D);
    float hbias[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int rr = rbeg + wave + 8 * t;
      hbias[t] = a.head_bias && rr < V ? a.head_bias[rr] : 0.f;
    }
    const int lp = (a.layers - 1) & 1;
    if (!ll_get<2>(a.xb + (lp * kRX + w % kRX) * a.sx, D, EH - 8u + 4u, xin, a.err)) return;
    const float inv = ns.stage<false>(xin, D, a.eps, xs, red);
    XSlice<16> xv;
    xv.load(xs, lane);
    float best = -INFINITY;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int rr = rbeg + wave + 8 * t;
      if (wave + 8 * t < per && rr < V) {  // uniform per wave
        const float v = wdot(dh4[t], xv) * inv + hbias[t];
        if (lane == 0) a.logits[rr] = v;
        if (v > best) {  // rows ascend within the wave
          best = v;
          bidx = rr;
        }
      }
    }
    if (lane == 0) {
      hb_val[wave] = best;
      hb_i[wave] = bidx;
    }
    __syncthreads();
    if (!a.select) return;
    if (tid == 0) {
      float b = hb_val[0];
      int bi = hb_i[0];
      for (int k = 1; k < kPT / 64; ++k)
        if (hb_val[k] > b || (hb_val[k] == b && hb_i[k] < bi)) {
          b = hb_val[k];
          bi = hb_i[k];
        }
      ll_put(a.arg + 2 * w, b, EH);
      ll_put(a.arg + 2 * w + 1, __int_as_float(bi), EH);
    }
    if (w != 0) return;
    float* cand = big;
    if (!ll_get<1>(a.arg, 2 * G, EH, cand, a.err)) return;
    // argmax over the workgroups' candidates: larger value, then the lower row
    uint64_t k = 0;
    if (tid < G) k = ((uint64_t)ord_bits(cand[2 * tid]) << 32) | (0xffffffffu - (uint32_t)__float_as_int(cand[2 * tid + 1]));
    k = wave_max_u64(k);
    if (lane == 0) hb_key[wave] = k;
    __syncthreads();
    uint64_t kb = hb_key[0];
#pragma unroll
    for (int i = 1; i < kPT / 64; ++i) kb = max(kb, hb_key[i]);
    int bi = (int)(0xffffffffu - (uint32_t)kb);
    if (bi < 0 || bi >= V) bi = 0;  // all-NaN logits: keep a valid row
    const int64_t id = bi;
    for (int64_t cc = tid; cc < a.emb.k; cc += kPT)
      a.x[cc] = (float)a.emb.q[id * a.emb.kp + cc] * sc_at(a.emb, id, cc);
    if (tid == 0) {
      a.history[pos + 1] = id;
      *a.token = id;
      *a.pos = pos + 1;
    }
  }
}


template <int LPR, int CPL, bool Q4>
void launch_gemv(const GemvArgs& a, hipStream_t st) {
  const int64_t rows_per_block = 4 * (64 / LPR) / (a.mode == 2 ? 2 : 1);
  const dim3 grid((unsigned)ceil_div(a.n, rows_per_block));
  const size_t lds = (size_t)LPR * CPL * kCodes<Q4> * sizeof(float);
#define CV3_GEMV_LAUNCH(MODE)                                                                  \
  if (a.w.sf16)                                                                               \
    hipLaunchKernelGGL((k_dec_gemv<LPR, CPL, MODE, true, Q4>), grid, dim3(256), lds, st, a);  \
  else                                                                                        \
    hipLaunchKernelGGL((k_dec_gemv<LPR, CPL, MODE, false, Q4>), grid, dim3(256), lds, st, a);
  if (a.mode == 2) {
    CV3_GEMV_LAUNCH(2)
  } else if (a.mode == 1) {
    CV3_GEMV_LAUNCH(1)
  } else {
    CV3_GEMV_LAUNCH(0)
  }
#undef CV3_GEMV_LAUNCH
}

// Lanes per row and 16-byte chunks per lane for a row of nch chunks.  Every
// shape stages at most 1024 * 16 floats of vector in LDS (64 KiB).
template <bool Q4>
int gemv_shape(const GemvArgs& a, hipStream_t st) {
  const int64_t nch = (Q4 ? a.w.kp / 2 : a.w.kp) / 16;
  if (Q4 && nch <= 8 * 4) {
    launch_gemv<8, 4, Q4>(a, st);    // q4, K <= 1024: 128 contiguous bytes per row group
  } else if (!Q4 && a.mode == 2 && nch <= 16 * 4) {
    launch_gemv<16, 4, Q4>(a, st);   // q8 [gate; up], K <= 1024: half the chunks per lane of 8 x 8
  } else if (nch <= 8 * 8) {
    launch_gemv<8, 8, Q4>(a, st);
  } else if (a.mode == 2 && nch <= 16 * 20) {
    launch_gemv<16, 20, Q4>(a, st);  // SwiGLU pairs two row groups of one wave
  } else if (Q4 && a.mode != 2 && nch <= 64 * 3) {
    launch_gemv<64, 3, Q4>(a, st);   // q4, K = 4864: one row per wave
  } else if (a.mode != 2 && nch <= 64 * 5) {
    launch_gemv<64, 5, Q4>(a, st);   // q8, K = 4864: one row per wave, 4 rows per workgroup
  } else if (a.mode != 2 && nch * kCodes<Q4> <= 64 * 16 * 16) {
    launch_gemv<64, Q4 ? 8 : 16, Q4>(a, st);
  } else {
    return fail(CV3_EUNSUPPORTED, "decode GEMV K=%lld too large", (long long)a.w.kp);
  }
  CV3_LAUNCHED();
  return CV3_OK;
}

int gemv(const GemvArgs& a, hipStream_t st) { return a.w.q4 ? gemv_shape<true>(a, st) : gemv_shape<false>(a, st); }

}  // namespace

extern "C" {

// One decode step: the layers, the head, then greedy selection (smp == nullptr) or the sampler.
static int decode_step(const cv3_qwen2_model* m, const cv3_qwen2_state* s, const cv3_sampler* smp,
                       cv3_stream_t stream) {
  CV3_REQUIRE(m && s, CV3_EINVAL, "null model or state");
  const int64_t H = m->heads, Hk = m->kv_heads, dh = m->head_dim, D = m->hidden, I = m->inter;
  CV3_REQUIRE(H > 0 && Hk > 0 && H % Hk == 0 && H / Hk <= 8, CV3_EINVAL, "heads %lld / kv heads %lld",
              (long long)H, (long long)Hk);
  CV3_REQUIRE(dh > 0 && dh <= 64 && dh % 2 == 0 && H * dh == D, CV3_EINVAL, "head dim %lld", (long long)dh);
  CV3_REQUIRE(m->layers > 0 && s->cap > 0 && s->cap % KCH == 0, CV3_EINVAL, "cache capacity must be a multiple of 64");
  int rc;
  if ((rc = check_qw(m->qkv, "qkv", D))) return rc;
  if ((rc = check_qw(m->o, "o_proj", H * dh))) return rc;
  if ((rc = check_qw(m->gate_up, "gate_up", D))) return rc;
  if ((rc = check_qw(m->down, "down", I))) return rc;
  if ((rc = check_qw(m->head, "llm_decoder", D))) return rc;
  if ((rc = check_qw(m->embedding, "speech_embedding", D))) return rc;
  CV3_REQUIRE(m->qkv.rows == (H + 2 * Hk) * dh && m->o.rows == D && m->gate_up.rows == 2 * I && m->down.rows == D,
              CV3_EINVAL, "stacked weight rows do not match the geometry");
  CV3_REQUIRE(m->qkv.kp <= 1024, CV3_EUNSUPPORTED, "qkv K too large for the fused rotary GEMV");
  CV3_REQUIRE(s->cap / KCH <= NSMAX, CV3_EUNSUPPORTED, "cache capacity above %d positions", NSMAX * KCH);
  CV3_REQUIRE(H <= 16 && dh % 4 == 0 && D % 4 == 0 && I % 4 == 0, CV3_EUNSUPPORTED, "decode geometry");
  CV3_REQUIRE(m->o.kp <= 1024, CV3_EUNSUPPORTED, "o_proj K too large");
  CV3_REQUIRE(m->embedding.kind == CV3_KIND_Q8, CV3_EUNSUPPORTED, "speech_embedding must be q8");
  CV3_REQUIRE(s->workspace_floats >= kWsQ + H * NSMAX * 64 + H * NSMAX * 2 + I + 64, CV3_EINVAL,
              "workspace too small");
  if (smp) {
    CV3_REQUIRE(smp->ctl, CV3_EINVAL, "sampler: null control block");
    CV3_REQUIRE(smp->top_k >= 1 && smp->top_k <= kTopKMax, CV3_EUNSUPPORTED, "sampler: top_k %lld (1..%d)",
                (long long)smp->top_k, kTopKMax);
    CV3_REQUIRE(m->head.rows <= (int64_t)kSampleThreads * kSamplePerThread, CV3_EUNSUPPORTED,
                "sampler: vocabulary %lld above %d", (long long)m->head.rows, kSampleThreads * kSamplePerThread);
    CV3_REQUIRE(smp->win_size >= 0 && smp->speech_token_size >= 0, CV3_EINVAL, "sampler: window / stop ids");
  }
  hipStream_t st = stream_of(stream);
  const QW qkv = make_qw(m->qkv), o = make_qw(m->o), gu = make_qw(m->gate_up), dn = make_qw(m->down);
  const QW head = make_qw(m->head), emb = make_qw(m->embedding);
  // workspace: q [1024] | part_o [H, NSMAX, 64] | part_ml [H, NSMAX, 2] | h [I] (16-byte aligned pieces)
  float* qbuf = s->workspace;
  float* part_o = qbuf + kWsQ;
  float* part_ml = part_o + H * NSMAX * 64;
  float* hbuf = part_ml + ((H * NSMAX * 2 + 3) / 4) * 4;
  const float scale = 1.0f / sqrtf((float)dh);
  for (int64_t l = 0; l < m->layers; ++l) {
    float* kc = s->k_cache + l * Hk * s->cap * dh;
    float* vc = s->v_cache + l * Hk * s->cap * dh;
    QkvArgs qa{qkv, l * qkv.rows, s->x, m->ln1 + l * D, m->eps, m->qkv_bias + l * qkv.rows, (int)H, (int)Hk,
               (int)dh, m->rope_cos, m->rope_sin, s->pos, qbuf, kc, vc, s->cap};
    const int64_t pairs = (H + 2 * Hk) * dh / 2;
    const dim3 gq((unsigned)ceil_div(pairs, 16));
    const size_t lds = 1024 * sizeof(float);  // 8 lanes x 8 q8 chunks x 16 codes = 8 x 4 q4 chunks x 32 codes
    if (qkv.q4) {
      if (qkv.sf16)
        hipLaunchKernelGGL((k_dec_qkv<4, true, true>), gq, dim3(256), lds, st, qa);
      else
        hipLaunchKernelGGL((k_dec_qkv<4, false, true>), gq, dim3(256), lds, st, qa);
    } else if (qkv.sf16) {
      hipLaunchKernelGGL((k_dec_qkv<8, true, false>), gq, dim3(256), lds, st, qa);
    } else {
      hipLaunchKernelGGL((k_dec_qkv<8, false, false>), gq, dim3(256), lds, st, qa);
    }
    CV3_LAUNCHED();
    AttnArgs aa{qbuf, kc, vc, (int)H, (int)Hk, (int)dh, s->cap, s->pos, scale, part_o, part_ml};
    hipLaunchKernelGGL(k_dec_attn, dim3((unsigned)(s->cap / KCH), (unsigned)Hk), dim3(512), 0, st, aa);
    CV3_LAUNCHED();
    OprojArgs oa{o, l * o.rows, D, part_o, part_ml, (int)H, (int)dh, s->pos, s->x};
    const dim3 go((unsigned)ceil_div(D, 32));
    if (o.q4) {
      if (o.sf16)
        hipLaunchKernelGGL((k_dec_oproj<4, true, true>), go, dim3(256), lds, st, oa);
      else
        hipLaunchKernelGGL((k_dec_oproj<4, false, true>), go, dim3(256), lds, st, oa);
    } else if (o.sf16) {
      hipLaunchKernelGGL((k_dec_oproj<8, true, false>), go, dim3(256), lds, st, oa);
    } else {
      hipLaunchKernelGGL((k_dec_oproj<8, false, false>), go, dim3(256), lds, st, oa);
    }
    CV3_LAUNCHED();
    GemvArgs gb{gu, l * gu.rows, I, s->x, m->ln2 + l * D, m->eps, nullptr, hbuf, 2};
    if ((rc = gemv(gb, st))) return rc;
    GemvArgs gc{dn, l * dn.rows, D, hbuf, nullptr, 0.f, nullptr, s->x, 1};
    if ((rc = gemv(gc, st))) return rc;
  }
  GemvArgs gh{head, 0, head.rows, s->x, m->norm, m->eps, m->head_bias, s->logits, 0};
  if ((rc = gemv(gh, st))) return rc;
  NextArgs na{s->logits, head.rows, emb, s->x, s->pos, s->history, s->token};
  if (smp) {
    SampleArgs sa{na, smp->top_p, smp->rep_threshold, smp->top_k, smp->win_size, smp->speech_token_size,
                  smp->min_len, smp->strict_min_len, reinterpret_cast<int64_t*>(smp->ctl)};
    hipLaunchKernelGGL(k_dec_sample, dim3(1), dim3(1024), 0, st, sa);
  } else {
    hipLaunchKernelGGL(k_dec_next, dim3(1), dim3(1024), 0, st, na);
  }
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_qwen2_decode_step(const cv3_qwen2_model* m, const cv3_qwen2_state* s, cv3_stream_t stream) {
  CV3_ALIVE();
  return decode_step(m, s, nullptr, stream);
}

int cv3_qwen2_decode_step_sampled(const cv3_qwen2_model* m, const cv3_qwen2_state* s, const cv3_sampler* smp,
                                  cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(smp, CV3_EINVAL, "null sampler");
  return decode_step(m, s, smp, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The decode step without a caller workspace: its q / attention-partial /
// SwiGLU buffers live in a fixed device array, so a caller that cannot
// allocate (graph capture, a serving loop that forbids hipMalloc) still gets a
// step.  Nothing in that scratch must start at zero: every piece a kernel reads
// was written earlier in the same step (q and h by their GEMVs, the partials of
// chunks 0..pos/64 by the attention kernel, and only those are merged).
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t kScratchInterMax = 16384;
constexpr int64_t kScratchFloats = kWsQ + 16 * NSMAX * 64 + ((16 * NSMAX * 2 + 3) / 4) * 4 + kScratchInterMax + 64;
constexpr int kScratchDevices = 64;
}  // namespace

static __device__ __align__(256) float scratch[kScratchFloats];

namespace {
std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchDevices] = {};   // per device: the device address of `scratch`

// The device address of this device's copy of `scratch` (looked up once per device, with
// that device current); nullptr and the error text set on failure.
float* scratch_of_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    fail(CV3_EHIP, "decode scratch: no current device below %d", kScratchDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(CV3_EHIP, "hipGetSymbolAddress(decode scratch) failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  return g_scratch_ptr[dev];
}

// Calls of the no-workspace step on one device share its scratch.  The device's event marks
// where the last call's step ended; a call from another stream waits for it first, so calls from
// different streams or threads run one after another (under graph capture the graph's launches
// order them instead).  Created once per device at init (a library event: cv3_shutdown releases it).
struct ScratchOrder {
  void* ev = nullptr;
  hipStream_t last = nullptr;
  bool recorded = false;
};
static ScratchOrder g_scratch_order[kScratchDevices];
static std::mutex g_scratch_order_mu;
}  // namespace

extern "C" int cv3_event_create(void** ev);
extern "C" int cv3_event_record(void* ev, cv3_stream_t s);
extern "C" int cv3_stream_wait_event(cv3_stream_t s, void* ev);

namespace cv3 {
// Called by cv3_init with the selected device current.
int decode_scratch_setup() {
  if (!scratch_of_current_device()) return CV3_EHIP;
  int dev = 0;
  CV3_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_scratch_order_mu);
  ScratchOrder& o = g_scratch_order[dev];
  return o.ev ? CV3_OK : cv3_event_create(&o.ev);
}
}  // namespace cv3

extern "C" {

int cv3_qwen2_decode_step_noalloc(const cv3_qwen2_model* m, const cv3_qwen2_state* s, cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(m && s, CV3_EINVAL, "null model or state");
  const int64_t H = m->heads, I = m->inter;
  CV3_REQUIRE(H > 0 && H <= 16 && I > 0 && I <= kScratchInterMax, CV3_EINVAL,
              "decode step without workspace: %lld heads and intermediate size %lld exceed its fixed scratch "
              "(at most 16 heads and an intermediate size of %lld, %lld floats)",
              (long long)H, (long long)I, (long long)kScratchInterMax, (long long)kScratchFloats);
  float* ws = scratch_of_current_device();
  if (!ws) return CV3_EHIP;
  int dev = 0;
  CV3_HIP(hipGetDevice(&dev));
  hipStream_t st = stream_of(stream);
  CV3_REQUIRE(st, CV3_EINVAL, "%s", cv3_last_error());
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  CV3_HIP(hipStreamIsCapturing(st, &cs));
  const bool order = cs == hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lk(g_scratch_order_mu);
  ScratchOrder& o = g_scratch_order[dev];
  CV3_REQUIRE(o.ev, CV3_EINVAL, "decode step without workspace: device %d was not set up by cv3_init", dev);
  int rc;
  if (order && o.recorded && o.last != st && (rc = cv3_stream_wait_event(stream, o.ev))) return rc;
  cv3_qwen2_state t = *s;
  t.workspace = ws;
  t.workspace_floats = kScratchFloats;
  if ((rc = decode_step(m, &t, nullptr, stream))) return rc;
  if (order) {
    if ((rc = cv3_event_record(o.ev, stream))) return rc;
    o.last = st;
    o.recorded = true;
  }
  return CV3_OK;
}

// Words between replicas of an n-word vector: whole 4 KiB pages plus 512 bytes,
// so the copies start in different channels.
static int64_t replica_stride(int64_t n) { return (n + 511) / 512 * 512 + 64; }

static int64_t persist_words(const cv3_qwen2_model* m, int workgroups) {
  const int64_t D = m->hidden, R = (m->heads + 2 * m->kv_heads) * m->head_dim;
  return 2 * kRX * replica_stride(D) + 2 * R + 2 * replica_stride((int64_t)kPChunks * m->heads * kPPart) +
         2 * kRA * replica_stride(D) +
         2 * kRM * replica_stride(D) + 2 * kRH * replica_stride(m->inter) + 2 * (int64_t)workgroups;
}

int cv3_qwen2_persist_words(const cv3_qwen2_model* m, int workgroups, int64_t* words) {
  CV3_ALIVE();
  CV3_REQUIRE(m && words && workgroups > 0, CV3_EINVAL, "null model or output, or no workgroups");
  *words = persist_words(m, workgroups);
  return CV3_OK;
}

int cv3_qwen2_decode_step_persistent(const cv3_qwen2_model* m, const cv3_qwen2_state* s, const cv3_persist* p,
                                     int select, cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(m && s && p, CV3_EINVAL, "null model, state or exchange block");
  const int64_t H = m->heads, Hk = m->kv_heads, dh = m->head_dim, D = m->hidden, I = m->inter;
  CV3_REQUIRE(H > 0 && Hk > 0 && H % Hk == 0 && H / Hk <= 8 && dh == 64 && H * dh == D, CV3_EUNSUPPORTED,
              "persistent step: heads %lld / kv heads %lld / head dim %lld", (long long)H, (long long)Hk,
              (long long)dh);
  const bool q4 = m->qkv.kind == CV3_KIND_Q4;
  CV3_REQUIRE(D <= 1024 && D % 4 == 0 && I <= (q4 ? 6144 : 5120) && I >= kPMinG, CV3_EUNSUPPORTED,
              "persistent step: hidden %lld / inter %lld", (long long)D, (long long)I);
  CV3_REQUIRE(m->layers > 0 && m->layers * 8 + 8 <= 256, CV3_EUNSUPPORTED, "persistent step: %lld layers (at most 31)",
              (long long)m->layers);
  CV3_REQUIRE(s->cap > 0 && s->cap <= (int64_t)kPChunks * kPKeys, CV3_EUNSUPPORTED,
              "persistent step: cache capacity above %d positions", kPChunks * kPKeys);
  int rc;
  if ((rc = check_qw(m->qkv, "qkv", D))) return rc;
  if ((rc = check_qw(m->o, "o_proj", D))) return rc;
  if ((rc = check_qw(m->gate_up, "gate_up", D))) return rc;
  if ((rc = check_qw(m->down, "down", I))) return rc;
  if ((rc = check_qw(m->head, "llm_decoder", D))) return rc;
  if ((rc = check_qw(m->embedding, "speech_embedding", D))) return rc;
  // the body's four matrices share one kind (q8, or q4 with float16 scales); the head and the
  // speech embedding are q8; one scale dtype throughout
  const cv3_qweight* body[4] = {&m->qkv, &m->o, &m->gate_up, &m->down};
  for (const cv3_qweight* w : body)
    CV3_REQUIRE(w->kind == m->qkv.kind && (w->kind == CV3_KIND_Q8 || w->kind == CV3_KIND_Q4) &&
                    w->scale_dtype == m->qkv.scale_dtype,
                CV3_EUNSUPPORTED, "persistent step: body weights of one int8 or q4 kind and one scale dtype");
  CV3_REQUIRE(m->head.kind == CV3_KIND_Q8 && m->embedding.kind == CV3_KIND_Q8 &&
                  m->head.scale_dtype == m->qkv.scale_dtype && m->embedding.scale_dtype == m->qkv.scale_dtype &&
                  (!q4 || m->qkv.scale_dtype == CV3_F16),
              CV3_EUNSUPPORTED, "persistent step: q8 head and embedding with the body's scale dtype (f16 for q4)");
  CV3_REQUIRE(m->qkv.rows == (H + 2 * Hk) * dh && m->o.rows == D && m->gate_up.rows == 2 * I && m->down.rows == D &&
                  m->embedding.rows >= m->head.rows,
              CV3_EINVAL, "stacked weight rows do not match the geometry");
  int dev = 0, cus = 0;
  CV3_HIP(hipGetDevice(&dev));
  CV3_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const bool sf16 = m->qkv.scale_dtype == CV3_F16;
  // phase D on the matrix cores: q8 [gate; up] rows with one scale per row (per-channel)
  const bool mx = !q4 && m->gate_up.kp <= m->gate_up.block && D <= 64 * kMxSteps;
  const void* fn = q4     ? (const void*)k_dec_persist<true, true>
                   : mx   ? (sf16 ? (const void*)k_dec_persist<true, false, true> : (const void*)k_dec_persist<false, false, true>)
                   : sf16 ? (const void*)k_dec_persist<true, false>
                          : (const void*)k_dec_persist<false, false>;
  int per_cu = 0;
  CV3_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kPT, 0));
  const int G = p->workgroups > 0 ? p->workgroups : (int)std::min<int64_t>(std::min(cus, 256), I);
  // phases C and E at most 8 rows (one per wave) on min(kPOproj, G) and min(kPDown, G)
  CV3_REQUIRE(G >= kPMinG && G <= per_cu * cus && G <= I && (D + std::min(kPDown, G) - 1) / std::min(kPDown, G) <= 8,
              CV3_EUNSUPPORTED, "persistent step: %d workgroups (needs %d..%d resident, at most inter %lld)", G,
              kPMinG, per_cu * cus,
              (long long)I);
  CV3_REQUIRE((H + 2 * Hk) * dh / 2 <= 8LL * G && I <= 24LL * G && m->head.rows <= 32LL * G &&
                  H * kPChunks <= G && 2LL * G <= 8192,
              CV3_EUNSUPPORTED, "persistent step: too few workgroups for the geometry");
  CV3_REQUIRE(p->words && p->err && p->words_len >= persist_words(m, G), CV3_EINVAL,
              "persistent step: exchange words missing or too few");
  CV3_REQUIRE(p->epoch_base != 0, CV3_EINVAL, "persistent step: epoch base 0 is the cleared state");
  PersistArgs a{};
  a.qkv = make_qw(m->qkv);
  a.o = make_qw(m->o);
  a.gu = make_qw(m->gate_up);
  a.dn = make_qw(m->down);
  a.head = make_qw(m->head);
  a.emb = make_qw(m->embedding);
  a.ln1 = m->ln1;
  a.ln2 = m->ln2;
  a.norm = m->norm;
  a.qkv_bias = m->qkv_bias;
  a.head_bias = m->head_bias;
  a.rope_cos = m->rope_cos;
  a.rope_sin = m->rope_sin;
  a.layers = (int)m->layers;
  a.D = (int)D;
  a.H = (int)H;
  a.Hk = (int)Hk;
  a.dh = (int)dh;
  a.I = (int)I;
  a.eps = m->eps;
  a.scale = 1.0f / sqrtf((float)dh);
  a.k_cache = s->k_cache;
  a.v_cache = s->v_cache;
  a.cap = s->cap;
  a.pos = s->pos;
  a.token = s->token;
  a.history = s->history;
  a.x = s->x;
  a.logits = s->logits;
  const int64_t R = (H + 2 * Hk) * dh;
  uint64_t* wds = p->words;
  a.sx = replica_stride(D);
  a.sp = replica_stride((int64_t)kPChunks * H * kPPart);
  a.sm = replica_stride(D);
  a.sh = replica_stride(I);
  a.xb = wds;
  a.qkvb = a.xb + 2 * kRX * a.sx;
  a.pb = a.qkvb + 2 * R;
  a.sa = replica_stride(D);
  a.ab = a.pb + 2 * a.sp;
  a.mb = a.ab + 2 * kRA * a.sa;
  a.hb = a.mb + 2 * kRM * a.sm;
  a.arg = a.hb + 2 * kRH * a.sh;
  a.err = p->err;
  a.epoch_base = p->epoch_base;
  a.select = select ? 1 : 0;
  if (p->cooperative) {
    void* args[] = {&a};
    CV3_HIP(hipLaunchCooperativeKernel(fn, dim3((unsigned)G), dim3(kPT), args, 0, stream_of(stream)));
  } else {
    if (q4)
      hipLaunchKernelGGL((k_dec_persist<true, true>), dim3((unsigned)G), dim3(kPT), 0, stream_of(stream), a);
    else if (mx && sf16)
      hipLaunchKernelGGL((k_dec_persist<true, false, true>), dim3((unsigned)G), dim3(kPT), 0, stream_of(stream), a);
    else if (mx)
      hipLaunchKernelGGL((k_dec_persist<false, false, true>), dim3((unsigned)G), dim3(kPT), 0, stream_of(stream), a);
    else if (sf16)
      hipLaunchKernelGGL((k_dec_persist<true, false>), dim3((unsigned)G), dim3(kPT), 0, stream_of(stream), a);
    else
      hipLaunchKernelGGL((k_dec_persist<false, false>), dim3((unsigned)G), dim3(kPT), 0, stream_of(stream), a);
    CV3_LAUNCHED();
  }
  return CV3_OK;
}

int cv3_qwen2_select(const cv3_qwen2_model* m, const cv3_qwen2_state* s, const cv3_sampler* smp,
                     cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(m && s, CV3_EINVAL, "null model or state");
  int rc;
  if ((rc = check_qw(m->head, "llm_decoder", m->hidden))) return rc;
  if ((rc = check_qw(m->embedding, "speech_embedding", m->hidden))) return rc;
  CV3_REQUIRE(m->embedding.kind == CV3_KIND_Q8, CV3_EUNSUPPORTED, "speech_embedding must be q8");
  const QW head = make_qw(m->head), emb = make_qw(m->embedding);
  NextArgs na{s->logits, head.rows, emb, s->x, s->pos, s->history, s->token};
  hipStream_t st = stream_of(stream);
  if (smp) {
    CV3_REQUIRE(smp->ctl, CV3_EINVAL, "sampler: null control block");
    CV3_REQUIRE(smp->top_k >= 1 && smp->top_k <= kTopKMax, CV3_EUNSUPPORTED, "sampler: top_k %lld (1..%d)",
                (long long)smp->top_k, kTopKMax);
    CV3_REQUIRE(head.rows <= (int64_t)kSampleThreads * kSamplePerThread, CV3_EUNSUPPORTED,
                "sampler: vocabulary %lld above %d", (long long)head.rows, kSampleThreads * kSamplePerThread);
    CV3_REQUIRE(smp->win_size >= 0 && smp->speech_token_size >= 0, CV3_EINVAL, "sampler: window / stop ids");
    SampleArgs sa{na, smp->top_p, smp->rep_threshold, smp->top_k, smp->win_size, smp->speech_token_size,
                  smp->min_len, smp->strict_min_len, reinterpret_cast<int64_t*>(smp->ctl)};
    hipLaunchKernelGGL(k_dec_sample, dim3(1), dim3(kSampleThreads), 0, st, sa);
  } else {
    hipLaunchKernelGGL(k_dec_next, dim3(1), dim3(1024), 0, st, na);
  }
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_pcg64_random(int64_t* pcg, int64_t n, double* out, cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(pcg && n >= 0 && (n == 0 || out), CV3_EINVAL, "pcg64: null state or output");
  if (n == 0) return CV3_OK;
  hipLaunchKernelGGL(k_pcg64_random, dim3(1), dim3(1), 0, stream_of(stream), reinterpret_cast<uint64_t*>(pcg), n,
                     out);
  CV3_LAUNCHED();
  return CV3_OK;
}


int cv3_gemv_q8(const cv3_qweight* w, int64_t layer, const float* x, const float* rms_w, float eps, const float* bias,
                float* y, int mode, cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(w && x && y, CV3_EINVAL, "null argument");
  CV3_REQUIRE(mode >= 0 && mode <= 2, CV3_EINVAL, "gemv mode %d", mode);
  CV3_REQUIRE(layer >= 0, CV3_EINVAL, "negative layer");
  CV3_REQUIRE(mode != 2 || w->rows % 2 == 0, CV3_EINVAL, "SwiGLU needs [gate; up] rows");
  int rc;
  if ((rc = check_qw(*w, "gemv", w->k))) return rc;
  GemvArgs a{make_qw(*w), layer * w->rows, mode == 2 ? w->rows / 2 : w->rows, x, rms_w, eps, bias, y, mode};
  return gemv(a, stream_of(stream));
}

int cv3_qwen2_embed_token(const cv3_qwen2_model* m, const cv3_qwen2_state* s, cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(m && s, CV3_EINVAL, "null model or state");
  int rc;
  if ((rc = check_qw(m->embedding, "speech_embedding", m->hidden))) return rc;
  CV3_REQUIRE(m->embedding.kind == CV3_KIND_Q8, CV3_EUNSUPPORTED, "speech_embedding must be q8");
  hipLaunchKernelGGL(k_dec_embed, dim3(1), dim3(256), 0, stream_of(stream), make_qw(m->embedding), s->token, s->x);
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // extern "C"
