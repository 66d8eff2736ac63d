// Device helpers shared by the decode kernels (decode.hip: the five-kernel step
// and the one-launch step over the stacked weights; decode_stream.hip: the
// one-launch step over per-workgroup weight streams), and the wave sums of the
// one-wave-per-row layer norm (elementwise.hip).
#pragma once

#include "common.hpp"

namespace {

constexpr float kLog2E = 1.4426950408889634f;
constexpr int kPKeys = 128;              // keys per attention item
constexpr int kPChunks = 8;              // attention items per head: cache <= 1024 positions
constexpr int kPSpin = 1 << 18;          // polls (each with a short sleep) before a wait gives up
constexpr int kPPart = 66;               // words per attention partial: m, l, o[64]

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
// s_waitcnt immediate that waits for all but n vector-memory operations (gfx9 field layout)
#define CV3_VMCNT(n) (((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

struct QW {            // one stacked weight: layer l, row r at q + (l * rows + r) * row_bytes
  const int8_t* q;     // row_bytes = kp (q8) or kp / 2 (q4)
  const void* scales;  // [layers * rows, kp / block]
  int64_t rows, k, kp, block;
  int sf16;
  int q4;
};

__device__ __forceinline__ float sc_at(const QW& w, int64_t row, int64_t kk) {
  const int64_t nb = w.kp / w.block;
  const int64_t i = row * nb + kk / w.block;
  return w.sf16 ? __half2float(reinterpret_cast<const __half*>(w.scales)[i])
                : reinterpret_cast<const float*>(w.scales)[i];
}

// Scale of 16-code chunk c of a row whose scales start at `srow`: 32-bit index math
// (cpb = block / 16 chunks per scale).
__device__ __forceinline__ float sc_chunk(const QW& w, const void* srow, unsigned c, unsigned cpb) {
  const unsigned i = c / cpb;
  return w.sf16 ? __half2float(reinterpret_cast<const __half*>(srow)[i]) : reinterpret_cast<const float*>(srow)[i];
}

// Wave reductions through DPP row permutations (quad swaps, half-row and row
// mirrors: every lane ends with its 16-lane row's result) and four lane reads:
// no LDS round trips, unlike shuffles.  Called with every lane of the wave active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
  return ((uint64_t)dpp32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp32<CTRL>((uint32_t)v);
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), lane) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
}
// Orders one wave's LDS accesses around a point where its lanes exchange values
// (the wave's own LDS operations complete in order; this keeps the compiler from
// moving them and waits for the outstanding ones).  Not a workgroup barrier.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}
__device__ __forceinline__ double readlane_d(double v, int lane) {
  const int64_t b = __double_as_longlong(v);
  return __longlong_as_double(((int64_t)__builtin_amdgcn_readlane((int)(b >> 32), lane) << 32) |
                              (uint32_t)__builtin_amdgcn_readlane((int)b, lane));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
  k = max(k, dpp64<kDppXor1>(k));
  k = max(k, dpp64<kDppXor2>(k));
  k = max(k, dpp64<kDppHalfMirror>(k));
  k = max(k, dpp64<kDppMirror>(k));
  return max(max(readlane64(k, 0), readlane64(k, 16)), max(readlane64(k, 32), readlane64(k, 48)));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, __uint_as_float(dpp32<kDppXor1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp32<kDppXor2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp32<kDppHalfMirror>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp32<kDppMirror>(__float_as_uint(v))));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __uint_as_float(dpp32<kDppXor1>(__float_as_uint(v)));
  v += __uint_as_float(dpp32<kDppXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp32<kDppHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp32<kDppMirror>(__float_as_uint(v)));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ void ll_put(uint64_t* p, float v, uint32_t e) {
  __hip_atomic_store(p, ((uint64_t)e << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave sum in every lane without lane reads: DPP within each 16-lane row, then the
// row-pair and half swaps of gfx950 (v_permlane16_swap / v_permlane32_swap).  The
// additions group as ((row0 + row1) + (row2 + row3)), as in wave_sum_dpp, so the
// two give the same bits.
__device__ __forceinline__ float wave_sum_swap(float v) {
  v += __uint_as_float(dpp32<kDppXor1>(__float_as_uint(v)));
  v += __uint_as_float(dpp32<kDppXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp32<kDppHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp32<kDppMirror>(__float_as_uint(v)));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// float -> unsigned with the same order (NaN lowest), for an argmax key
__device__ __forceinline__ uint32_t ord_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return f != f ? 0u : (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

inline QW make_qw(const cv3_qweight& w) {
  QW q;
  q.q = reinterpret_cast<const int8_t*>(w.q);
  q.scales = w.scales;
  q.rows = w.rows;
  q.k = w.k;
  q.kp = w.kp;
  q.block = w.block;
  q.sf16 = w.scale_dtype == CV3_F16;
  q.q4 = w.kind == CV3_KIND_Q4;
  return q;
}

inline int check_qw(const cv3_qweight& w, const char* what, int64_t k) {
  CV3_REQUIRE(w.q && w.scales, CV3_EINVAL, "%s: missing weight", what);
  CV3_REQUIRE(w.kind == CV3_KIND_Q8 || w.kind == CV3_KIND_Q4, CV3_EINVAL, "%s: kind %d is neither q8 nor q4", what,
              w.kind);
  CV3_REQUIRE(w.k == k, CV3_EINVAL, "%s: K is %lld, expected %lld", what, (long long)w.k, (long long)k);
  const int64_t cpc = w.kind == CV3_KIND_Q4 ? 32 : 16;  // codes per 16-byte chunk
  CV3_REQUIRE(w.block > 0 && w.block % cpc == 0 && w.kp % w.block == 0 && w.kp >= w.k && w.kp % cpc == 0,
              CV3_EINVAL, "%s: block %lld / padded K %lld must be multiples of %lld", what, (long long)w.block,
              (long long)w.kp, (long long)cpc);
  CV3_REQUIRE((uintptr_t)w.q % 16 == 0, CV3_EINVAL, "%s: codes must be 16-byte aligned", what);
  CV3_REQUIRE(w.scale_dtype == CV3_F16 || w.scale_dtype == CV3_F32, CV3_EINVAL, "%s: scale dtype", what);
  return CV3_OK;
}

}  // namespace
