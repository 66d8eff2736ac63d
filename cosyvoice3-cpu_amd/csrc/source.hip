// The HiFT vocoder's front half after its F0 convolutions (cv3cpu/models/hift.py:56-111,
// 212-218): the F0 classifier and the neural-source-filter excitation, so that
// mel -> waveform runs without a host round trip.
//
//   classifier (hift.py:69-72, 216): f0[t] = float32(|sum_c x[c, t] w[c] + b|), the
//     sum in float64 over float32 activations (the reference's matmul promotes to
//     float64 against its float64 weight; inference() then casts f0 to float32).
//   phase (hift.py:98-100): rad[t, h] = ((f0[t] (h + 1)) / sr) mod 1 in float64 and
//     phase = cumsum_t(rad) * 2 pi * up.  The running sum is taken in frame order by
//     one lane per harmonic, as numpy's cumsum does, so the phases are bit-identical.
//   source (hift.py:101-111): per sample i of frame t = i / up,
//     s_h = float32(sin(phase[t, h])) * alpha, uv = f0[t] > threshold,
//     amp = uv sigma + (1 - uv) (alpha / 3), src_h = s_h uv + amp noise[i, h],
//     out[i] = tanh(sum_h src_h w_h + b).
//   The float32 products and sums are evaluated one rounding at a time, as NumPy
//   evaluates them (no contraction into fused multiply-adds).
#include "common.hpp"

using namespace cv3;

namespace {

constexpr int kMaxHarmonics = 16;
constexpr int kPhaseFrames = 256;  // frames per pass of the phase scan

__global__ __launch_bounds__(256) void k_f0_classify(const float* __restrict__ x, int64_t c, int64_t t, int64_t x_cs,
                                                     int64_t x_ts, const float* __restrict__ w,
                                                     const float* __restrict__ b, float* __restrict__ f0) {
  const int lane = threadIdx.x & 63;
  const int64_t fr = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (fr >= t) return;
  double acc = 0.0;
  for (int64_t ch = lane; ch < c; ch += 64) acc += (double)x[ch * x_cs + fr * x_ts] * (double)w[ch];
  acc = wave_sum_d(acc);
  if (lane == 0) f0[fr] = (float)fabs(acc + (double)b[0]);
}

__global__ __launch_bounds__(256) void k_nsf_phase(const float* __restrict__ f0, int64_t t, int nh, double sr,
                                                   double up, double* __restrict__ phase) {
  __shared__ double rad[kPhaseFrames * kMaxHarmonics];
  const int tid = threadIdx.x;
  double cum = 0.0;  // lane h < nh: running sum of harmonic h
  for (int64_t t0 = 0; t0 < t; t0 += kPhaseFrames) {
    const int n = (int)min((int64_t)kPhaseFrames, t - t0);
    if (tid < n) {
      const double f = (double)f0[t0 + tid];
      for (int h = 0; h < nh; ++h) rad[tid * nh + h] = fmod(f * (double)(h + 1) / sr, 1.0);
    }
    __syncthreads();
    if (tid < nh) {
      for (int j = 0; j < n; ++j) {
        cum += rad[j * nh + tid];
        phase[(t0 + j) * nh + tid] = cum * (2.0 * M_PI) * up;
      }
    }
    __syncthreads();
  }
}

struct SourceArgs {
  const float* f0;
  const double* phase;
  const float* noise;  // [up * t, nh]
  const float* lw;     // [nh]
  const float* lb;     // [1]
  float* out;          // [up * t]
  int64_t t;
  int up, nh;
  float alpha, alpha3, sigma, threshold;
};

__global__ __launch_bounds__(256) void k_nsf_source(SourceArgs a) {
#pragma clang fp contract(off)
  __shared__ float sines[kMaxHarmonics];
  const int64_t fr = blockIdx.x;
  if (threadIdx.x < a.nh) sines[threadIdx.x] = (float)sin(a.phase[fr * a.nh + threadIdx.x]) * a.alpha;
  __syncthreads();
  const float uv = a.f0[fr] > a.threshold ? 1.f : 0.f;
  const float amp = uv * a.sigma + (1.f - uv) * a.alpha3;
  const float bias = a.lb[0];
  for (int j = threadIdx.x; j < a.up; j += blockDim.x) {
    const int64_t i = fr * a.up + j;
    const float* nz = a.noise + i * a.nh;
    float acc = 0.f;
    for (int h = 0; h < a.nh; ++h) {
      const float src = sines[h] * uv + amp * nz[h];
      acc = fmaf(src, a.lw[h], acc);
    }
    a.out[i] = tanhf(acc + bias);
  }
}

}  // namespace

extern "C" {

int cv3_f0_classify(const float* x, int64_t c, int64_t t, int64_t x_cs, int64_t x_ts, const float* w, const float* b,
                    float* f0, cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(c > 0 && t >= 0, CV3_EINVAL, "f0 classifier: %lld channels, %lld frames", (long long)c, (long long)t);
  if (t == 0) return CV3_OK;
  CV3_REQUIRE(x && w && b && f0, CV3_EINVAL, "f0 classifier: null argument");
  hipLaunchKernelGGL(k_f0_classify, dim3((unsigned)ceil_div(t, 4)), dim3(256), 0, stream_of(stream), x, c, t, x_cs,
                     x_ts, w, b, f0);
  CV3_LAUNCHED();
  return CV3_OK;
}

int cv3_nsf_source(const float* f0, int64_t t, int up, int harmonics, double sampling_rate, double alpha, double sigma,
                   double voiced_threshold, const float* noise, const float* l_w, const float* l_b, double* phase,
                   float* out, cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(t >= 0 && up > 0, CV3_EINVAL, "nsf source: %lld frames, upsampling %d", (long long)t, up);
  CV3_REQUIRE(harmonics > 0 && harmonics <= kMaxHarmonics, CV3_EUNSUPPORTED, "nsf source: %d harmonics (at most %d)",
              harmonics, kMaxHarmonics);
  CV3_REQUIRE(sampling_rate > 0.0, CV3_EINVAL, "nsf source: sampling rate %g", sampling_rate);
  if (t == 0) return CV3_OK;
  CV3_REQUIRE(f0 && noise && l_w && l_b && phase && out, CV3_EINVAL, "nsf source: null argument");
  hipStream_t st = stream_of(stream);
  hipLaunchKernelGGL(k_nsf_phase, dim3(1), dim3(256), 0, st, f0, t, harmonics, sampling_rate, (double)up, phase);
  CV3_LAUNCHED();
  SourceArgs a;
  a.f0 = f0;
  a.phase = phase;
  a.noise = noise;
  a.lw = l_w;
  a.lb = l_b;
  a.out = out;
  a.t = t;
  a.up = up;
  a.nh = harmonics;
  // Python floats meet float32 arrays as float32 values; alpha / 3 is formed in
  // double first (hift.py:105)
  a.alpha = (float)alpha;
  a.alpha3 = (float)(alpha / 3.0);
  a.sigma = (float)sigma;
  a.threshold = (float)voiced_threshold;
  hipLaunchKernelGGL(k_nsf_source, dim3((unsigned)t), dim3(256), 0, st, a);
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // extern "C"
