// Short-time Fourier transforms for small n_fft (the vocoder uses 16):
// direct DFTs with twiddles computed in fp64, reflect padding by index mapping.
//
//   stft  (cv3cpu/ops.py:346-355): reflect-pad n_fft/2, frames at hop, window,
//         one-sided DFT -> re/im planes (F, frames).
//   istft (cv3cpu/ops.py:358-377): one-sided inverse DFT (imaginary parts of the
//         DC and Nyquist bins ignored, like irfft), window, overlap-add, divide by
//         the summed squared window where it exceeds 1e-11, trim n_fft/2.
//   HiFT head (cv3cpu/models/hift.py:204-210): magnitude clip(exp(min(x, 80)), 100)
//         and phase sin(x) from the conv_post output, then the istft and a clip
//         to +-audio_limit.
#include "common.hpp"

using namespace cv3;

namespace {

__device__ __forceinline__ int64_t reflect(int64_t i, int64_t n) {
  // numpy "reflect" (edge not repeated); valid for |overhang| < n
  if (i < 0) i = -i;
  if (i >= n) i = 2 * (n - 1) - i;
  return i;
}

__global__ void k_stft(const float* __restrict__ x, int64_t n, int n_fft, int hop, const float* __restrict__ win,
                       int center, int64_t frames, float* __restrict__ re, float* __restrict__ im) {
  const int nbins = n_fft / 2 + 1;
  const int64_t total = frames * nbins;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t f = i % frames;
    const int kbin = (int)(i / frames);
    float sr = 0.f, si = 0.f;
    for (int j = 0; j < n_fft; ++j) {
      int64_t u = f * hop + j - (center ? n_fft / 2 : 0);
      if (center) u = reflect(u, n);
      const float v = x[u] * win[j];
      const double ang = -2.0 * M_PI * (double)((int64_t)kbin * j % n_fft) / (double)n_fft;
      sr = fmaf(v, (float)cos(ang), sr);
      si = fmaf(v, (float)sin(ang), si);
    }
    re[(int64_t)kbin * frames + f] = sr;
    im[(int64_t)kbin * frames + f] = si;
  }
}

// Per-frame windowed time samples: fr[f, j] = win[j] * irfft(X_f)[j].
// mode 0: X from (re, im) planes.  mode 1: HiFT head, X from log-magnitude /
// phase planes: mag = min(exp(min(x, 80)), 100), ph = sin(y), X = mag (cos ph + i sin ph).
__global__ void k_irfft_frames(const float* __restrict__ a, const float* __restrict__ b, int64_t frames, int n_fft,
                               const float* __restrict__ win, int mode, float* __restrict__ fr) {
  const int nbins = n_fft / 2 + 1;
  const int64_t total = frames * n_fft;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t f = i / n_fft;
    const int j = (int)(i % n_fft);
    float acc = 0.f;
    for (int kbin = 0; kbin < nbins; ++kbin) {
      float xr, xi;
      if (mode == 0) {
        xr = a[(int64_t)kbin * frames + f];
        xi = b[(int64_t)kbin * frames + f];
      } else {
        const float mag = fminf(expf(fminf(a[(int64_t)kbin * frames + f], 80.0f)), 100.0f);
        const float ph = sinf(b[(int64_t)kbin * frames + f]);
        xr = mag * cosf(ph);
        xi = mag * sinf(ph);
      }
      const bool edge = kbin == 0 || (2 * kbin == n_fft);
      const double ang = 2.0 * M_PI * (double)((int64_t)kbin * j % n_fft) / (double)n_fft;
      const float c = (float)cos(ang), s = (float)sin(ang);
      const float term = edge ? xr * c : 2.0f * (xr * c - xi * s);
      acc += term;
    }
    fr[i] = (acc / (float)n_fft) * win[j];
  }
}

// Overlap-add of frames (stride hop), envelope normalisation, centre trim, clip.
__global__ void k_overlap_add(const float* __restrict__ fr, int64_t frames, int n_fft, int hop,
                              const float* __restrict__ win, int64_t offset, int64_t out_len, int64_t natural,
                              float limit, float* __restrict__ y) {
  const int64_t total_len = (frames - 1) * hop + n_fft;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < out_len; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t sidx = i + offset;
    float acc = 0.f, env = 0.f;
    if (sidx < total_len && i < natural) {
      // frames f with 0 <= sidx - f*hop < n_fft, visited in increasing j = sidx - f*hop
      int64_t f_hi = sidx / hop;
      if (f_hi > frames - 1) f_hi = frames - 1;
      for (int64_t f = f_hi; f >= 0; --f) {
        const int64_t j = sidx - f * hop;
        if (j >= n_fft) break;
        acc += fr[f * n_fft + j];
        env += win[j] * win[j];
      }
      if (fabsf(env) > 1e-11f) acc = acc / env;
    }
    if (limit > 0.f) acc = fminf(fmaxf(acc, -limit), limit);
    y[i] = acc;
  }
}

}  // namespace

extern "C" {

int cv3_stft(const float* x, int64_t n, int n_fft, int hop, const float* win, int center, float* re, float* im,
             int64_t* frames_ptr, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(n_fft > 0 && hop > 0, CV3_EINVAL, "bad stft geometry");
  CV3_REQUIRE(!center || n > n_fft / 2, CV3_EINVAL, "reflect padding needs more than n_fft/2 samples");
  const int64_t padded = n + (center ? 2 * (n_fft / 2) : 0);
  const int64_t frames = padded >= n_fft ? 1 + (padded - n_fft) / hop : 0;
  if (frames_ptr) *frames_ptr = frames;
  if (frames <= 0 || !re) return CV3_OK;
  const int64_t total = frames * (n_fft / 2 + 1);
  hipLaunchKernelGGL(k_stft, dim3((unsigned)std::min<int64_t>(ceil_div(total, 256), 65536)), dim3(256), 0,
                     stream_of(s), x, n, n_fft, hop, win, center, frames, re, im);
  CV3_LAUNCHED();
  return CV3_OK;
}

// mode 0: (re, im) spectrum planes; mode 1: HiFT head (log-magnitude, phase-source)
// planes with the +-limit clip (limit <= 0 disables the clip).  `frame_buf` is a
// caller-provided scratch of frames * n_fft floats.  Output length: (frames-1)*hop
// when centred (the torch.istft convention without `length`), else the full
// overlap-add length; `length` >= 0 truncates or zero-pads to that many samples.
int cv3_istft(int mode, const float* a, const float* b, int64_t frames, int n_fft, int hop, const float* win,
              int center, int64_t length, float limit, float* frame_buf, float* y, int64_t* out_len_ptr,
              cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(n_fft > 0 && n_fft % 2 == 0 && hop > 0, CV3_EINVAL, "istft needs an even n_fft");
  CV3_REQUIRE(frames > 0, CV3_EINVAL, "istft of zero frames");
  const int64_t total = (frames - 1) * hop + n_fft;
  const int64_t offset = center ? n_fft / 2 : 0;
  const int64_t natural = center ? total - 2 * (n_fft / 2) : total;
  const int64_t out_len = length >= 0 ? length : natural;
  if (out_len_ptr) *out_len_ptr = out_len;
  if (!y) return CV3_OK;
  hipStream_t st = stream_of(s);
  hipLaunchKernelGGL(k_irfft_frames, dim3((unsigned)std::min<int64_t>(ceil_div(frames * n_fft, 256), 65536)),
                     dim3(256), 0, st, a, b, frames, n_fft, win, mode, frame_buf);
  CV3_LAUNCHED();
  // samples past the natural length are zero padding (ops.py:375-377)
  hipLaunchKernelGGL(k_overlap_add, dim3((unsigned)std::min<int64_t>(ceil_div(out_len, 256), 65536)), dim3(256), 0,
                     st, frame_buf, frames, n_fft, hop, win, offset, out_len, natural, limit, y);
  CV3_LAUNCHED();
  return CV3_OK;
}

}  // extern "C"
