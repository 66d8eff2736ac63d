// Activation and linear-epilogue helpers shared by the GEMV, GEMM and conv
// kernels.  Each activation restates the float32 formula of the reference
// (cv3cpu/ops.py:30-81) with the accurate device libm (no fast-math paths).
#pragma once

#include "common.hpp"

namespace cv3 {

__device__ __forceinline__ float act_silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float act_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float act_gelu_tanh(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))   (ops.py:41-43)
  const float c = 0.7978845608028654f;
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}
__device__ __forceinline__ float act_gelu(float x) {
  // 0.5 x (1 + erf(x / sqrt 2)) with the Abramowitz-Stegun 7.1.26 erf (ops.py:46-60)
  const float z = x / 1.4142135623730951f;
  const float s = z > 0.f ? 1.f : (z < 0.f ? -1.f : 0.f);
  const float a = fabsf(z);
  const float t = 1.0f / (1.0f + 0.3275911f * a);
  const float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
  return 0.5f * x * (1.0f + s * (1.0f - poly * expf(-a * a)));
}
__device__ __forceinline__ float act_mish(float x) {
  // x tanh(softplus(x)), softplus = x above 20   (ops.py:63-66)
  const float sp = x > 20.f ? x : log1pf(expf(fminf(x, 20.f)));
  return x * tanhf(sp);
}
__device__ __forceinline__ float act_elu(float x, float alpha) { return x > 0.f ? x : alpha * expm1f(fminf(x, 0.f)); }
__device__ __forceinline__ float act_leaky(float x, float slope) { return x >= 0.f ? x : x * slope; }

__device__ __forceinline__ float apply_act(int act, float v, float param) {
  switch (act) {
    case CV3_ACT_SILU: return act_silu(v);
    case CV3_ACT_SIGMOID: return act_sigmoid(v);
    case CV3_ACT_GELU_TANH: return act_gelu_tanh(v);
    case CV3_ACT_GELU: return act_gelu(v);
    case CV3_ACT_MISH: return act_mish(v);
    case CV3_ACT_ELU: return act_elu(v, param);
    case CV3_ACT_LEAKY: return act_leaky(v, param);
    case CV3_ACT_TANH: return tanhf(v);
    default: return v;
  }
}

// y = residual + gate * act(v); `act_applied` skips the activation.
__device__ __forceinline__ float apply_epilogue(const cv3_epilogue& e, float v, int64_t row, int64_t col,
                                                bool act_applied) {
  if (!act_applied) v = apply_act(e.act, v, e.act_param);
  if (e.gate) v = e.gate[(row / (e.rows_per_gate > 0 ? e.rows_per_gate : 1)) * e.gate_stride + col] * v;
  if (e.residual) v = e.residual[row * e.ld_res + col] + v;
  return v;
}

}  // namespace cv3
