// Activations of the FFN steps on either side of a linear, evaluated in f32
// from bf16 operands and rounded once by the caller (and the bf16 sum of two
// input gradients of one shared input):
//   GELU (exact, erf form): components.py:159-160, bert/model.py:249;
//   SiLU-gated product silu(gate) * up: qwen3_vl/text.py:202.
// The same functions serve the GEMM epilogues and the elementwise kernels,
// so both produce identical bits.
#pragma once

#include "common.h"

namespace rpx {

// Output transforms applied to a linear's rounded output v.
enum ActMode : int {
  kActNone = 0,
  kActGeluFwd = 1,     // out = gelu(v); the pre-activation v is stored too
  kActSiluMulFwd = 2,  // out = silu(gate) * v; v (the up projection) is stored too
  kActGeluBwd = 3,     // out = v * gelu'(z)
  kActSiluMulBwd = 4,  // out = v * silu(gate) (d up), out2 = v * up * silu'(gate) (d gate)
  kActAddBwd = 5,      // out = v + z: an input gradient added to the one accumulated so far
};

constexpr float kInvSqrt2 = 0.70710678118654752440f;
constexpr float kInvSqrt2Pi = 0.39894228040143267794f;

// e^x through the hardware base-2 exponential (v_exp_f32).
__device__ __forceinline__ float act_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f);
}

__device__ __forceinline__ float act_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// erfc(x) for x >= 0 by the Chebyshev fit of Press et al., Numerical Recipes
// (2nd ed., sec. 6.2, "erfcc"): t = 1 / (1 + x / 2),
// erfc(x) = t exp(-x^2 + P(t)), fractional error < 1.2e-7 everywhere, so the
// tail stays accurate relative to its own size. One exp, one reciprocal and
// nine fma: the epilogues run it per output element.
__device__ __forceinline__ float act_erfc_pos(float x) {
  const float t = act_rcp(1.0f + 0.5f * x);
  float p = 0.17087277f;
  p = __builtin_fmaf(p, t, -0.82215223f);
  p = __builtin_fmaf(p, t, 1.48851587f);
  p = __builtin_fmaf(p, t, -1.13520398f);
  p = __builtin_fmaf(p, t, 0.27886807f);
  p = __builtin_fmaf(p, t, -0.18628806f);
  p = __builtin_fmaf(p, t, 0.09678418f);
  p = __builtin_fmaf(p, t, 0.37409196f);
  p = __builtin_fmaf(p, t, 1.00002368f);
  p = __builtin_fmaf(p, t, -1.26551223f);
  return t * act_exp(__builtin_fmaf(-x, x, p));
}

// Phi(z) = erfc(-z / sqrt 2) / 2, taken from the small side: no
// cancellation for negative z, where 1 + erf(z / sqrt 2) would keep only a
// few bits of a tiny result.
__device__ __forceinline__ float act_normal_cdf(float z) {
  const float u = -z * kInvSqrt2;
  const float e = 0.5f * act_erfc_pos(fabsf(u));
  return u >= 0.0f ? e : 1.0f - e;
}

__device__ __forceinline__ float act_gelu(float z) { return z * act_normal_cdf(z); }

// d/dz [z Phi(z)] = Phi(z) + z phi(z)
__device__ __forceinline__ float act_gelu_grad(float z) {
  return act_normal_cdf(z) + z * (act_exp(-0.5f * z * z) * kInvSqrt2Pi);
}

__device__ __forceinline__ float act_sigmoid(float g) { return act_rcp(1.0f + act_exp(-g)); }

// silu'(g) = s (1 + g (1 - s)) with s = sigmoid(g) and 1 - s = sigmoid(-g)
// taken directly (no cancellation for large g)
__device__ __forceinline__ float act_silu_grad(float g, float s) {
  return s * (1.0f + g * act_sigmoid(-g));
}

// One output element (two for kActSiluMulBwd) from v and the auxiliary
// operands a0 (z or gate) and a1 (up).
template <int ACT>
__device__ __forceinline__ float act_apply(float v, float a0, float a1, float* second) {
  if constexpr (ACT == kActGeluFwd) {
    return act_gelu(v);
  } else if constexpr (ACT == kActSiluMulFwd) {
    return a0 * act_sigmoid(a0) * v;
  } else if constexpr (ACT == kActGeluBwd) {
    return v * act_gelu_grad(a0);
  } else if constexpr (ACT == kActSiluMulBwd) {
    const float s = act_sigmoid(a0);
    *second = v * a1 * act_silu_grad(a0, s);
    return v * (a0 * s);
  } else if constexpr (ACT == kActAddBwd) {
    return v + a0;
  } else {
    return v;
  }
}

}  // namespace rpx
