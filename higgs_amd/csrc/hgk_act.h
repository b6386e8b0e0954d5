// hgk_act.h -- MLX's SwiGLU for 16-bit types, shared by the GLU kernels and
// the fused expert projection:
//   out = round_T(round_T(g * round_T(sigmoid(g))) * u)
// with MLX's sigmoid (y = 1/(1+exp(|g|)); g < 0 ? y : 1-y) and polynomial exp.
// The exact sigmoid costs ~40 VALU operations, so the value is first formed
// with the hardware exp2 and reciprocal and kept only when it cannot round
// differently: |g| <= 64 (there the fast value is within 3 f32 ulps of the
// exact one, measured over every 16-bit input) and it is more than
// kTieWindow ulps from a rounding tie of T. Everything else takes the exact
// path; a 16-bit input has only 65536 values, and the tests check them all.
#pragma once

#include "hgk_common.h"

namespace hgk {

constexpr int kTieWindow = 16;  // f32 ulps; the fast sigmoid errs by <= 3

// True when the f32 value `b` (bits) lies within kTieWindow ulps of a value
// halfway between two neighbours of T, or where T's rounding is not decided
// by the low bits alone (f16 subnormal range).
template <class X>
__device__ inline bool near_tie(uint32_t b) {
  if constexpr (X::kCode == DT_BF16) {
    const int d = (int)(b & 0xffffu) - 0x8000;
    return d <= kTieWindow && d >= -kTieWindow;
  } else {
    const int d = (int)(b & 0x1fffu) - 0x1000;
    return (d <= kTieWindow && d >= -kTieWindow) || (b & 0x7fffffffu) < 0x38800000u;
  }
}

// Fast sigmoid with MLX's branch structure; *slow is set when the result may
// round differently from the exact one.
template <class X>
__device__ inline float sigmoid16_fast(float g, bool* slow) {
  const float e = __builtin_amdgcn_exp2f(fabsf(g) * 1.4426950408889634f);
  const float y = __builtin_amdgcn_rcpf(1.0f + e);
  const float sg = g < 0.0f ? y : 1.0f - y;
  *slow = !(fabsf(g) <= 64.0f) || near_tie<X>(f2u(sg));  // !(<=) also catches NaN
  return sg;
}

// N SwiGLU outputs round_T(round_T(g*round_T(sigmoid(g))) * u) for 16-bit T,
// bit-identical to the exact MLX composition: all fast sigmoids first, then
// one (rarely taken) branch that redoes the flagged ones exactly.
template <class X, int N>
__device__ inline void swiglu16(const float* g, const float* u, float* o) {
  float sg[N];
  bool fl[N];
  bool any = false;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    sg[e] = sigmoid16_fast<X>(g[e], &fl[e]);
    any |= fl[e];
  }
  if (any) {
#pragma unroll
    for (int e = 0; e < N; ++e)
      if (fl[e]) sg[e] = mlx_sigmoid(g[e]);
  }
#pragma unroll
  for (int e = 0; e < N; ++e) o[e] = X::round(X::round(g[e] * X::round(sg[e])) * u[e]);
}

// The sigmoids of two values of a 16-bit type X, rounded to X, as MLX's exact
// sigmoid rounds them: the hardware exp2 / reciprocal form where it provably
// rounds the same way (sigmoid16_fast), the exact form elsewhere.
template <class X>
__device__ inline void sigmoid2_rounded(float z0, float z1, float& s0, float& s1) {
  if constexpr (X::kBytes == 2) {
    bool f0, f1;
    s0 = sigmoid16_fast<X>(z0, &f0);
    s1 = sigmoid16_fast<X>(z1, &f1);
    if (f0) s0 = mlx_sigmoid(z0);
    if (f1) s1 = mlx_sigmoid(z1);
  } else {
    s0 = mlx_sigmoid(z0);
    s1 = mlx_sigmoid(z1);
  }
  round2<X>(s0, s1);
}

// One GLU output before its rounding to the output type: SwiGLU (as above,
// for 16-bit and f32 inputs) or GeGLU, which runs in f32: 0.5*g*(1+tanh(k0*(g
// + k1*g^3))) * u evaluated as g / (1 + exp(-2*k0*(g + k1*g^3))) * u with the
// hardware exp2 and reciprocal.
template <class X, int ACT>
__device__ inline float glu1(float g, float u) {
  if constexpr (ACT == 0) {  // HGK_ACT_SILU
    if constexpr (X::kBytes == 2) {
      float o;
      swiglu16<X, 1>(&g, &u, &o);
      return o;
    } else {
      const float sg = X::round(mlx_sigmoid(g));
      const float s = X::round(g * sg);
      return X::round(s * u);
    }
  } else {
    // exp(-2*k0*(g + k1*g^3)) = exp2(g * (c1 + c2*g^2)) with k0 = sqrt(2/pi),
    // k1 = 0.044715, c1 = -2*k0*log2(e), c2 = c1*k1: three VALU operations
    // before the exp2 instead of six
    const float c1 = -2.302208198144325f, c2 = -0.1029432395800235f;
    const float z = g * __builtin_fmaf(g * g, c2, c1);
    const float e = __builtin_amdgcn_exp2f(z);
    const float gl = g * __builtin_amdgcn_rcpf(1.0f + e);
    return gl * u;
  }
}

}  // namespace hgk
