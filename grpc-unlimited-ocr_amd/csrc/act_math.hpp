// act_math.hpp: the activations' arithmetic, shared by the elementwise
// kernels (act.hip) and the projections' activation epilogue (gemm.hip), so
// that an activation fused into a product's epilogue is bitwise the
// elementwise op.

#pragma once

#include <hip/hip_runtime.h>

namespace uocr_rocm {

// GELU(x) = x Phi(x), Phi the standard normal CDF, from the upper tail
// Q(t) = Phi(-t) = 2^P(t): Phi(x) = 1 - Q(|x|) for x >= 0 and Q(|x|) for
// x < 0, with P a polynomial of log2 Q on [0, 5.5] (a Chebyshev fit;
// csrc/fit_normal_tail.py derives the coefficients and measures the error)
// and 2^y from v_exp_f32. The negative side has no cancellation. Past
// x < -5.5 the result is x * 0: the reference's 0.5 x (1 + erff(x / sqrt 2))
// (src/backend/reference/ops.cpp:151-155) is x * 0 below -5.5426, where fp32
// erff has rounded to -1, and between there and -5.5 it is fp32 noise (one
// ulp of 1 + erff, |result| < 2e-7) about as far from the exact GELU as 0.
//   fp32 activations: degree 10; Q relative error below 3e-6, Phi absolute
//     error below 1.4e-7, x Phi(x) within 1e-7 max(1, |x|).
//   bf16 activations: degree 6, four FMAs fewer per element (the kernel is
//     close to ALU-bound on packed-fp32-free code); Q relative error below
//     3e-5, Phi absolute error below 1.1e-5, far inside a bf16 ulp (2^-8
//     relative): every finite bf16 input above -4.6 gives the oracle's fp32
//     result rounded to bf16, or its neighbour, as degree 10 does. Below
//     -4.6 the reference's own 1 + erff(x / sqrt 2) cancels, and both
//     degrees sit nearer the exact GELU than the reference does.
template <int kDegree>
__device__ __forceinline__ float gelu_f(float x) {
  static_assert(kDegree == 10 || kDegree == 6, "fitted degrees");
  constexpr float kT = 5.5f;
  const float t = fminf(fabsf(x), kT);
  float p;
  if constexpr (kDegree == 10) {
    p = -1.725302567e-08f;
    p = fmaf(p, t, 5.477549507e-07f);
    p = fmaf(p, t, -7.458289474e-06f);
    p = fmaf(p, t, 5.484473149e-05f);
    p = fmaf(p, t, -2.005067072e-04f);
    p = fmaf(p, t, -1.761470485e-04f);
    p = fmaf(p, t, 7.180649787e-03f);
    p = fmaf(p, t, -5.261564627e-02f);
    p = fmaf(p, t, -4.591561556e-01f);
    p = fmaf(p, t, -1.151113272e+00f);
    p = fmaf(p, t, -9.999998212e-01f);
  } else {
    p = 2.630473136e-05f;
    p = fmaf(p, t, -6.637311308e-04f);
    p = fmaf(p, t, 7.507435977e-03f);
    p = fmaf(p, t, -5.203327164e-02f);
    p = fmaf(p, t, -4.602325559e-01f);
    p = fmaf(p, t, -1.150642157e+00f);
    p = fmaf(p, t, -1.000029564e+00f);
  }
  const float q = __builtin_amdgcn_exp2f(p);
  float phi = x >= 0.0f ? 1.0f - q : q;
  phi = x < -kT ? 0.0f : phi;
  return x * phi;
}

// The GELU of an element of storage type T.
template <class T>
__device__ __forceinline__ float gelu_of(float x) {
  return gelu_f<sizeof(T) == 2 ? 6 : 10>(x);
}

// quick_gelu: v sigmoid(1.702 v) (src/backend/reference/ops.cpp:157-161), the
// CLIP MLP's activation, on the same exp2 / reciprocal as silu.
__device__ __forceinline__ float quick_gelu_f(float v) {
  const float e = __builtin_amdgcn_exp2f(v * (-1.702f * 1.4426950408889634f));
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace uocr_rocm
