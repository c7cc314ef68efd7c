// tanh-GELU forward and backward for one element as dtrain/autograd.py:133-144
// writes them (constants rounded to the dtype as NumPy rounds them; every
// operation in dtrain's order; float32 takes tanh from the exponential).
// Shared by the elementwise GELU kernels and the GEMM epilogues that fuse
// them, so fused and unfused results are the same bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

namespace dtmi {

template <typename T>
struct GeluConst;
template <>
struct GeluConst<float> {
  static constexpr float c = 0.7978845608028654f;  // float(sqrt(2/pi))
  static constexpr float a = 0.044715f;
  static constexpr float a3 = 0.134145f;           // float(3 * 0.044715)
};
template <>
struct GeluConst<double> {
  static constexpr double c = 0.7978845608028654;
  static constexpr double a = 0.044715;
  static constexpr double a3 = 0.134145;  // == 3 * 0.044715 in double
};

template <typename T>
__device__ __forceinline__ T gelu_tanh_arg(T x) {
  T x3 = x * x * x;
  T inner = x + GeluConst<T>::a * x3;
  return GeluConst<T>::c * inner;
}

// tanh(u) = 1 - 2 / (1 + e^(2u)) with e^(2u) = 2^(2u log2(e)) on v_exp_f32
// and the reciprocal on v_rcp_f32: about 6 vector instructions instead of the
// library tanhf's ~30 (the GELU epilogue of a GEMM shares the SIMD with the
// float32 MFMAs). Saturates to +-1 for large |u|; the absolute error is below
// 2e-7 everywhere, which GELU (0.5 x (1 + t), and 1 - t^2 in its backward)
// needs -- not a small relative error of t near 0.
__device__ __forceinline__ float gelu_tanh(float u) {
  const float e = __builtin_amdgcn_exp2f(u * 2.8853900817779268f);  // 2 log2(e)
  return 1.f - 2.f * __builtin_amdgcn_rcpf(1.f + e);
}
__device__ __forceinline__ double gelu_tanh(double u) { return tanh(u); }

template <typename T>
__device__ __forceinline__ T gelu_f(T x) {
  T t = gelu_tanh(gelu_tanh_arg(x));
  T one_t = T(1) + t;
  T hx = T(0.5) * x;
  return hx * one_t;
}

template <typename T>
__device__ __forceinline__ T gelu_b(T x, T g) {
  T t = gelu_tanh(gelu_tanh_arg(x));
  T x2 = x * x;
  T du = GeluConst<T>::c * (T(1) + GeluConst<T>::a3 * x2);
  T left = T(0.5) * (T(1) + t);
  T right = T(0.5) * x;
  right = right * (T(1) - t * t);
  right = right * du;
  return g * (left + right);
}

}  // namespace dtmi
