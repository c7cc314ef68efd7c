// tanh-GELU forward and backward for one element, exactly as
// dtrain/autograd.py:133-144 writes them (constants rounded to the dtype as
// NumPy rounds them; every operation in dtrain's order). Shared by the
// elementwise GELU kernels and the GEMM epilogues that fuse them.
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

template <typename T>
__device__ __forceinline__ T gelu_f(T x) {
  T t = tanh(gelu_tanh_arg(x));
  T one_t = T(1) + t;
  T hx = T(0.5) * x;
  return hx * one_t;
}

template <typename T>
__device__ __forceinline__ T gelu_b(T x, T g) {
  T t = tanh(gelu_tanh_arg(x));
  T x2 = x * x;
  T du = GeluConst<T>::c * (T(1) + GeluConst<T>::a3 * x2);
  T left = T(0.5) * (T(1) + t);
  T right = T(0.5) * x;
  right = right * (T(1) - t * t);
  right = right * du;
  return g * (left + right);
}

}  // namespace dtmi
