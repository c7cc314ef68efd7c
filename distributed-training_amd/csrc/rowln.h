// Row-in-registers LayerNorm forward (dtrain/autograd.py:207-214), shared by
// the LayerNorm kernel and the GEMM split-K reduction that ends in one: one
// 64-lane wave owns a row of `cols` elements, lane `lane` holding elements
// VW*lane + 64*VW*j + e (j < NV, e < VW). Both callers run this same code, so
// the mean, rstd and outputs are the same bits whichever kernel computed them.
#pragma once

#include "common.h"

namespace dtmi {

template <typename T>
__device__ __forceinline__ T wave_sum(T x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <typename T, int VW>
__device__ __forceinline__ void load_vec(T (&dst)[VW], const T* __restrict__ src) {
  if constexpr (VW * sizeof(T) == 16) {
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  } else {
#pragma unroll
    for (int e = 0; e < VW; ++e) dst[e] = src[e];
  }
}

template <typename T, int VW>
__device__ __forceinline__ void store_vec(T* __restrict__ dst, const T (&src)[VW]) {
  if constexpr (VW * sizeof(T) == 16) {
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  } else {
#pragma unroll
    for (int e = 0; e < VW; ++e) dst[e] = src[e];
  }
}

// xv: the row (entries past `cols` are 0). Writes y = (x - mean) * rstd * w + b
// for the row at yr, and mean / rstd of the row by lane 0:
// mean = sum(x) / n; var = sum((x - mean)^2) / n; rstd = 1 / sqrt(var + eps).
template <typename T, int NV, int VW>
__device__ __forceinline__ void ln_row_fwd(const T (&xv)[NV][VW], int cols, int lane, const T* __restrict__ w,
                                           const T* __restrict__ b, T eps, T* __restrict__ yr, T* mean_out,
                                           T* rstd_out) {
  T s = T(0);
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < VW; ++e) s += xv[j][e];
  const T n = (T)cols;
  const T mu = wave_sum(s) / n;
  T q = T(0);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = VW * lane + 64 * VW * j;
    if (c < cols) {
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        T xc = xv[j][e] - mu;
        q += xc * xc;
      }
    }
  }
  const T var = wave_sum(q) / n;
  const T rstd = T(1) / sqrt(var + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = VW * lane + 64 * VW * j;
    if (c < cols) {
      T wv[VW], bv[VW], o[VW];
      load_vec<T, VW>(wv, w + c);
      load_vec<T, VW>(bv, b + c);
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        T xh = (xv[j][e] - mu) * rstd;
        o[e] = xh * wv[e] + bv[e];
      }
      store_vec<T, VW>(yr + c, o);
    }
  }
  if (lane == 0) {
    *mean_out = mu;
    *rstd_out = rstd;
  }
}

// Vectors per lane for rows of `per_lane` vectors (the compiled set).
inline int ln_pick_nv(int64_t per_lane) {
  static const int opts[] = {1, 2, 3, 4, 6, 8, 12, 16};
  for (int o : opts)
    if (per_lane <= o) return o;
  return -1;
}

#define LN_NV_SWITCH(nv, CALL) \
  switch (nv) {                \
    case 1: CALL(1); break;    \
    case 2: CALL(2); break;    \
    case 3: CALL(3); break;    \
    case 4: CALL(4); break;    \
    case 6: CALL(6); break;    \
    case 8: CALL(8); break;    \
    case 12: CALL(12); break;  \
    default: CALL(16); break;  \
  }

}  // namespace dtmi
