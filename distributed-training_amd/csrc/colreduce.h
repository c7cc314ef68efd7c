// Deterministic second stage of the column reductions (LayerNorm dgamma/dbeta,
// bias gradients): out[c] (+)= sum_p parts[p * cols + c].
//
// A 256-thread block covers 32 columns with 8 groups of 32 lanes; group g adds
// the parts p = g, g + 8, g + 16, ... in increasing order (eight independent
// loads in flight per step), then the eight group sums are added in group
// order. The grouping depends only on nparts, so results are reproducible.
#pragma once

#include "common.h"

namespace dtmi {

// blockIdx.y selects one of two (out, parts) pairs, so two reductions of the
// same shape (LayerNorm's dgamma and dbeta) share one launch.
template <typename T>
__global__ void __launch_bounds__(256) colreduce_kernel(T* __restrict__ out, const T* __restrict__ parts, int nparts,
                                                         int64_t cols, int accumulate, T* __restrict__ out1,
                                                         const T* __restrict__ parts1) {
  if (blockIdx.y == 1) {
    out = out1;
    parts = parts1;
  }
  __shared__ T sh[8][32];
  const int cl = threadIdx.x & 31, grp = threadIdx.x >> 5;
  const int64_t c = (int64_t)blockIdx.x * 32 + cl;
  T acc = T(0);
  if (c < cols) {
    int p = grp;
    for (; p + 8 * 7 < nparts; p += 64) {
      T v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = parts[(int64_t)(p + 8 * u) * cols + c];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = acc + v[u];
    }
    for (; p < nparts; p += 8) acc = acc + parts[(int64_t)p * cols + c];
  }
  sh[grp][cl] = acc;
  __syncthreads();
  if (grp == 0 && c < cols) {
    T r = sh[0][cl];
#pragma unroll
    for (int g = 1; g < 8; ++g) r = r + sh[g][cl];
    out[c] = accumulate ? out[c] + r : r;
  }
}

template <typename T>
inline void launch_colreduce(T* out, const T* parts, int nparts, int64_t cols, int accumulate, T* out1 = nullptr,
                             const T* parts1 = nullptr) {
  dim3 grid((unsigned)cdiv(cols, 32), out1 ? 2u : 1u);
  colreduce_kernel<T><<<grid, 256, 0, stream()>>>(out, parts, nparts, cols, accumulate, out1, parts1);
}

}  // namespace dtmi
