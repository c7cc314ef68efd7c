// Deterministic second stage of the column reductions (LayerNorm dgamma/dbeta,
// bias gradients): out[c] (+)= sum_p parts[p * cols + c].
//
// A 1024-thread block covers 16 columns with 64 groups of 16 lanes; group g
// adds the parts p = g, g + 64, g + 128, ... in increasing order (eight
// independent loads in flight per step: one step for 512 parts), then the 64
// group sums of a column are combined by a fixed butterfly across a wave. The
// grouping depends only on nparts, so results are reproducible.
#pragma once

#include "common.h"

namespace dtmi {

// blockIdx.y selects one of two (out, parts) pairs, so two reductions of the
// same shape (LayerNorm's dgamma and dbeta) share one launch.
template <typename T>
__global__ void __launch_bounds__(1024) colreduce_kernel(T* __restrict__ out, const T* __restrict__ parts, int nparts,
                                                          int64_t cols, int accumulate, T* __restrict__ out1,
                                                          const T* __restrict__ parts1) {
  if (blockIdx.y == 1) {
    out = out1;
    parts = parts1;
  }
  __shared__ T sh[64][17];
  const int cl = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int64_t c0 = (int64_t)blockIdx.x * 16;
  const int64_t c = c0 + cl;
  T acc = T(0);
  if (c < cols) {
    int p = grp;
    for (; p + 64 * 7 < nparts; p += 512) {
      T v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = parts[(int64_t)(p + 64 * u) * cols + c];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = acc + v[u];
    }
    for (; p < nparts; p += 64) acc = acc + parts[(int64_t)p * cols + c];
  }
  sh[grp][cl] = acc;
  __syncthreads();
  // wave w now takes column w and lane g its group g; the 64 group sums are
  // combined by a fixed butterfly
  const int col = threadIdx.x >> 6, g = threadIdx.x & 63;
  T r = sh[g][col];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) r = r + __shfl_xor(r, off, 64);
  const int64_t cc = c0 + col;
  if (g == 0 && cc < cols) out[cc] = accumulate ? out[cc] + r : r;
}

template <typename T>
inline void launch_colreduce(T* out, const T* parts, int nparts, int64_t cols, int accumulate, T* out1 = nullptr,
                             const T* parts1 = nullptr) {
  dim3 grid((unsigned)cdiv(cols, 16), out1 ? 2u : 1u);
  colreduce_kernel<T><<<grid, 1024, 0, stream()>>>(out, parts, nparts, cols, accumulate, out1, parts1);
}

}  // namespace dtmi
