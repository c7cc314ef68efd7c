// Embedding gather and its deterministic scatter-add backward
// (dtrain/autograd.py:199-204).
//
// Backward: dtrain zero-fills dW and runs np.add.at(gw, idx, g), which adds
// the rows of g into gw one index at a time in increasing position order. The
// host sorts the (host-resident) index array stably once per forward, giving
// for every distinct row v the positions that hit it in increasing order
// (perm[seg_start[s] .. seg_start[s+1]) for v = seg_row[s]). One block per
// distinct row then sums g[perm[j], :] in that order starting from 0 -- the
// same additions in the same order as np.add.at, so the result is bit-exact,
// and no atomics are involved. Rows nobody indexes keep the zero fill.
#include "common.h"

namespace dtmi {

template <typename T>
__global__ void __launch_bounds__(256) embed_fwd_kernel(T* __restrict__ out, const T* __restrict__ w,
                                                         const int64_t* __restrict__ idx, int64_t n, int64_t V,
                                                         int64_t C) {
  const int64_t i = blockIdx.x;
  if (i >= n) return;
  const int64_t v = idx[i];
  T* o = out + i * C;
  if (v < 0 || v >= V) {  // rejected on the host; never read out of bounds here
    for (int64_t c = threadIdx.x; c < C; c += blockDim.x) o[c] = T(NAN);
    return;
  }
  const T* src = w + v * C;
  for (int64_t c = threadIdx.x; c < C; c += blockDim.x) o[c] = src[c];
}

template <typename T>
__global__ void __launch_bounds__(256) embed_bwd_kernel(T* __restrict__ dw, const T* __restrict__ g,
                                                         const int32_t* __restrict__ perm,
                                                         const int32_t* __restrict__ seg_start,
                                                         const int32_t* __restrict__ seg_row, int64_t V, int64_t C) {
  const int s = blockIdx.x;
  const int32_t v = seg_row[s];
  if (v < 0 || v >= V) return;
  const int32_t j0 = seg_start[s], j1 = seg_start[s + 1];
  for (int64_t c = threadIdx.x; c < C; c += blockDim.x) {
    T acc = T(0);
    for (int32_t j = j0; j < j1; ++j) acc = acc + g[(int64_t)perm[j] * C + c];
    dw[(int64_t)v * C + c] = acc;
  }
}

}  // namespace dtmi

using namespace dtmi;

DTMI_EXPORT int dtmi_embedding_fwd(int dtype, void* out, const void* weight, const int64_t* idx, int64_t n_idx,
                                   int64_t vocab, int64_t cols) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n_idx >= 0 && vocab > 0 && cols > 0 && n_idx < (1LL << 31), "dtmi_embedding_fwd: bad shape");
  if (n_idx == 0) return DTMI_OK;
  DTMI_CHECK(out && weight && idx, "dtmi_embedding_fwd: NULL pointer");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  TimedLaunch tl(DTMI_FAM_OTHER, 2.0 * (double)n_idx * cols * es);
  if (dtype == DTMI_F32)
    embed_fwd_kernel<float><<<(unsigned)n_idx, 256, 0, stream()>>>((float*)out, (const float*)weight, idx, n_idx,
                                                                   vocab, cols);
  else
    embed_fwd_kernel<double><<<(unsigned)n_idx, 256, 0, stream()>>>((double*)out, (const double*)weight, idx, n_idx,
                                                                    vocab, cols);
  LAUNCH_CHECK("embed_fwd_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_embedding_bwd(int dtype, void* dweight, const void* dout, const int32_t* perm,
                                   const int32_t* seg_start, const int32_t* seg_row, int nseg, int64_t vocab,
                                   int64_t cols, int zero_fill) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(nseg >= 0 && vocab > 0 && cols > 0, "dtmi_embedding_bwd: bad shape");
  DTMI_CHECK(dweight != nullptr, "dtmi_embedding_bwd: NULL dweight");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  if (zero_fill) {
    int rc = dtmi_zero_bytes(dweight, (size_t)vocab * cols * es);
    if (rc) return rc;
  }
  if (nseg == 0) return DTMI_OK;
  DTMI_CHECK(dout && perm && seg_start && seg_row, "dtmi_embedding_bwd: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, 2.0 * (double)nseg * cols * es);
  if (dtype == DTMI_F32)
    embed_bwd_kernel<float><<<(unsigned)nseg, 256, 0, stream()>>>((float*)dweight, (const float*)dout, perm,
                                                                  seg_start, seg_row, vocab, cols);
  else
    embed_bwd_kernel<double><<<(unsigned)nseg, 256, 0, stream()>>>((double*)dweight, (const double*)dout, perm,
                                                                   seg_start, seg_row, vocab, cols);
  LAUNCH_CHECK("embed_bwd_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}
