// Embedding gather and its deterministic scatter-add backward
// (dtrain/autograd.py:199-204).
//
// Backward: dtrain zero-fills dW and runs np.add.at(gw, idx, g), which adds
// the rows of g into gw one index at a time in increasing position order. The
// index array is sorted stably once per forward, giving for every distinct
// row v the positions that hit it in increasing order (perm[seg_start[s] ..
// seg_start[s+1]) for v = seg_row[s]). One block per distinct row then sums
// g[perm[j], :] in that order starting from 0 -- the same additions in the
// same order as np.add.at, so the result is bit-exact, and no atomics are
// involved. Rows nobody indexes keep the zero fill.
//
// The sort runs on the device (dtmi_embedding_segments) from the index array
// already in HBM: the 64-bit keys (row << 32) | position are unique, so any
// correct sort of them is the stable sort by row. Chunks of kSegChunk keys
// are sorted in LDS by one block each (bitonic network), sorted runs are
// merged pairwise by rank (an element's place in the merged run is its place
// in its own run plus the count of smaller keys in the other, by binary
// search), and a scan over the row changes lays out the segments.
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

// Segment sums with the segment count read on the device: launched with one
// block per index position (the most segments there can be); blocks past the
// count leave at once.
template <typename T>
__global__ void __launch_bounds__(256) embed_bwd_dev_kernel(T* __restrict__ dw, const T* __restrict__ g,
                                                             const int32_t* __restrict__ perm,
                                                             const int32_t* __restrict__ seg_start,
                                                             const int32_t* __restrict__ seg_row,
                                                             const int32_t* __restrict__ nseg, int64_t V, int64_t C) {
  const int s = blockIdx.x;
  if (s >= *nseg) return;
  const int32_t v = seg_row[s];
  if (v < 0 || v >= V) return;
  const int32_t j0 = seg_start[s], j1 = seg_start[s + 1];
  for (int64_t c = threadIdx.x; c < C; c += blockDim.x) {
    T acc = T(0);
    for (int32_t j = j0; j < j1; ++j) acc = acc + g[(int64_t)perm[j] * C + c];
    dw[(int64_t)v * C + c] = acc;
  }
}

// ------------------------------------------------------ segments on device
constexpr int kSegChunk = 8192;  // keys per block sort: 64 KB of LDS
constexpr int kSegThreads = 1024;
constexpr int kSegScan = 1024;  // keys per block of the segment scan

__device__ __forceinline__ uint64_t seg_key(const int64_t* __restrict__ idx, int64_t i) {
  return ((uint64_t)(uint32_t)idx[i] << 32) | (uint64_t)(uint32_t)i;
}

// Block b sorts keys [b * kSegChunk, ...) ascending in LDS (padding keys of
// all ones sort last and are not written back).
__global__ void __launch_bounds__(kSegThreads) seg_chunk_sort_kernel(const int64_t* __restrict__ idx, int64_t n,
                                                                      uint64_t* __restrict__ keys) {
  __shared__ uint64_t k[kSegChunk];
  const int64_t base = (int64_t)blockIdx.x * kSegChunk;
  const int cnt = (int)(n - base < kSegChunk ? n - base : kSegChunk);
  int len = 1;  // the network's size: the chunk rounded up to a power of two
  while (len < cnt) len <<= 1;
  for (int i = threadIdx.x; i < len; i += kSegThreads) k[i] = i < cnt ? seg_key(idx, base + i) : ~0ull;
  __syncthreads();
  for (int size = 2; size <= len; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < len / 2; t += kSegThreads) {
        // compare-exchange pair (lo, lo + stride) of the t-th pair
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t a = k[lo], b = k[hi];
        if ((a > b) == up) {
          k[lo] = b;
          k[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < cnt; i += kSegThreads) keys[base + i] = k[i];
}

// Merge sorted runs of length R pairwise: [2mR, 2mR + R) with
// [2mR + R, 2mR + 2R) (the second run may be short or absent).
__global__ void __launch_bounds__(256) seg_merge_kernel(const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                                                         int64_t n, int64_t R) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t base = (i / (2 * R)) * 2 * R;
  const bool first = i < base + R;
  const int64_t o0 = first ? base + R : base;  // the other run
  const int64_t o1 = first ? (base + 2 * R < n ? base + 2 * R : n) : base + R;
  const uint64_t key = in[i];
  int64_t lo = o0, hi = o1;  // count of keys in the other run below key
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (in[mid] < key)
      lo = mid + 1;
    else
      hi = mid;
  }
  out[base + (i - (first ? base : base + R)) + (lo - o0)] = key;
}

// A segment starts at sorted position j when j == 0 or its row differs from
// position j - 1's.
__device__ __forceinline__ int seg_flag(const uint64_t* __restrict__ keys, int64_t j) {
  return j == 0 || (keys[j] >> 32) != (keys[j - 1] >> 32);
}

// Segment starts per scan block.
__global__ void __launch_bounds__(256) seg_count_kernel(const uint64_t* __restrict__ keys, int64_t n,
                                                         int32_t* __restrict__ counts) {
  __shared__ int part[4];
  const int64_t b0 = (int64_t)blockIdx.x * kSegScan;
  int c = 0;
  for (int t = threadIdx.x; t < kSegScan; t += 256) {
    const int64_t j = b0 + t;
    if (j < n) c += seg_flag(keys, j);
  }
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

// Exclusive scan of the per-block counts in place (one block, in order),
// the total into *nseg and seg_start[total] = n.
__global__ void __launch_bounds__(256) seg_offsets_kernel(int32_t* __restrict__ counts, int64_t nb, int64_t n,
                                                           int32_t* __restrict__ nseg, int32_t* __restrict__ seg_start) {
  __shared__ int32_t run;
  __shared__ int32_t wsum[4];
  if (threadIdx.x == 0) run = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int64_t c0 = 0; c0 < nb; c0 += 256) {
    const int64_t i = c0 + threadIdx.x;
    const int32_t v = i < nb ? counts[i] : 0;
    int32_t x = v;  // inclusive scan within the wave
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int32_t before = run;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    if (i < nb) counts[i] = before + x - v;
    __syncthreads();
    if (threadIdx.x == 0) run += wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    *nseg = run;
    seg_start[run] = (int32_t)n;
  }
}

// perm[j] = position of sorted key j; for each segment start, its place and row.
__global__ void __launch_bounds__(256) seg_write_kernel(const uint64_t* __restrict__ keys, int64_t n,
                                                         const int32_t* __restrict__ offs, int32_t* __restrict__ perm,
                                                         int32_t* __restrict__ seg_start,
                                                         int32_t* __restrict__ seg_row) {
  __shared__ int32_t wsum[4];
  __shared__ int32_t run;
  const int64_t b0 = (int64_t)blockIdx.x * kSegScan;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) run = offs[blockIdx.x];
  __syncthreads();
  for (int t0 = 0; t0 < kSegScan; t0 += 256) {
    const int64_t j = b0 + t0 + threadIdx.x;
    const int f = j < n ? seg_flag(keys, j) : 0;
    int32_t x = f;
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int32_t before = run;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    if (j < n) {
      const uint64_t key = keys[j];
      perm[j] = (int32_t)(uint32_t)key;
      if (f) {
        const int32_t s = before + x - 1;
        seg_start[s] = (int32_t)j;
        seg_row[s] = (int32_t)(key >> 32);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) run += wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
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

DTMI_EXPORT int dtmi_embedding_segments(const int64_t* idx, int64_t n_idx, int32_t* perm, int32_t* seg_start,
                                        int32_t* seg_row, int32_t* nseg) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(n_idx >= 0 && n_idx < (1LL << 31), "dtmi_embedding_segments: bad index count %lld", (long long)n_idx);
  DTMI_CHECK(seg_start && nseg, "dtmi_embedding_segments: NULL pointer");
  if (n_idx == 0) {
    int rc = dtmi_zero_bytes(nseg, sizeof(int32_t));
    if (rc) return rc;
    return dtmi_zero_bytes(seg_start, sizeof(int32_t));  // seg_start[0] = n = 0
  }
  DTMI_CHECK(idx && perm && seg_row, "dtmi_embedding_segments: NULL pointer");
  const int64_t nch = cdiv(n_idx, (int64_t)kSegChunk);
  const int64_t nb = cdiv(n_idx, (int64_t)kSegScan);
  void* work = nullptr;
  const size_t kb = (size_t)n_idx * sizeof(uint64_t);
  int rc = pool_alloc(&work, 2 * kb + (size_t)nb * sizeof(int32_t));
  if (rc) return rc;
  uint64_t* k0 = (uint64_t*)work;
  uint64_t* k1 = (uint64_t*)((char*)work + kb);
  int32_t* counts = (int32_t*)((char*)work + 2 * kb);
  {
    TimedLaunch tl(DTMI_FAM_OTHER, (double)n_idx * (8.0 + 8.0 * 2 + 12.0));
    seg_chunk_sort_kernel<<<(unsigned)nch, kSegThreads, 0, stream()>>>(idx, n_idx, k0);
    for (int64_t R = kSegChunk; R < n_idx; R *= 2) {
      seg_merge_kernel<<<(unsigned)cdiv(n_idx, 256LL), 256, 0, stream()>>>(k0, k1, n_idx, R);
      std::swap(k0, k1);
    }
    seg_count_kernel<<<(unsigned)nb, 256, 0, stream()>>>(k0, n_idx, counts);
    seg_offsets_kernel<<<1, 256, 0, stream()>>>(counts, nb, n_idx, nseg, seg_start);
    seg_write_kernel<<<(unsigned)nb, 256, 0, stream()>>>(k0, n_idx, counts, perm, seg_start, seg_row);
  }
  hipError_t le = hipGetLastError();
  pool_free(work);
  if (le != hipSuccess) return fail_hip(le, "embedding segment kernels", __FILE__, __LINE__);
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_embedding_bwd_segs(int dtype, void* dweight, const void* dout, const int32_t* perm,
                                        const int32_t* seg_start, const int32_t* seg_row, const int32_t* nseg,
                                        int64_t n_idx, int64_t vocab, int64_t cols, int zero_fill) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n_idx >= 0 && n_idx < (1LL << 31) && vocab > 0 && cols > 0, "dtmi_embedding_bwd_segs: bad shape");
  DTMI_CHECK(dweight != nullptr, "dtmi_embedding_bwd_segs: NULL dweight");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  if (zero_fill) {
    int rc = dtmi_zero_bytes(dweight, (size_t)vocab * cols * es);
    if (rc) return rc;
  }
  if (n_idx == 0) return DTMI_OK;
  DTMI_CHECK(dout && perm && seg_start && seg_row && nseg, "dtmi_embedding_bwd_segs: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, 2.0 * (double)n_idx * cols * es);
  if (dtype == DTMI_F32)
    embed_bwd_dev_kernel<float><<<(unsigned)n_idx, 256, 0, stream()>>>((float*)dweight, (const float*)dout, perm,
                                                                       seg_start, seg_row, nseg, vocab, cols);
  else
    embed_bwd_dev_kernel<double><<<(unsigned)n_idx, 256, 0, stream()>>>((double*)dweight, (const double*)dout,
                                                                        perm, seg_start, seg_row, nseg, vocab, cols);
  LAUNCH_CHECK("embed_bwd_dev_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}
