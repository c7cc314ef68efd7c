// Cross-entropy forward and backward over vocabulary rows, and the standalone
// row-wise softmax backward (dtrain/autograd.py:250-266 and :242).
//
// Cross entropy: one 256-thread block per row. The forward makes a single pass
// over the row with an online (max, sum of exp) pair per thread, 16-byte
// vector loads, then combines the 256 pairs in a fixed tree; it saves the row
// max and the row sum for the backward and the row's log p[target]. The loss
// is -(sum of log p[target]) / n, summed in a fixed order by one block. The
// backward re-reads the row once and writes (exp(z - max) / sum - [j == t]) *
// (g / n) with g read from device memory (the upstream gradient of the loss
// node), so no host synchronisation is needed between forward and backward.
//
// A row of 50304 float32 logits is 196 KiB, more than the 160 KiB of LDS of a
// CU, hence the online single pass instead of an LDS-resident row.
#include <cmath>

#include "common.h"

namespace dtmi {

template <typename T>
__device__ __forceinline__ void online_add(T& m, T& s, T z) {
  if (z > m) {
    s = s * exp(m - z) + T(1);
    m = z;
  } else {
    s += exp(z - m);
  }
}

template <typename T>
__device__ __forceinline__ void online_merge(T& m, T& s, T m2, T s2) {
  if (m2 > m) {
    s = s * exp(m - m2) + s2;
    m = m2;
  } else if (m2 == m) {
    s += s2;
  } else {
    s += s2 * exp(m2 - m);
  }
}

template <typename T>
__global__ void __launch_bounds__(256) xent_fwd_kernel(T* __restrict__ rowmax, T* __restrict__ rowsum,
                                                        T* __restrict__ logp_t, const T* __restrict__ z,
                                                        const int64_t* __restrict__ targets, int64_t V, int vec) {
  __shared__ T sm[256], ss[256];
  const int64_t row = blockIdx.x;
  const T* zr = z + row * V;
  const T ninf = -INFINITY;
  T m = ninf, s = T(0);
  if (vec) {
    constexpr int N = 16 / sizeof(T);
    const int64_t nv = V / N;
    for (int64_t i = threadIdx.x; i < nv; i += 256) {
      T v[N];
      *reinterpret_cast<uint4*>(v) = reinterpret_cast<const uint4*>(zr)[i];
      T lm = v[0];
#pragma unroll
      for (int e = 1; e < N; ++e) lm = v[e] > lm ? v[e] : lm;
      if (lm > m) {
        s = (m == ninf) ? T(0) : s * exp(m - lm);
        m = lm;
      }
#pragma unroll
      for (int e = 0; e < N; ++e) s += exp(v[e] - m);
    }
    for (int64_t k = nv * N + threadIdx.x; k < V; k += 256) online_add(m, s, zr[k]);
  } else {
    for (int64_t k = threadIdx.x; k < V; k += 256) online_add(m, s, zr[k]);
  }
  sm[threadIdx.x] = m;
  ss[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (threadIdx.x < w) {
      T m1 = sm[threadIdx.x], s1 = ss[threadIdx.x];
      T m2 = sm[threadIdx.x + w], s2 = ss[threadIdx.x + w];
      if (m2 != ninf) online_merge(m1, s1, m2, s2);
      sm[threadIdx.x] = m1;
      ss[threadIdx.x] = s1;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const T M = sm[0], S = ss[0];
    rowmax[row] = M;
    rowsum[row] = S;
    const int64_t t = targets[row];
    // (z - zmax) - log(s), dtrain/autograd.py:255
    logp_t[row] = (t >= 0 && t < V) ? (zr[t] - M) - log(S) : T(NAN);
  }
}

// loss = -(sum_r logp_t[r]) / n ; one block, fixed order.
template <typename T>
__global__ void __launch_bounds__(256) xent_loss_kernel(T* __restrict__ loss, const T* __restrict__ logp_t,
                                                         int64_t rows) {
  __shared__ T sh[256];
  T a = T(0);
  for (int64_t r = threadIdx.x; r < rows; r += 256) a += logp_t[r];
  sh[threadIdx.x] = a;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) *loss = -(sh[0] / (T)rows);
}

// dlogits = (exp(z - max) / sum - onehot) * (g / n)    (dtrain/autograd.py:262-265)
template <typename T>
__global__ void __launch_bounds__(256) xent_bwd_kernel(T* __restrict__ dz, const T* __restrict__ z,
                                                        const T* __restrict__ rowmax, const T* __restrict__ rowsum,
                                                        const int64_t* __restrict__ targets,
                                                        const T* __restrict__ g_dev, T g_host, int64_t n, int64_t V,
                                                        int vec) {
  const int64_t row = blockIdx.x;
  const T M = rowmax[row], S = rowsum[row];
  const T g = g_dev ? *g_dev : g_host;
  const T gn = g / (T)n;
  const int64_t t = targets[row];
  const T* zr = z + row * V;
  T* dr = dz + row * V;
  if (vec) {
    constexpr int N = 16 / sizeof(T);
    const int64_t nv = V / N;
    for (int64_t i = threadIdx.x; i < nv; i += 256) {
      T v[N];
      *reinterpret_cast<uint4*>(v) = reinterpret_cast<const uint4*>(zr)[i];
#pragma unroll
      for (int e = 0; e < N; ++e) {
        T p = exp(v[e] - M) / S;
        if (i * N + e == t) p = p - T(1);
        v[e] = p * gn;
      }
      reinterpret_cast<uint4*>(dr)[i] = *reinterpret_cast<uint4*>(v);
    }
    for (int64_t k = nv * N + threadIdx.x; k < V; k += 256) {
      T p = exp(zr[k] - M) / S;
      if (k == t) p = p - T(1);
      dr[k] = p * gn;
    }
  } else {
    for (int64_t k = threadIdx.x; k < V; k += 256) {
      T p = exp(zr[k] - M) / S;
      if (k == t) p = p - T(1);
      dr[k] = p * gn;
    }
  }
}

// Forward and gradient in one pass (float32, rows of up to 65536 logits):
// one 1024-thread block per row holds the row in registers (NV 16-byte
// vectors per thread), so the logits are read once and dlogits written once
// (the two-kernel form reads them twice). dlogits = (exp(z - max) * (1 / sum)
// - onehot) * (1 / n): the gradient for an upstream gradient of 1, which
// xent_grad_scale_kernel rescales in place when the upstream gradient is not
// 1. Max and sum are combined in a fixed order: a butterfly per wave, then
// the 16 wave results in wave order.
template <int NV>
__global__ void __launch_bounds__(1024) xent_fused_kernel(float* __restrict__ dz, float* __restrict__ rowmax,
                                                           float* __restrict__ rowsum, float* __restrict__ logp_t,
                                                           const float* __restrict__ z,
                                                           const int64_t* __restrict__ targets, int64_t V,
                                                           float inv_n) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const f4* zr = reinterpret_cast<const f4*>(z + row * V);
  f4* dr = reinterpret_cast<f4*>(dz + row * V);
  const int nv = (int)(V / 4);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  f4 v[NV];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = tid + 1024 * j;
    v[j] = i < nv ? zr[i] : f4(-INFINITY);
#pragma unroll
    for (int e = 0; e < 4; ++e) m = fmaxf(m, v[j][e]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) M = fmaxf(M, red[w]);
  __syncthreads();
  // v becomes exp(z - max) (0 past the row end), reused by the gradient
  float sl = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[j][e] = (tid + 1024 * j < nv) ? expf(v[j][e] - M) : 0.f;
      sl += v[j][e];
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sl += __shfl_xor(sl, off, 64);
  if (lane == 0) red[wave] = sl;
  __syncthreads();
  float S = red[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) S += red[w];
  const int64_t t = targets[row];
  if (tid == 0) {
    rowmax[row] = M;
    rowsum[row] = S;
    // (z - zmax) - log(s), dtrain/autograd.py:255
    logp_t[row] = (t >= 0 && t < V) ? (z[row * V + t] - M) - logf(S) : NAN;
  }
  // p = e * (1 / s): within 1.5 ulp of e / s, and one multiply per logit
  // instead of a division (the block's vector work does not overlap its
  // loads, one row block fills a CU). V < 2^31 here, so 32-bit indices.
  const float rS = 1.f / S;
  const int t32 = (t >= 0 && t < V) ? (int)t : -1;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = tid + 1024 * j;
    if (i < nv) {
      f4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float p = v[j][e] * rS;
        if (4 * i + e == t32) p = p - 1.f;
        o[e] = p * inv_n;
      }
      dr[i] = o;
    }
  }
}

// x *= g[0] unless g[0] == 1 (then x is already the gradient).
template <typename T>
__global__ void __launch_bounds__(256) xent_grad_scale_kernel(T* __restrict__ x, const T* __restrict__ g, int64_t n) {
  const T gv = *g;
  if (gv == T(1)) return;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) x[i] = x[i] * gv;
}

// dS = P * (dP - rowsum(dP * P)); one wave per row.
template <typename T>
__global__ void __launch_bounds__(256) softmax_bwd_kernel(T* __restrict__ ds, const T* __restrict__ p,
                                                           const T* __restrict__ dp, int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* pr = p + row * cols;
  const T* dr = dp + row * cols;
  T a = T(0);
  for (int64_t c = lane; c < cols; c += 64) a += dr[c] * pr[c];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) a += __shfl_xor(a, off, 64);
  T* o = ds + row * cols;
  for (int64_t c = lane; c < cols; c += 64) o[c] = pr[c] * (dr[c] - a);
}

template <typename T>
static int xent_fwd(void* loss, void* rowmax, void* rowsum, const void* logits, const int64_t* targets, int64_t rows,
                    int64_t V) {
  bool vec = V % (16 / sizeof(T)) == 0 && aligned(logits, 16);
  void* lp = nullptr;
  int rc = pool_alloc(&lp, (size_t)rows * sizeof(T));
  if (rc) return rc;
  {
    TimedLaunch tl(DTMI_FAM_XENT, (double)rows * V * sizeof(T));
    xent_fwd_kernel<T><<<(unsigned)rows, 256, 0, stream()>>>((T*)rowmax, (T*)rowsum, (T*)lp, (const T*)logits,
                                                             targets, V, vec ? 1 : 0);
    xent_loss_kernel<T><<<1, 256, 0, stream()>>>((T*)loss, (const T*)lp, rows);
  }
  hipError_t le = hipGetLastError();
  pool_free(lp);
  if (le != hipSuccess) return fail_hip(le, "xent forward kernels", __FILE__, __LINE__);
  return DTMI_OK;
}

}  // namespace dtmi

using namespace dtmi;

DTMI_EXPORT int dtmi_xent_fwd(int dtype, void* loss, void* rowmax, void* rowsum, const void* logits,
                              const int64_t* targets, int64_t rows, int64_t vocab) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows > 0 && vocab > 0 && rows < (1LL << 31), "dtmi_xent_fwd: bad shape [%lld, %lld]", (long long)rows,
             (long long)vocab);
  DTMI_CHECK(loss && rowmax && rowsum && logits && targets, "dtmi_xent_fwd: NULL pointer");
  if (dtype == DTMI_F32) return xent_fwd<float>(loss, rowmax, rowsum, logits, targets, rows, vocab);
  return xent_fwd<double>(loss, rowmax, rowsum, logits, targets, rows, vocab);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_xent_bwd(int dtype, void* dlogits, const void* logits, const void* rowmax, const void* rowsum,
                              const int64_t* targets, const void* g_dev, double g_host, int64_t rows, int64_t vocab) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows > 0 && vocab > 0 && rows < (1LL << 31), "dtmi_xent_bwd: bad shape [%lld, %lld]", (long long)rows,
             (long long)vocab);
  DTMI_CHECK(dlogits && logits && rowmax && rowsum && targets, "dtmi_xent_bwd: NULL pointer");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  bool vec = vocab % (int64_t)(16 / es) == 0 && aligned(logits, 16) && aligned(dlogits, 16);
  TimedLaunch tl(DTMI_FAM_XENT, 2.0 * (double)rows * vocab * es);
  if (dtype == DTMI_F32)
    xent_bwd_kernel<float><<<(unsigned)rows, 256, 0, stream()>>>(
        (float*)dlogits, (const float*)logits, (const float*)rowmax, (const float*)rowsum, targets,
        (const float*)g_dev, (float)g_host, rows, vocab, vec ? 1 : 0);
  else
    xent_bwd_kernel<double><<<(unsigned)rows, 256, 0, stream()>>>(
        (double*)dlogits, (const double*)logits, (const double*)rowmax, (const double*)rowsum, targets,
        (const double*)g_dev, g_host, rows, vocab, vec ? 1 : 0);
  LAUNCH_CHECK("xent_bwd_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_xent_fused(int dtype, void* loss, void* dlogits, void* rowmax, void* rowsum, const void* logits,
                                const int64_t* targets, int64_t rows, int64_t vocab) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows > 0 && vocab > 0 && rows < (1LL << 31), "dtmi_xent_fused: bad shape [%lld, %lld]",
             (long long)rows, (long long)vocab);
  DTMI_CHECK(loss && dlogits && rowmax && rowsum && logits && targets, "dtmi_xent_fused: NULL pointer");
  const int64_t nv = vocab / 4;
  const bool fused = dtype == DTMI_F32 && vocab % 4 == 0 && nv <= 16 * 1024 && aligned(logits, 16) &&
                     aligned(dlogits, 16);
  if (!fused) {  // the two-kernel form: forward, then the gradient for an upstream gradient of 1
    int rc = dtmi_xent_fwd(dtype, loss, rowmax, rowsum, logits, targets, rows, vocab);
    if (rc) return rc;
    return dtmi_xent_bwd(dtype, dlogits, logits, rowmax, rowsum, targets, nullptr, 1.0, rows, vocab);
  }
  float* logp = nullptr;
  int rc = pool_alloc((void**)&logp, (size_t)rows * sizeof(float));
  if (rc) return rc;
  {
    TimedLaunch tl(DTMI_FAM_XENT, 2.0 * (double)rows * vocab * 4);
    const float inv_n = 1.f / (float)rows;
    auto go = [&](auto nvc) {
      constexpr int NV = decltype(nvc)::value;
      xent_fused_kernel<NV><<<(unsigned)rows, 1024, 0, stream()>>>((float*)dlogits, (float*)rowmax, (float*)rowsum,
                                                                   logp, (const float*)logits, targets, vocab, inv_n);
    };
    const int need = (int)cdiv(nv, 1024);
    if (need <= 1)
      go(std::integral_constant<int, 1>());
    else if (need <= 2)
      go(std::integral_constant<int, 2>());
    else if (need <= 4)
      go(std::integral_constant<int, 4>());
    else if (need <= 8)
      go(std::integral_constant<int, 8>());
    else if (need <= 13)
      go(std::integral_constant<int, 13>());
    else
      go(std::integral_constant<int, 16>());
    xent_loss_kernel<float><<<1, 256, 0, stream()>>>((float*)loss, logp, rows);
  }
  hipError_t le = hipGetLastError();
  pool_free(logp);
  if (le != hipSuccess) return fail_hip(le, "xent_fused kernels", __FILE__, __LINE__);
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_xent_grad_scale(int dtype, void* dlogits, const void* g_dev, int64_t n) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(dlogits && g_dev && n >= 0, "dtmi_xent_grad_scale: bad arguments");
  if (n == 0) return DTMI_OK;
  const int grid = (int)(cdiv(n, 256 * 8) < 4096 ? cdiv(n, 256 * 8) : 4096);
  if (dtype == DTMI_F32)
    xent_grad_scale_kernel<float><<<grid, 256, 0, stream()>>>((float*)dlogits, (const float*)g_dev, n);
  else
    xent_grad_scale_kernel<double><<<grid, 256, 0, stream()>>>((double*)dlogits, (const double*)g_dev, n);
  LAUNCH_CHECK("xent_grad_scale_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_softmax_bwd(int dtype, void* ds, const void* p, const void* dp, int64_t rows, int64_t cols) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(rows >= 0 && cols >= 0, "dtmi_softmax_bwd: negative shape");
  if (rows == 0 || cols == 0) return DTMI_OK;
  DTMI_CHECK(ds && p && dp, "dtmi_softmax_bwd: NULL pointer");
  const size_t es = dtype == DTMI_F32 ? 4 : 8;
  TimedLaunch tl(DTMI_FAM_OTHER, 3.0 * (double)rows * cols * es);
  unsigned grid = (unsigned)cdiv(rows, 4);
  if (dtype == DTMI_F32)
    softmax_bwd_kernel<float><<<grid, 256, 0, stream()>>>((float*)ds, (const float*)p, (const float*)dp, rows, cols);
  else
    softmax_bwd_kernel<double><<<grid, 256, 0, stream()>>>((double*)ds, (const double*)p, (const double*)dp, rows,
                                                           cols);
  LAUNCH_CHECK("softmax_bwd_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}
